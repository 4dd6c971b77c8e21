// Per-nonce noise kernels of the cuPOW miner on gfx950 (the commitment is uwc_commit.hip):
//   uniform noise E and the noise pairs P (kernels.cu:246-301, reference.py:67-93);
//   operand noising + rank-r projections in balanced base-128 limbs + max |projection|
//   (kernels.cu:303-404): a general-shape per-row form and the matrix-core forms.
#include "uwc_common.h"

// ------------------------------------------------------------------ noise generation
// random_hash(index, label, key, prepend): keyed digest of msg with msg[prepend] = 1 + index,
// msg[8..15] = label (reference.py:67-71).
__device__ __forceinline__ void random_hash(u32 index, const u32* label, const u32* key, int prepend, u32 out[8]) {
  u32 msg[16], k8[8];
#pragma unroll
  for (int i = 0; i < 8; i++) { msg[i] = 0; msg[8 + i] = label[i]; k8[i] = key[i]; }
  msg[prepend] = 1u + index;
  b3_keyed64(k8, msg, out);
}

// rows x r int8 in [-32, 31], one thread per 32-byte hash block; also zeroes zero_me[0..zero_n)
// so per-call counters start clean inside the same launch.
__global__ void noise_uniform_kernel(i8* __restrict__ out, u32 nblocks, const u32* __restrict__ label,
                                     const u32* __restrict__ key, i32* __restrict__ zero_me, int zero_n) {
  const u32 b = blockIdx.x * blockDim.x + threadIdx.x;
  if (zero_me && b < (u32)zero_n) zero_me[b] = 0;
  if (b >= nblocks) return;
  u32 h[8];
  random_hash(b, label, key, 0, h);
  u32 packed[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    // per byte: (y & 63) - 32 is the 6-bit two's-complement value (y & 63) ^ 32, sign-extended
    // to 8 bits by copying its bit 5 into bits 6 and 7 (no carries cross byte lanes).
    const u32 z = (h[i] & 0x3F3F3F3Fu) ^ 0x20202020u, s = z & 0x20202020u;
    packed[i] = z | (s << 1) | (s << 2);
  }
  v4i* dst = reinterpret_cast<v4i*>(out + (u64)b * 32);
  dst[0] = v4i{(int)packed[0], (int)packed[1], (int)packed[2], (int)packed[3]};
  dst[1] = v4i{(int)packed[4], (int)packed[5], (int)packed[6], (int)packed[7]};
}

// k pairs (first | second << 16), one thread per 8 pairs (one digest).
__global__ void noise_perm_kernel(u32* __restrict__ out, u32 k, u32 r, const u32* __restrict__ label,
                                  const u32* __restrict__ key) {
  const u32 i = blockIdx.x * blockDim.x + threadIdx.x;
  if ((u64)i * 8 >= k) return;
  u32 h[8];
  random_hash(i, label, key, 1, h);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const u32 l = i * 8 + j;
    if (l < k) {
      const u32 u = h[j], first = u & (r - 1);
      const u32 second = first ^ (1u + __umulhi(r - 1, u));
      out[l] = first | (second << 16);
    }
  }
}

extern "C" int uwc_noise_uniform(int8_t* out, uint32_t nblocks, const uint32_t* label, const uint32_t* key,
                                 int32_t* zero_me, int zero_n, hipStream_t stream) {
  if (!out || !label || !key) return uwc_fail("uwc_noise_uniform: null out, label or key");
  if (((uintptr_t)out & 15u) != 0) return uwc_fail("uwc_noise_uniform: out must be 16-byte aligned");
  if (zero_n < 0 || (zero_n > 0 && !zero_me)) return uwc_fail("uwc_noise_uniform: bad zero_me/zero_n");
  const u32 work = nblocks > (u32)zero_n ? nblocks : (u32)zero_n;
  if (work == 0) return UWC_OK;
  hipLaunchKernelGGL(noise_uniform_kernel, dim3((work + 255) / 256), dim3(256), 0, stream, out, nblocks, label, key,
                     zero_me, zero_n);
  return uwc_launch_status("noise_uniform");
}

extern "C" int uwc_noise_perm(uint32_t* out, uint32_t k, uint32_t r, const uint32_t* label, const uint32_t* key,
                              hipStream_t stream) {
  if (!out || !label || !key) return uwc_fail("uwc_noise_perm: null out, label or key");
  if (r < 2 || r > 65536 || (r & (r - 1))) return uwc_fail("uwc_noise_perm: r=%u must be a power of two in 2..65536", r);
  if (k == 0) return UWC_OK;
  const u32 nh = (k + 7) / 8;
  hipLaunchKernelGGL(noise_perm_kernel, dim3((nh + 127) / 128), dim3(128), 0, stream, out, k, r, label, key);
  return uwc_launch_status("noise_perm");
}

// ------------------------------------------------------------------ operand noising + projections
// The general-shape form (rows % 8, k % 4) of the per-row operand pass, for shapes the matrix-core
// kernels below do not take. Each of the workgroup's 8 waves owns one row and a private LDS
// region: the row's E entries and its r projection bins. The wave walks the row a dword per lane
// (4 columns, 256 columns per wave step) and, per column l,
//   noising:    dst[l] = int8(src[l] + E[row][Pn.first(l)] - E[row][Pn.second(l)])
//   projection: bin[Pp.first(l)] += src[l], bin[Pp.second(l)] -= src[l]   (LDS integer adds)
// (kernels.cu:303-372). Integer addition is associative, so the order in which the lanes' adds
// land does not change a bin. After one barrier each wave writes its row's bins as `lmax`
// balanced base-128 limbs, copies its E row into every limb, and the workgroup contributes one
// atomic max of |bin| to *maxabs.
#define NRW_WAVES 8
#define NRW_MAXR 256

__device__ __forceinline__ void row_limbs(i8* __restrict__ out, u64 limb_stride, int v, int lmax) {
  // balanced base-128 digits: d = ((v + 64) mod 128) - 64, v <- (v - d) / 128 (exact)
  for (int li = 0; li < lmax; li++) {
    const int d = ((v + 64) & 127) - 64;
    out[li * limb_stride] = (i8)d;
    v = (v - d) >> 7;
  }
}

__global__ void __launch_bounds__(NRW_WAVES * 64) rows_noise_kernel(
    const i8* __restrict__ src, int rows, int k, int r, const i8* __restrict__ E, const u32* __restrict__ Pn,
    i8* __restrict__ dst, const u32* __restrict__ Pp, i8* __restrict__ corr, int corr_off, int ecopy_off,
    i32* __restrict__ maxabs, int lmax) {
  __shared__ i32 bins[NRW_WAVES][NRW_MAXR];
  __shared__ i8 erow[NRW_WAVES][NRW_MAXR];
  __shared__ int wave_max[NRW_WAVES];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * NRW_WAVES + w;
  const i8* srow = src + (u64)row * k;
  for (int j = lane; j < r; j += 64) {
    if (E) erow[w][j] = E[(u64)row * r + j];
    bins[w][j] = 0;
  }
  __syncthreads();
  for (int l0 = 4 * lane; l0 < k; l0 += 256) {
    const u32 word = *reinterpret_cast<const u32*>(srow + l0);
    u32 noised = 0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int x = (int)(i8)(u8)(word >> (8 * b));
      if (dst) {
        const u32 pn = Pn[l0 + b];
        noised |= (u32)(u8)(x + erow[w][pn & 0xFFFF] - erow[w][pn >> 16]) << (8 * b);
      }
      if (Pp) {
        const u32 pp = Pp[l0 + b];
        atomicAdd(&bins[w][pp & 0xFFFF], x);
        atomicAdd(&bins[w][pp >> 16], -x);
      }
    }
    if (dst) *reinterpret_cast<u32*>(dst + (u64)row * k + l0) = noised;
  }
  __syncthreads();
  const u64 limb_stride = (u64)rows * 2 * r, base = (u64)row * 2 * r;
  int mx = 0;
  for (int j = lane; j < r; j += 64) {
    if (Pp) {
      const int v = bins[w][j];
      mx = max(mx, abs(v));
      if (corr_off >= 0) row_limbs(corr + base + corr_off + j, limb_stride, v, lmax);
    }
    if (E && ecopy_off >= 0)
      for (int li = 0; li < lmax; li++) corr[li * limb_stride + base + ecopy_off + j] = erow[w][j];
  }
  if (Pp && maxabs) {
    for (int s = 32; s >= 1; s >>= 1) mx = max(mx, __shfl_xor(mx, s));
    if (lane == 0) wave_max[w] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
      int m = 0;
      for (int i = 0; i < NRW_WAVES; i++) m = max(m, wave_max[i]);
      atomicMax(maxabs, m);  // one same-address atomic per workgroup
    }
  }
}

extern "C" int uwc_noise_rows(const int8_t* src, int rows, int k, int r, const int8_t* E, const uint32_t* Pn,
                              int8_t* dst, const uint32_t* Pp, int8_t* corr, int corr_off, int ecopy_off,
                              int32_t* maxabs, int lmax, hipStream_t stream) {
  if (!src || rows <= 0 || k <= 0 || r <= 0) return uwc_fail("uwc_noise_rows: empty or null src");
  if (rows % NRW_WAVES || k % 4)
    return uwc_fail("uwc_noise_rows: rows=%d must be a multiple of %d and k=%d of 4", rows, NRW_WAVES, k);
  if (r > NRW_MAXR) return uwc_fail("uwc_noise_rows: r=%d above %d", r, NRW_MAXR);
  if (((uintptr_t)src & 3u) || (dst && ((uintptr_t)dst & 3u))) return uwc_fail("uwc_noise_rows: src/dst must be 4-byte aligned");
  if (dst && (!E || !Pn)) return uwc_fail("uwc_noise_rows: noising needs E and Pn");
  if (!corr && ((corr_off >= 0 && Pp) || (ecopy_off >= 0 && E)))
    return uwc_fail("uwc_noise_rows: the limbs (corr_off) and the E copy (ecopy_off) need corr");
  if (!corr) corr_off = ecopy_off = -1;  // nothing to write them from: no projection, no E
  if (corr_off >= 0 || ecopy_off >= 0) {
    if (lmax < 1 || lmax > 4) return uwc_fail("uwc_noise_rows: limbs need lmax in 1..4");
    if ((corr_off >= 0 && corr_off != 0 && corr_off != r) || (ecopy_off >= 0 && ecopy_off != 0 && ecopy_off != r))
      return uwc_fail("uwc_noise_rows: corr_off/ecopy_off must be 0 or r");
  }
  hipLaunchKernelGGL(rows_noise_kernel, dim3(rows / NRW_WAVES), dim3(NRW_WAVES * 64), 0, stream, src, rows, k, r, E, Pn,
                     dst, Pp, corr, corr_off, ecopy_off, maxabs, corr ? lmax : 0);
  return uwc_launch_status("noise_rows");
}

// ------------------------------------------------------------------ projections on the matrix cores
// The projection src * S^T with S the r x k selection matrix of a noise permutation
// (S[j][l] = [P.first(l) == j] - [P.second(l) == j]) is an exact int8 GEMM with N = r: it runs
// on v_mfma_i32_16x16x64_i8 instead of LDS atomics (the reference's PROJ_GEMM path,
// ops.py:145-168). The noising of the same rows rides along in the one pass over src.
//
// Workgroup: 16 rows x all of k, 4 waves; wave w takes the 64-wide k steps j = w, w+4, ...
// Lane l holds 16 bytes of row (l & 15) at k = 64 j + 16 (l >> 4) (the A operand), the same
// k bytes of S row 16 b + (l & 15) (the B operand of output block b), and accumulates
// X[4 (l >> 4) + e][16 b + (l & 15)] in element e. The waves' partial sums meet in LDS.
#define NP_ROWS 16
#define NP_MAXR 128

__global__ void proj_matrix_kernel(const u32* __restrict__ P, int k, int r, i8* __restrict__ St) {
  const u64 total = (u64)r * (k / 16);
  for (u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (u64)gridDim.x * blockDim.x) {
    const int j = (int)(i / (k / 16)), l0 = (int)(i - (u64)j * (k / 16)) * 16;
    u32 w[4];
#pragma unroll
    for (int d = 0; d < 4; d++) {
      u32 o = 0;
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const u32 p = P[l0 + 4 * d + b];
        const int v = (int)((p & 0xFFFF) == (u32)j) - (int)((p >> 16) == (u32)j);
        o |= ((u32)(u8)v) << (8 * b);
      }
      w[d] = o;
    }
    *reinterpret_cast<v4i*>(St + (u64)j * k + l0) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  }
}

// 16 waves per workgroup: wave w takes 64-wide k steps j = w, w + 16, ..., loading every
// fragment of a group of NPF steps before its first MFMA so the memory latency is paid once per
// group, not once per step.
#define NP_WAVES 16
#define NP_THREADS (NP_WAVES * 64)

template <bool NOISE, bool PROJ, int NB, int NPF>
__global__ void __launch_bounds__(NP_THREADS) noise_project_kernel(const i8* __restrict__ src, int rows, int k, int r,
                                                                   const i8* __restrict__ E,
                                                                   const u32* __restrict__ Pn, i8* __restrict__ dst,
                                                                   const i8* __restrict__ St, i8* __restrict__ corr,
                                                                   int corr_off, int ecopy_off,
                                                                   i32* __restrict__ maxabs, int lmax) {
  extern __shared__ __attribute__((aligned(16))) u32 np_P[];  // Pn, k words (NOISE)
  // E rows at stride r + 4 bytes: the 16 rows a wave looks up at once fall in distinct banks
  __shared__ i8 Es[NP_ROWS * (NP_MAXR + 4)];
  __shared__ i32 Xs[NP_ROWS * NP_MAXR];
  __shared__ int wmax[NP_WAVES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int row0 = blockIdx.x * NP_ROWS, es = r + 4;
  if (E)
    for (int i = tid; i < NP_ROWS * r; i += NP_THREADS) Es[(i / r) * es + (i % r)] = E[(u64)row0 * r + i];
  if constexpr (NOISE)
    for (int i = tid; i < k / 4; i += NP_THREADS) reinterpret_cast<v4i*>(np_P)[i] = reinterpret_cast<const v4i*>(Pn)[i];
  if constexpr (PROJ)
    for (int i = tid; i < NP_ROWS * r; i += NP_THREADS) Xs[i] = 0;
  __syncthreads();

  const int rr = lane & 15, kq = (lane >> 4) * 16;
  v4i acc[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) acc[b] = v4i{0, 0, 0, 0};
  const i8* srow = src + (u64)(row0 + rr) * k;
  const int nsteps = k >> 6;
  for (int j0 = wave; j0 < nsteps; j0 += NP_WAVES * NPF) {
    v4i a[NPF], s[NPF][NB];
#pragma unroll
    for (int t = 0; t < NPF; t++) {
      const int j = j0 + t * NP_WAVES;
      if (j < nsteps) {
        a[t] = *reinterpret_cast<const v4i*>(srow + j * 64 + kq);
        if constexpr (PROJ) {
#pragma unroll
          for (int b = 0; b < NB; b++) s[t][b] = *reinterpret_cast<const v4i*>(St + (u64)(b * 16 + rr) * k + j * 64 + kq);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < NPF; t++) {
      const int j = j0 + t * NP_WAVES;
      if (j >= nsteps) break;
      const int kk = j * 64 + kq;
      if constexpr (NOISE) {
        const i8* er = Es + rr * es;
        v4i o;
#pragma unroll
        for (int d = 0; d < 4; d++) {
          const v4i p4 = *reinterpret_cast<const v4i*>(np_P + kk + 4 * d);
          const u32 x = (u32)a[t][d];
          u32 w = 0;
#pragma unroll
          for (int b = 0; b < 4; b++) {
            const u32 p = (u32)p4[b];
            const int v = (int)(i8)(u8)(x >> (8 * b)) + (int)er[p & 0xFFFF] - (int)er[p >> 16];
            w |= ((u32)(u8)v) << (8 * b);
          }
          o[d] = (int)w;
        }
        *reinterpret_cast<v4i*>(dst + (u64)(row0 + rr) * k + kk) = o;
      }
      if constexpr (PROJ) {
#pragma unroll
        for (int b = 0; b < NB; b++) acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[t], s[t][b], acc[b], 0, 0, 0);
      }
    }
  }
  if constexpr (PROJ) {
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int e = 0; e < 4; e++) atomicAdd(&Xs[(4 * (lane >> 4) + e) * r + b * 16 + (lane & 15)], acc[b][e]);
  }
  __syncthreads();
  const u64 limb_stride = (u64)rows * 2 * r;
  int local_max = 0;
  for (int i = tid; i < NP_ROWS * r; i += NP_THREADS) {
    const int ro = i / r, j = i - ro * r;
    const u64 base = (u64)(row0 + ro) * 2 * r;
    if (PROJ && corr_off >= 0) {
      local_max = max(local_max, abs(Xs[i]));
      row_limbs(corr + base + corr_off + j, limb_stride, Xs[i], lmax);
    }
    if (E && ecopy_off >= 0) {
      const i8 e = Es[ro * es + j];
      for (int li = 0; li < lmax; li++) corr[li * limb_stride + base + ecopy_off + j] = e;
    }
  }
  if (PROJ && maxabs) {
    // one global atomic per workgroup: same-address atomics serialize in L2
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) local_max = max(local_max, __shfl_xor(local_max, s));
    if (lane == 0) wmax[wave] = local_max;
    __syncthreads();
    if (tid == 0) {
      int mx = 0;
      for (int w = 0; w < NP_WAVES; w++) mx = max(mx, wmax[w]);
      atomicMax(maxabs, mx);
    }
  }
}

static int np_check(const char* fn, const int8_t* src, int rows, int k, int r) {
  if (!src || rows <= 0 || k <= 0) return uwc_fail("%s: empty or null src", fn);
  if (rows % NP_ROWS || k % 64) return uwc_fail("%s: rows=%d must be a multiple of %d and k=%d of 64", fn, rows, NP_ROWS, k);
  if (r != 16 && r != 32 && r != 64 && r != 128) return uwc_fail("%s: r=%d must be 16, 32, 64 or 128", fn, r);
  if (((uintptr_t)src & 15u)) return uwc_fail("%s: src must be 16-byte aligned", fn);
  if ((size_t)k * 4 > 96 * 1024) return uwc_fail("%s: k=%d too large for the staged noise pairs", fn, k);
  return UWC_OK;
}

template <bool NOISE, bool PROJ, int NB, int NPF>
static void np_go(size_t smem, dim3 grid, hipStream_t stream, const int8_t* src, int rows, int k, int r,
                  const int8_t* E, const uint32_t* Pn, int8_t* dst, const int8_t* St, int8_t* corr, int corr_off,
                  int ecopy_off, int32_t* maxabs, int lmax) {
  auto kern = noise_project_kernel<NOISE, PROJ, NB, NPF>;
  if (smem > 64 * 1024) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
  hipLaunchKernelGGL(kern, grid, dim3(NP_THREADS), smem, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off,
                     ecopy_off, maxabs, lmax);
}

template <int NB, int NPF>
static void np_modes(bool noise, bool proj, size_t smem, dim3 grid, hipStream_t stream, const int8_t* src, int rows,
                     int k, int r, const int8_t* E, const uint32_t* Pn, int8_t* dst, const int8_t* St, int8_t* corr,
                     int corr_off, int ecopy_off, int32_t* maxabs, int lmax) {
  if (noise && proj)
    np_go<true, true, NB, NPF>(smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax);
  else if (noise)
    np_go<true, false, NB, NPF>(smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax);
  else
    np_go<false, true, NB, NPF>(smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax);
}

static int np_launch(bool noise, bool proj, const int8_t* src, int rows, int k, int r, const int8_t* E,
                     const uint32_t* Pn, int8_t* dst, const int8_t* St, int8_t* corr, int corr_off, int ecopy_off,
                     int32_t* maxabs, int lmax, hipStream_t stream) {
  const size_t smem = noise ? (size_t)k * 4 : 0;
  const dim3 grid(rows / NP_ROWS);
  switch (r / 16) {
    case 1: np_modes<1, 4>(noise, proj, smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax); break;
    case 2: np_modes<2, 4>(noise, proj, smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax); break;
    case 4: np_modes<4, 2>(noise, proj, smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax); break;
    case 8: np_modes<8, 1>(noise, proj, smem, grid, stream, src, rows, k, r, E, Pn, dst, St, corr, corr_off, ecopy_off, maxabs, lmax); break;
    default: return uwc_fail("noise_project: r=%d must be 16, 32, 64 or 128", r);
  }
  return uwc_launch_status("noise_project");
}

extern "C" int uwc_proj_matrix(const uint32_t* P, int k, int r, int8_t* St, hipStream_t stream) {
  if (!P || !St || k <= 0 || r <= 0) return uwc_fail("uwc_proj_matrix: null or empty arguments");
  if (k % 16) return uwc_fail("uwc_proj_matrix: k=%d must be a multiple of 16", k);
  if (((uintptr_t)St & 15u) || ((uintptr_t)P & 15u)) return uwc_fail("uwc_proj_matrix: P and St must be 16-byte aligned");
  const u64 total = (u64)r * (k / 16);
  const u64 blocks = (total + 255) / 256;
  hipLaunchKernelGGL(proj_matrix_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream, P, k, r,
                     St);
  return uwc_launch_status("proj_matrix");
}

extern "C" int uwc_project(const int8_t* src, int rows, int k, int r, const int8_t* St, int8_t* corr, int corr_off,
                           int32_t* maxabs, int lmax, hipStream_t stream) {
  int st = np_check("uwc_project", src, rows, k, r);
  if (st) return st;
  if (!St || !corr || lmax < 1 || (corr_off != 0 && corr_off != r))
    return uwc_fail("uwc_project: needs St, corr, lmax >= 1 and corr_off 0 or r");
  return np_launch(false, true, src, rows, k, r, nullptr, nullptr, nullptr, St, corr, corr_off, -1, maxabs, lmax, stream);
}

extern "C" int uwc_noise_project(const int8_t* src, int rows, int k, int r, const int8_t* E, const uint32_t* Pn,
                                 int8_t* dst, const int8_t* St, int8_t* corr, int corr_off, int ecopy_off,
                                 int32_t* maxabs, int lmax, hipStream_t stream) {
  int st = np_check("uwc_noise_project", src, rows, k, r);
  if (st) return st;
  if (!E || !Pn || !dst || ((uintptr_t)dst & 15u) || ((uintptr_t)Pn & 15u))
    return uwc_fail("uwc_noise_project: needs E, 16-byte aligned Pn and dst");
  if (St && (!corr || lmax < 1 || (corr_off != 0 && corr_off != r)))
    return uwc_fail("uwc_noise_project: a projection needs corr, lmax >= 1 and corr_off 0 or r");
  if (ecopy_off >= 0 && (!corr || lmax < 1 || (ecopy_off != 0 && ecopy_off != r)))
    return uwc_fail("uwc_noise_project: the E copy needs corr, lmax >= 1 and ecopy_off 0 or r");
  return np_launch(true, St != nullptr, src, rows, k, r, E, Pn, dst, St, corr, St ? corr_off : -1, ecopy_off, maxabs,
                   corr ? lmax : 0, stream);
}
