// Per-nonce noise kernels of the cuPOW miner on gfx950 (the commitment is uwc_commit.hip):
//   uniform noise E and the noise pairs P (kernels.cu:246-301, reference.py:67-93);
//   operand noising + rank-r projections in balanced base-128 limbs + max |projection|
//   (kernels.cu:303-372).
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
// For NR_ROWS rows per workgroup, optionally:
//   dst[l]  = int8(src[l] + E[row][Pn.first(l)] - E[row][Pn.second(l)])           (noising)
//   proj[j] = sum_l src[l] ([Pp.first(l) == j] - [Pp.second(l) == j])             (projection)
// then proj in `lmax` balanced base-128 limbs to corr[li][row][corr_off + j] (row stride 2r),
// E rows copied to corr[li][row][ecopy_off + j] for every limb, and max |proj| into *maxabs.
// Projection sums use LDS integer atomics: integer addition is associative, so the order in
// which lanes land does not change the result.
#define NR_ROWS 8
__global__ void __launch_bounds__(256) noise_rows_kernel(const i8* __restrict__ src, int rows, int k, int r,
                                                         const i8* __restrict__ E, const u32* __restrict__ Pn,
                                                         i8* __restrict__ dst, const u32* __restrict__ Pp,
                                                         i8* __restrict__ corr, int corr_off, int ecopy_off,
                                                         i32* __restrict__ maxabs, int lmax) {
  extern __shared__ __attribute__((aligned(16))) u8 nr_smem[];
  i8* Es = reinterpret_cast<i8*>(nr_smem);                              // NR_ROWS * r
  i32* proj = reinterpret_cast<i32*>(nr_smem + NR_ROWS * r);            // NR_ROWS * r
  const int row0 = blockIdx.x * NR_ROWS, tid = threadIdx.x;
  if (E)
    for (int i = tid; i < NR_ROWS * r; i += 256) Es[i] = E[(u64)row0 * r + i];
  if (Pp)
    for (int i = tid; i < NR_ROWS * r; i += 256) proj[i] = 0;
  __syncthreads();
  const int quads = k >> 2, total = NR_ROWS * quads;
  for (int it = tid; it < total; it += 256) {
    const int rr = it / quads, q = it - rr * quads;
    const u64 off = (u64)(row0 + rr) * k + 4 * q;
    const u32 w = *reinterpret_cast<const u32*>(src + off);
    u32 o = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int l = 4 * q + j;
      const int x = (int)(i8)(u8)(w >> (8 * j));
      if (dst) {
        const u32 pn = Pn[l];
        const int nv = x + (int)Es[rr * r + (pn & 0xFFFF)] - (int)Es[rr * r + (pn >> 16)];
        o |= ((u32)(u8)nv) << (8 * j);
      }
      if (Pp) {
        const u32 pp = Pp[l];
        atomicAdd(&proj[rr * r + (pp & 0xFFFF)], x);
        atomicSub(&proj[rr * r + (pp >> 16)], x);
      }
    }
    if (dst) *reinterpret_cast<u32*>(dst + off) = o;
  }
  __syncthreads();
  const u64 limb_stride = (u64)rows * 2 * r;
  int local_max = 0;
  for (int i = tid; i < NR_ROWS * r; i += 256) {
    const int rr = i / r, j = i - rr * r;
    const u64 base = (u64)(row0 + rr) * 2 * r;
    if (Pp && corr_off >= 0) {
      int v = proj[i];
      local_max = max(local_max, abs(v));
      for (int li = 0; li < lmax; li++) {
        const int d = ((v + 64) & 127) - 64;
        corr[li * limb_stride + base + corr_off + j] = (i8)d;
        v = (v - d) >> 7;
      }
    }
    if (E && ecopy_off >= 0) {
      const i8 e = Es[i];
      for (int li = 0; li < lmax; li++) corr[li * limb_stride + base + ecopy_off + j] = e;
    }
  }
  if (Pp && maxabs) {
    // wave64 max, then one atomic per wave
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) local_max = max(local_max, __shfl_xor(local_max, s));
    if ((tid & 63) == 0) atomicMax(maxabs, local_max);
  }
}

extern "C" int uwc_noise_rows(const int8_t* src, int rows, int k, int r, const int8_t* E, const uint32_t* Pn,
                              int8_t* dst, const uint32_t* Pp, int8_t* corr, int corr_off, int ecopy_off,
                              int32_t* maxabs, int lmax, hipStream_t stream) {
  if (!src || rows <= 0 || k <= 0 || r <= 0) return uwc_fail("uwc_noise_rows: empty or null src");
  if (rows % NR_ROWS || k % 4) return uwc_fail("uwc_noise_rows: rows=%d must be a multiple of %d and k=%d of 4", rows, NR_ROWS, k);
  if (((uintptr_t)src & 3u) || (dst && ((uintptr_t)dst & 3u))) return uwc_fail("uwc_noise_rows: src/dst must be 4-byte aligned");
  if (dst && (!E || !Pn)) return uwc_fail("uwc_noise_rows: noising needs E and Pn");
  if ((corr_off >= 0 && Pp) || (ecopy_off >= 0 && E)) {
    if (!corr || lmax < 1) return uwc_fail("uwc_noise_rows: limbs need corr and lmax >= 1");
    if ((corr_off >= 0 && corr_off + r > 2 * r) || (ecopy_off >= 0 && ecopy_off + r > 2 * r))
      return uwc_fail("uwc_noise_rows: corr_off/ecopy_off must be 0 or r");
  }
  const size_t smem = (size_t)NR_ROWS * r * 5;
  if (smem > 64 * 1024) return uwc_fail("uwc_noise_rows: r=%d too large", r);
  hipLaunchKernelGGL(noise_rows_kernel, dim3(rows / NR_ROWS), dim3(256), smem, stream, src, rows, k, r, E, Pn, dst, Pp,
                     corr, corr ? corr_off : -1, corr ? ecopy_off : -1, maxabs, corr ? lmax : 0);
  return uwc_launch_status("noise_rows");
}
