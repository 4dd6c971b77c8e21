// gfx950 skinny int8 GEMM for the decode and small-batch shapes (m <= 64): C = X * W^T with
// X m x k (activations) and W n x k (weights), both k-contiguous int8; int32, bf16 or the
// fused detrt fp32 dequant out. At these shapes the product is bound by streaming W from HBM
// once (arithmetic intensity ~2m ops per byte), so the design is about bytes in flight, not
// about matrix-core tiling:
//   * a workgroup owns 16 RG rows of W (output columns) and all m tokens; its KW waves split k
//     into 128-byte slices dealt round-robin (wave w takes slices w, w + KW, ...), so at any
//     time the workgroup reads KW * 128 contiguous bytes of each of its W rows;
//   * W and X fragments go straight from memory to VGPRs (no LDS staging: each W byte is used
//     by exactly one MFMA), U k-steps per batch, the next batch loading while the current one
//     runs on v_mfma_i32_16x16x64_i8 (A = 16 W rows, B = 16 tokens; lane l holds row / token
//     l & 15 and k bytes 16 (l >> 4) .. + 16 of a 64-byte k step);
//   * the KW per-wave int32 partials are summed through LDS (integer sums are exact, so the
//     result does not depend on the split), then the epilogue writes 16 RG contiguous outputs
//     per token row.
// Rows of W past n and tokens past m read a clamped in-bounds row and are never stored.
//
// Replaces, for m <= 64, the exact GEMM of DetLinear.int_gemm / __call__
// (runtime/detrt/qwen3.py:106-126; the reference pads m to 32 and calls torch._int_mm).
#include "uwc_common.h"

#ifndef SK_U
#define SK_U 4  // k steps per load batch
#endif
#define SK_SG 2  // consecutive 64-byte k steps per slice (128 contiguous bytes per W row)
#ifndef SK_RG2_ROWS16
#define SK_RG2_ROWS16 2048  // 16-row groups of W from which a workgroup takes two groups
#endif
#ifndef SK_KW_GRID
#define SK_KW_GRID 512  // workgroups from which a workgroup has 4 waves instead of 8
#endif

typedef const void __attribute__((address_space(1)))* sk_gptr;

__device__ __forceinline__ v4i sk_load(const i8* p) { return *reinterpret_cast<const v4i*>(p); }

__device__ __forceinline__ u32 sk_bf16_rne(float f) {
  const u32 u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// k step index of a wave's j-th step
__device__ __forceinline__ int sk_step(int j, int wave, int KW) {
  return (j / SK_SG) * KW * SK_SG + wave * SK_SG + (j % SK_SG);
}

template <int MT, int RG, int OUT>
__global__ void __launch_bounds__(512) skinny_gemm_kernel(const i8* __restrict__ X, const i8* __restrict__ W, int m,
                                                          int n, int k, const float* __restrict__ sx,
                                                          const float* __restrict__ sw, void* __restrict__ out) {
  extern __shared__ i32 sk_red[];  // [KW][RG][MT][4][64]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, KW = blockDim.x >> 6;
  const int row0 = blockIdx.x * 16 * RG;
  const int ksteps = k >> 6, lr = lane & 15, kb = (lane >> 4) * 16;
  const i8* wp[RG];
  const i8* xp[MT];
#pragma unroll
  for (int g = 0; g < RG; g++) wp[g] = W + (long)min(row0 + 16 * g + lr, n - 1) * k + kb;
#pragma unroll
  for (int t = 0; t < MT; t++) xp[t] = X + (long)min(16 * t + lr, m - 1) * k + kb;

  v4i acc[RG][MT];
#pragma unroll
  for (int g = 0; g < RG; g++)
#pragma unroll
    for (int t = 0; t < MT; t++) acc[g][t] = v4i{0, 0, 0, 0};

  auto load = [&](int j0, v4i w[SK_U][RG], v4i x[SK_U][MT]) {
#pragma unroll
    for (int u = 0; u < SK_U; u++) {
      const long off = (long)sk_step(j0 + u, wave, KW) * 64;
#pragma unroll
      for (int g = 0; g < RG; g++) w[u][g] = sk_load(wp[g] + off);
#pragma unroll
      for (int t = 0; t < MT; t++) x[u][t] = sk_load(xp[t] + off);
    }
  };
  auto mma = [&](const v4i w[SK_U][RG], const v4i x[SK_U][MT]) {
#pragma unroll
    for (int u = 0; u < SK_U; u++)
#pragma unroll
      for (int g = 0; g < RG; g++)
#pragma unroll
        for (int t = 0; t < MT; t++) acc[g][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[u][g], x[u][t], acc[g][t], 0, 0, 0);
  };

  // this wave's steps: j = 0, 1, ... while sk_step(j) < ksteps (steps increase with j)
  int j = 0;
  if (sk_step(SK_U - 1, wave, KW) < ksteps) {
    v4i wa[SK_U][RG], xa[SK_U][MT];
    load(0, wa, xa);
    j = SK_U;
    while (true) {
      const bool more = sk_step(j + SK_U - 1, wave, KW) < ksteps;
      v4i wb[SK_U][RG], xb[SK_U][MT];
      if (more) load(j, wb, xb);
      mma(wa, xa);
      if (!more) break;
#pragma unroll
      for (int u = 0; u < SK_U; u++) {
#pragma unroll
        for (int g = 0; g < RG; g++) wa[u][g] = wb[u][g];
#pragma unroll
        for (int t = 0; t < MT; t++) xa[u][t] = xb[u][t];
      }
      j += SK_U;
    }
  }
  for (; sk_step(j, wave, KW) < ksteps; j++) {
    const long off = (long)sk_step(j, wave, KW) * 64;
#pragma unroll
    for (int g = 0; g < RG; g++) {
      const v4i w = sk_load(wp[g] + off);
#pragma unroll
      for (int t = 0; t < MT; t++) acc[g][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, sk_load(xp[t] + off), acc[g][t], 0, 0, 0);
    }
  }

  // C layout of a 16 x 16 MFMA block: lane l holds rows 4 (l >> 4) + i, column l & 15
#pragma unroll
  for (int g = 0; g < RG; g++)
#pragma unroll
    for (int t = 0; t < MT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) sk_red[(((wave * RG + g) * MT + t) * 4 + i) * 64 + lane] = acc[g][t][i];
  __syncthreads();
  // output o = token * 16 RG + column: consecutive threads write consecutive columns of a token row
  constexpr int NO = 256 * RG * MT;
  for (int o = threadIdx.x; o < NO; o += blockDim.x) {
    const int tl = o / (16 * RG), jl = o % (16 * RG);
    const int tok = tl, col = row0 + jl;
    if (tok >= m || col >= n) continue;
    const int g = jl >> 4, jj = jl & 15, t = tl >> 4;
    const int src = (((g * MT + t) * 4 + (jj & 3)) * 64) + (jj >> 2) * 16 + (tl & 15);
    i32 v = 0;
    for (int w = 0; w < KW; w++) v += sk_red[w * RG * MT * 256 + src];
    const long oi = (long)tok * n + col;
    if constexpr (OUT == UWC_OUT_I32) {
      reinterpret_cast<i32*>(out)[oi] = v;
    } else {
      const float y = __fmul_rn(__fmul_rn((float)v, sx[tok]), sw[col]);
      if constexpr (OUT == UWC_OUT_F32)
        reinterpret_cast<float*>(out)[oi] = y;
      else
        reinterpret_cast<uint16_t*>(out)[oi] = (uint16_t)sk_bf16_rne(y);
    }
  }
}

// The X-stationary form, used when X fits in LDS. At these sizes the kernel is bound by memory
// latency as much as by bandwidth (a 12 MB weight streams in ~2.5 us, one HBM round trip under
// load is ~2 us), so everything a workgroup needs is requested as early as possible:
//   * a persistent workgroup first DMAs all of X into LDS (global_load_lds, no VGPR staging;
//     rows padded by 16 bytes so the 16 rows of a fragment read sit in distinct banks), then
//     issues its first W batch, so X's L2 round trip overlaps W's HBM one;
//   * its 8 waves are KS k-splits x RR row groups: wave (ks, rr) owns W rows rr * 16 RG .. + 16 RG
//     of a row block and the 128-byte k slices ks, ks + KS, ...; the host picks KS and the batch
//     size U so that each wave's share of a row block is one or few batches;
//   * every row block is the same number of U-step batches for every wave and W loads are
//     unconditional (steps past k reload the last step and skip their MFMAs), so the loads run
//     one batch ahead across row-block boundaries with statically known wait counts;
//   * at the end of a row block the KS partials of each row group are summed through LDS, one
//     token group at a time (integer sums: the split cannot change the result).
typedef const void __attribute__((address_space(1)))* s2_gptr;
typedef void __attribute__((address_space(3)))* s2_lptr;

// One wave-wide 16-byte-per-lane DMA into LDS at lds + 16 lane (lds wave-uniform, in M0).
__device__ __forceinline__ void s2_dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// Workgroup barrier for LDS traffic only: waits for this wave's LDS operations, not for its
// global loads and stores (__syncthreads() also fences global memory, which would drain the
// prefetched W loads and the epilogue's output stores at every barrier).
__device__ __forceinline__ void s2_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int MT, int RG, int U, int OUT>
__global__ void __launch_bounds__(512) skinny2_kernel(const i8* __restrict__ X, const i8* __restrict__ W, int m,
                                                      int n, int k, int ks_log, int xpitch,
                                                      const float* __restrict__ sx, const float* __restrict__ sw,
                                                      void* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) u8 s2_lds[];
  i32* red = reinterpret_cast<i32*>(s2_lds + (((long)m * xpitch + 15) & ~15L));  // [8 waves][RG][4][64]
  float* sxl = reinterpret_cast<float*>(red + 8 * RG * 256);                           // [m] token scales
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KS = 1 << ks_log, RR = 8 >> ks_log;
  const int ks = wave & (KS - 1), rr = wave >> ks_log;
  const int rows_blk = RR * 16 * RG;
  const int nblk = (n + rows_blk - 1) / rows_blk;
  const int ksteps = k >> 6, lr = lane & 15, kb = (lane >> 4) * 16;
  // steps of this wave: s(j) = (j / SG) KS SG + ks SG + j % SG; every wave runs nbat batches
  const int nj = SK_SG * ((ksteps + KS * SK_SG - 1) / (KS * SK_SG));
  const int nbat = (nj + U - 1) / U;
  const int G = gridDim.x, bid = blockIdx.x;
  const int nmine = bid < nblk ? (nblk - 1 - bid) / G + 1 : 0;
  const int T = nmine * nbat;
  auto step_of = [&](int j) { return (j / SK_SG) * KS * SK_SG + ks * SK_SG + (j % SK_SG); };
  auto load_unit = [&](int t, v4i w[U][RG]) {
    const int b = t % nbat, rb = bid + (t / nbat) * G;
#pragma unroll
    for (int g = 0; g < RG; g++) {
      const i8* wp = W + (long)min(rb * rows_blk + rr * 16 * RG + 16 * g + lr, n - 1) * k + kb;
#pragma unroll
      for (int u = 0; u < U; u++) w[u][g] = sk_load(wp + (long)min(step_of(b * U + u), ksteps - 1) * 64);
    }
  };

  // X -> LDS: row r, 1 KiB segment s (lanes past the row's end idle); wave w takes segments w, w + 8, ...
  {
    const u32 lbase = (u32)(uintptr_t)(s2_lptr)s2_lds;
    const int spr = (k + 1023) >> 10, cpr = k >> 4;
    for (int seg = wave; seg < m * spr; seg += 8) {
      const int r = seg / spr, sg = seg - r * spr;
      const u32 l = __builtin_amdgcn_readfirstlane(lbase + (u32)(r * xpitch + sg * 1024));
      if (sg * 64 + lane < cpr) s2_dma16(X + (long)r * k + sg * 1024 + lane * 16, l);
    }
  }
  // scales for the dequant epilogue, requested now so no epilogue waits on memory: the token
  // scales go to LDS; a thread's output column is the same in every pass of a row block
  // (512 % rows_blk == 0), so it holds that column's weight scale for the current block
  constexpr bool SCALED = OUT != UWC_OUT_I32;
  float sxv = 0.f, swv = 0.f;
  if constexpr (SCALED) {
    if (threadIdx.x < m) sxv = sx[threadIdx.x];
    if (T > 0) swv = sw[min(bid * rows_blk + (int)threadIdx.x % rows_blk, n - 1)];
  }
  v4i wa[U][RG];
  if (T > 0) load_unit(0, wa);
  if constexpr (SCALED)
    if (threadIdx.x < m) sxl[threadIdx.x] = sxv;
  // the DMAs are older than the U * RG loads just issued: wait for them, then every wave's
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(U * RG) : "memory");
  s2_lds_barrier();
  int xoff[MT];
#pragma unroll
  for (int tg = 0; tg < MT; tg++) xoff[tg] = min(16 * tg + lr, m - 1) * xpitch + kb;

  v4i acc[RG][MT];
#pragma unroll
  for (int g = 0; g < RG; g++)
#pragma unroll
    for (int tg = 0; tg < MT; tg++) acc[g][tg] = v4i{0, 0, 0, 0};

  // unit t: MFMAs on its W registers; after a row block's last unit, the cross-wave reduction
  // and the epilogue
  auto process = [&](int t, const v4i w[U][RG]) {
    const int b = t % nbat;
    if constexpr (SCALED)
      if (b == 0 && t > 0) swv = sw[min((bid + (t / nbat) * G) * rows_blk + (int)threadIdx.x % rows_blk, n - 1)];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int s = step_of(b * U + u);
      if (s < ksteps) {
        v4i xr[MT];
#pragma unroll
        for (int tg = 0; tg < MT; tg++) xr[tg] = *reinterpret_cast<const v4i*>(s2_lds + xoff[tg] + s * 64);
#pragma unroll
        for (int g = 0; g < RG; g++)
#pragma unroll
          for (int tg = 0; tg < MT; tg++) acc[g][tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w[u][g], xr[tg], acc[g][tg], 0, 0, 0);
      }
    }
    if (b == nbat - 1) {
      // row block done: sum the KS partials of each row group, one token group at a time
      const int rb = bid + (t / nbat) * G;
#pragma unroll
      for (int tg = 0; tg < MT; tg++) {
#pragma unroll
        for (int g = 0; g < RG; g++)
#pragma unroll
          for (int i = 0; i < 4; i++) red[((wave * RG + g) * 4 + i) * 64 + lane] = acc[g][tg][i];
        s2_lds_barrier();
        // outputs of this token group: 16 tokens x rows_blk columns, columns fastest
        for (int o = threadIdx.x; o < 16 * rows_blk; o += 512) {
          const int tl = o / rows_blk, cl = o % rows_blk;
          const int tok = 16 * tg + tl, col = rb * rows_blk + cl;
          if (tok < m && col < n) {
            const int orr = cl / (16 * RG), g = (cl / 16) % RG, jj = cl & 15;
            const int src = ((g * 4 + (jj & 3)) * 64) + (jj >> 2) * 16 + tl;
            i32 v = 0;
            for (int q = 0; q < KS; q++) v += red[((orr << ks_log) | q) * RG * 256 + src];
            const long oi = (long)tok * n + col;
            if constexpr (OUT == UWC_OUT_I32) {
              reinterpret_cast<i32*>(out)[oi] = v;
            } else {
              const float y = __fmul_rn(__fmul_rn((float)v, sxl[tok]), swv);
              if constexpr (OUT == UWC_OUT_F32)
                reinterpret_cast<float*>(out)[oi] = y;
              else
                reinterpret_cast<uint16_t*>(out)[oi] = (uint16_t)sk_bf16_rne(y);
            }
          }
        }
        s2_lds_barrier();
      }
#pragma unroll
      for (int g = 0; g < RG; g++)
#pragma unroll
        for (int tg = 0; tg < MT; tg++) acc[g][tg] = v4i{0, 0, 0, 0};
    }
  };
  // two register buffers in turn: unit t + 1 loads while unit t computes, with no copies
  v4i wb[U][RG];
  for (int t = 0; t < T; t += 2) {
    if (t + 1 < T) load_unit(t + 1, wb);
    process(t, wa);
    if (t + 1 >= T) break;
    if (t + 2 < T) load_unit(t + 2, wa);
    process(t + 1, wb);
  }
}

template <int MT, int RG, int U>
static void s2_launch(int out_mode, dim3 grid, size_t lds, hipStream_t s, const i8* X, const i8* W, int m, int n,
                      int k, int ks_log, int xpitch, const float* sx, const float* sw, void* out) {
  auto kern = skinny2_kernel<MT, RG, U, UWC_OUT_F32>;
  if (out_mode == UWC_OUT_I32) kern = skinny2_kernel<MT, RG, U, UWC_OUT_I32>;
  else if (out_mode == UWC_OUT_BF16) kern = skinny2_kernel<MT, RG, U, UWC_OUT_BF16>;
  // one attribute call per instantiation and process (the largest LDS size any launch uses)
  static bool attr[3] = {false, false, false};
  const int oi = out_mode == UWC_OUT_I32 ? 0 : out_mode == UWC_OUT_BF16 ? 1 : 2;
  if (!attr[oi]) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr[oi] = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(512), lds, s, X, W, m, n, k, ks_log, xpitch, sx, sw, out);
}

template <int RG, int U>
static void s2_mt(int mt, int out_mode, dim3 grid, size_t lds, hipStream_t s, const i8* X, const i8* W, int m, int n,
                  int k, int ks_log, int xpitch, const float* sx, const float* sw, void* out) {
  switch (mt) {
    case 1: s2_launch<1, RG, U>(out_mode, grid, lds, s, X, W, m, n, k, ks_log, xpitch, sx, sw, out); break;
    case 2: s2_launch<2, RG, U>(out_mode, grid, lds, s, X, W, m, n, k, ks_log, xpitch, sx, sw, out); break;
    case 3: s2_launch<3, RG, U>(out_mode, grid, lds, s, X, W, m, n, k, ks_log, xpitch, sx, sw, out); break;
    default: s2_launch<4, RG, U>(out_mode, grid, lds, s, X, W, m, n, k, ks_log, xpitch, sx, sw, out); break;
  }
}

template <int MT, int RG>
static void sk_launch(int out_mode, dim3 grid, dim3 block, size_t lds, hipStream_t s, const i8* X, const i8* W, int m,
                      int n, int k, const float* sx, const float* sw, void* out) {
  switch (out_mode) {
    case UWC_OUT_I32:
      hipLaunchKernelGGL((skinny_gemm_kernel<MT, RG, UWC_OUT_I32>), grid, block, lds, s, X, W, m, n, k, sx, sw, out);
      break;
    case UWC_OUT_BF16:
      hipLaunchKernelGGL((skinny_gemm_kernel<MT, RG, UWC_OUT_BF16>), grid, block, lds, s, X, W, m, n, k, sx, sw, out);
      break;
    default:
      hipLaunchKernelGGL((skinny_gemm_kernel<MT, RG, UWC_OUT_F32>), grid, block, lds, s, X, W, m, n, k, sx, sw, out);
      break;
  }
}

template <int RG>
static void sk_mt(int mt, int out_mode, dim3 grid, dim3 block, size_t lds, hipStream_t s, const i8* X, const i8* W,
                  int m, int n, int k, const float* sx, const float* sw, void* out) {
  switch (mt) {
    case 1: sk_launch<1, RG>(out_mode, grid, block, lds, s, X, W, m, n, k, sx, sw, out); break;
    case 2: sk_launch<2, RG>(out_mode, grid, block, lds, s, X, W, m, n, k, sx, sw, out); break;
    case 3: sk_launch<3, RG>(out_mode, grid, block, lds, s, X, W, m, n, k, sx, sw, out); break;
    default: sk_launch<4, RG>(out_mode, grid, block, lds, s, X, W, m, n, k, sx, sw, out); break;
  }
}

#ifndef S2_KS_LOG
#define S2_KS_LOG -1  // k splits per workgroup (log2); -1 = chosen per shape
#endif
#ifndef S2_MAX_LDS
#define S2_MAX_LDS (160 * 1024)  // LDS a workgroup of the X-stationary form may use
#endif
#ifndef S2_RG
#define S2_RG 1
#endif

// Called by uwc_noisy_gemm for plain GEMMs (no flags) with 1 <= m <= 64, k % 64 == 0,
// out_mode I32 / BF16 / F32, operands already checked (16-byte aligned).
int uwc_skinny_gemm(const int8_t* X, const int8_t* W, int m, int n, int k, const float* sx, const float* sw,
                    void* out, int out_mode, hipStream_t stream) {
  const int mt = (m + 15) / 16;
  // X-stationary form when X (padded rows) and the reduction buffer fit in LDS
  const int xpitch = k + 16;
  const int RG2 = S2_RG;
  const size_t lds2 = (((size_t)m * xpitch + 15) & ~(size_t)15) + (size_t)8 * RG2 * 1024 + (size_t)m * 4;
  if (lds2 <= S2_MAX_LDS) {
    const int cus = uwc_cu_count();
    const int per_cu = lds2 <= 80 * 1024 ? 2 : 1;
    const long maxg = (long)cus * per_cu;
    const int ksteps = k >> 6;
    // KS (k splits) and U (steps per batch): the fewest batches per workgroup among the choices
    // that keep at least 3/4 of the workgroup slots busy (or all row blocks, if fewer)
    auto grid_for = [&](int kl) {
      const long rows_blk = (long)(8 >> kl) * 16 * RG2;
      const long nblk = (n + rows_blk - 1) / rows_blk;
      const long iters = (nblk + maxg - 1) / maxg;
      return (nblk + iters - 1) / iters;
    };
    const long fill = grid_for(3);  // KS = 8 always qualifies
    int best_ks = 3, best_u = 8;
    long best_t = -1, best_grid = 0;
    for (int kl = 0; kl <= 3; kl++) {
      if (S2_KS_LOG >= 0 && kl != S2_KS_LOG) continue;
      const long rows_blk = (long)(8 >> kl) * 16 * RG2;
      const long nblk = (n + rows_blk - 1) / rows_blk;
      const long iters = (nblk + maxg - 1) / maxg, grid = grid_for(kl);
      if (S2_KS_LOG < 0 && grid * 4 < fill * 3) continue;
      const int nj = SK_SG * ((ksteps + (SK_SG << kl) - 1) / (SK_SG << kl));
      const int u = nj <= 4 ? 4 : 8;
      const long t = iters * ((nj + u - 1) / u);
      if (best_t < 0 || t < best_t || (t == best_t && grid > best_grid)) {
        best_t = t;
        best_grid = grid;
        best_ks = kl;
        best_u = u;
      }
    }
    const dim3 grid((unsigned)best_grid);
    if (RG2 == 2) {
      if (best_u == 4) s2_mt<2, 4>(mt, out_mode, grid, lds2, stream, X, W, m, n, k, best_ks, xpitch, sx, sw, out);
      else s2_mt<2, 8>(mt, out_mode, grid, lds2, stream, X, W, m, n, k, best_ks, xpitch, sx, sw, out);
    } else {
      if (best_u == 4) s2_mt<1, 4>(mt, out_mode, grid, lds2, stream, X, W, m, n, k, best_ks, xpitch, sx, sw, out);
      else s2_mt<1, 8>(mt, out_mode, grid, lds2, stream, X, W, m, n, k, best_ks, xpitch, sx, sw, out);
    }
    return uwc_launch_status("skinny2_gemm");
  }
  const int rows16 = (n + 15) / 16;
  const int RG = rows16 >= SK_RG2_ROWS16 ? 2 : 1;
  const int grid = (rows16 + RG - 1) / RG;
  const int KW = grid >= SK_KW_GRID ? 4 : 8;
  const size_t lds = (size_t)KW * RG * mt * 256 * sizeof(i32);
  if (RG == 2) sk_mt<2>(mt, out_mode, dim3(grid), dim3(64 * KW), lds, stream, X, W, m, n, k, sx, sw, out);
  else sk_mt<1>(mt, out_mode, dim3(grid), dim3(64 * KW), lds, stream, X, W, m, n, k, sx, sw, out);
  return uwc_launch_status("skinny_gemm");
}
