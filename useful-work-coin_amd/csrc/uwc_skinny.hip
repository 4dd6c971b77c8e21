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
#include <algorithm>

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
// The same with the non-temporal hint, for W: every weight byte is read once per call, and
// cached normally its stream evicts X and the scales, which every workgroup of the XCD rereads
// (Llama-3.1-8B decode layer at M = 1: 51.0 -> 47.7 us).
__device__ __forceinline__ void s2_dma16_nt(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds) : "memory", "m0");
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

// ---------------------------------------------------------------------------------------------
// The DMA-streamed form (k % 1024 == 0): the fastest form wherever the X of a token group fits in
// LDS next to a weight ring of >= 4 entries. Measured on this part, three facts shape it:
//   * W must move as whole 128-byte lines: a wave load of 16 rows x 64 bytes (the MFMA operand
//     layout) streams 25-50% slower than 1 KB contiguous per instruction, while global_load_lds
//     of 1 KB row pieces runs at the contiguous rate. So W goes to LDS by DMA, one 1 KB piece of
//     one row per wave instruction, and is read back in the operand layout (rows padded to 1040
//     bytes: the 16 rows of a fragment read fall in distinct banks);
//   * requests of a CU return in issue order: an L2 hit issued after HBM misses waits for them.
//     X (a few KB to 64 KB, L2-resident) is therefore requested before any W;
//   * X replicated into every CU costs more than streaming W when m k is large (64 x 2048 bytes
//     per workgroup against 48 KB of W each at 64 x 6144 x 2048). Above one group's LDS budget the
//     tokens are split into ts = 2 groups: each workgroup holds half of X and reads its W rows,
//     and the two workgroups of a row block run in the same round on one XCD (round-robin
//     dispatch puts workgroup b on XCD b % 8) so the second read of W is served by that XCD's
//     L2. The mapping is only a locality hint: any placement gives the same result.
// When X is too large to stay resident (e.g. 32 x 14336), it is streamed instead (XS): every ring
// entry carries, ahead of its W rows, the same 1 KB chunk of the group's X rows (8 XD of them),
// and each entry is read once. X then crosses each CU once per block instead of once per
// workgroup, which is the same when a workgroup has one block (n <= 16 x CUs).
// Roles: 8 compute waves and 2 helper waves. Compute wave w DMAs rows w and w + 8 of each ring
// entry (16 rows x 1 KB of one k chunk) and runs the MFMAs of the 128-byte piece w of every
// chunk: v_mfma_i32_16x16x64_i8 with A = 16 W rows from the ring, B = 16 tokens from the X copy.
// At a block's end the 8 partial sums go to LDS; helper (block % 2) adds them, applies the
// epilogue and stores. Only DMAs ever touch the compute waves' vmcnt, so every wait count is
// static. Stores live in the helpers; the weight scales of the workgroup's blocks are DMA'd to
// LDS at the start (lane l of a DMA gathers 16 bytes of block l / 4), so a helper's block loop
// has no global loads, and with blocks alternating between two helpers the register reuse that
// makes a helper wait for its stores finds them two blocks old.
#define SD_PITCH 1040  // LDS bytes per W row of a ring entry (1 KB + 16)
#define SD_ENTRY (16 * SD_PITCH)
#define SD_MAX_NE 6

typedef void __attribute__((address_space(3)))* sd_lptr;

// wait until at most `younger` ring entries (ND DMAs each) issued after the awaited one are pending
template <int N>
__device__ __forceinline__ void sd_waitv() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
template <int NE, int ND>
__device__ __forceinline__ void sd_wait_entries(int younger) {
  switch (younger) {
    case 0: sd_waitv<0>(); break;
    case 1: if constexpr (NE >= 3) sd_waitv<ND>(); break;
    case 2: if constexpr (NE >= 4) sd_waitv<2 * ND>(); break;
    case 3: if constexpr (NE >= 5) sd_waitv<3 * ND>(); break;
    default: if constexpr (NE >= 6) sd_waitv<4 * ND>(); break;
  }
}

// XD: 0 = X resident; > 0 = X streamed, 8 XD X rows per entry (XD DMAs per compute wave)
template <int MT, int NE, int NPB, int XD, int OUT>
__global__ void __launch_bounds__(640) skinny_dma_kernel(const i8* __restrict__ X, const i8* __restrict__ W, int m, int n,
                                                         int k, int ts, const float* __restrict__ sx,
                                                         const float* __restrict__ sw, void* __restrict__ out) {
  static_assert(NE >= 2 && NE <= SD_MAX_NE, "ring depth");
  constexpr int PART = 8 * MT * 1024;        // bytes of one partials buffer: [8 waves][MT][64 lanes] v4i
  constexpr int XR = 8 * XD;                 // X rows of a streamed entry (before its 16 W rows)
  constexpr int ENTRY = (XR + 16) * SD_PITCH;
  constexpr int ND = 2 + XD;                 // DMAs per compute wave per entry
  extern __shared__ __attribute__((aligned(16))) u8 sd_lds[];
  const u32 lbase = (u32)(uintptr_t)(sd_lptr)sd_lds;
  const int cpb = k >> 10;       // 1 KB chunks per row
  const int mg = m / ts;         // tokens of a group
  const int xpitch = XD ? SD_PITCH : k + 16;
  u8* xl = sd_lds + NE * ENTRY;  // resident X (XD == 0)
  v4i* part = reinterpret_cast<v4i*>(xl + (XD ? 0 : (((long)mg * xpitch + 15) & ~15L)));
  const float* swl = reinterpret_cast<const float*>(part + NPB * (PART / 16));  // [block][16] weight scales
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nblk = (n + 15) >> 4;
  // tasks (16-row block, token group): workgroup b = 8 l + x takes group h = l % ts and, in round
  // r, block x + 8 ((r G / 8 + l) / ts)
  const int x8 = blockIdx.x & 7, l = blockIdx.x >> 3, G8 = gridDim.x >> 3;
  const int h = l % ts;
  const int tasks = (x8 < nblk ? (nblk - 1 - x8) / 8 + 1 : 0) * ts;
  const int nmine = l < tasks ? (tasks - 1 - l) / G8 + 1 : 0;
  const int E = nmine * cpb;  // ring entries of this workgroup
  if (E == 0) return;
  auto block_of = [&](int r) { return x8 + 8 * ((r * G8 + l) / ts); };
  const i8* Xg = X + (long)h * mg * k;

  if (wave < 8) {
    // resident X of the group first (row r by wave r % 8), then the first NE - 1 ring entries
    if constexpr (XD == 0) {
      for (int r = wave; r < mg; r += 8)
        for (int c = 0; c < cpb; c++)
          s2_dma16(Xg + (long)r * k + c * 1024 + lane * 16,
                   __builtin_amdgcn_readfirstlane(lbase + (u32)(NE * ENTRY + r * xpitch + c * 1024)));
    }
    auto dma_entry = [&](int e) {
      const int i = e / cpb, c = e - i * cpb;
      const int row0 = block_of(i) * 16;
      const u32 slot = lbase + (u32)((e % NE) * ENTRY);
#pragma unroll
      for (int t = 0; t < XD; t++) {  // streamed X rows (rows past the group repeat its last one)
        const int r = wave + 8 * t;
        s2_dma16(Xg + (long)min(r, mg - 1) * k + c * 1024 + lane * 16,
                 __builtin_amdgcn_readfirstlane(slot + r * SD_PITCH));
      }
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const int r = wave + 8 * t;
        s2_dma16_nt(W + (long)min(row0 + r, n - 1) * k + c * 1024 + lane * 16,
                    __builtin_amdgcn_readfirstlane(slot + (XR + r) * SD_PITCH));
      }
    };
    const int pro = min(NE - 1, E);
    for (int e = 0; e < pro; e++) dma_entry(e);
    int xo[MT];
#pragma unroll
    for (int tg = 0; tg < MT; tg++) xo[tg] = min(16 * tg + (lane & 15), mg - 1) * xpitch + 128 * wave + 16 * (lane >> 4);
    const int wo = (XR + (lane & 15)) * SD_PITCH + 128 * wave + 16 * (lane >> 4);
    v4i acc[MT];
#pragma unroll
    for (int tg = 0; tg < MT; tg++) acc[tg] = v4i{0, 0, 0, 0};
    int i = 0, c = 0;
    for (int e = 0; e < E; e++) {
      // entry e landed (the X copy too, being older), in every wave's share
      sd_wait_entries<NE, ND>(min(NE - 2, E - 1 - e));
      s2_lds_barrier();
      if (e + NE - 1 < E) dma_entry(e + NE - 1);
      const u8* slot = sd_lds + (e % NE) * ENTRY;
      const u8* xc = XD ? slot : xl + c * 1024;  // this chunk's X rows
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const v4i a = *reinterpret_cast<const v4i*>(slot + wo + 64 * u);
        v4i b[MT];
#pragma unroll
        for (int tg = 0; tg < MT; tg++) b[tg] = *reinterpret_cast<const v4i*>(xc + xo[tg] + 64 * u);
#pragma unroll
        for (int tg = 0; tg < MT; tg++) acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[tg], acc[tg], 0, 0, 0);
      }
      if (++c == cpb) {
        v4i* pb = part + (NPB == 2 ? (i & 1) * (PART / 16) : 0);
#pragma unroll
        for (int tg = 0; tg < MT; tg++) {
          pb[(wave * MT + tg) * 64 + lane] = acc[tg];
          acc[tg] = v4i{0, 0, 0, 0};
        }
        s2_lds_barrier();
        c = 0;
        i++;
      }
    }
  } else {
    // helpers: per block, the sum of the 8 partials and the epilogue. Lane l holds outputs
    // (token 16 tg + (l & 15) of the group, columns 4 (l >> 4) .. + 3 of the block). Every
    // barrier of a helper waits for its LDS reads first: the partials buffer a helper reads is
    // written again only after a later barrier.
    constexpr bool SCALED = OUT != UWC_OUT_I32;
    const int hw = wave - 8;
    float sxv[MT];
#pragma unroll
    for (int tg = 0; tg < MT; tg++) sxv[tg] = SCALED ? sx[h * mg + min(16 * tg + (lane & 15), mg - 1)] : 0.f;
    if constexpr (SCALED) {
      // the blocks' weight scales to LDS: DMA q, lane l -> block 16 q + l / 4, floats 4 (l % 4) ..
      const u32 swb = lbase + (u32)((const u8*)swl - sd_lds);
      for (int q = 0; q < (nmine + 15) / 16; q++) {
        const int bi = min(16 * q + (lane >> 2), nmine - 1);
        s2_dma16(sw + min(block_of(bi) * 16 + 4 * (lane & 3), n - 4), __builtin_amdgcn_readfirstlane(swb + q * 1024));
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    for (int i = 0; i < nmine; i++) {
      for (int c = 0; c < cpb; c++) s2_lds_barrier();  // the block's ring entries
      s2_lds_barrier();                                 // its partials written
      if ((i & 1) != hw) continue;
      const int col = block_of(i) * 16 + 4 * (lane >> 4);
      const v4i* pb = part + (NPB == 2 ? (i & 1) * (PART / 16) : 0);
      v4i s[MT];
#pragma unroll
      for (int tg = 0; tg < MT; tg++) {
        s[tg] = pb[tg * 64 + lane];
#pragma unroll
        for (int w = 1; w < 8; w++) s[tg] += pb[(w * MT + tg) * 64 + lane];
      }
      float4 y[MT];
      if constexpr (SCALED) {
        const float4 swv = *reinterpret_cast<const float4*>(swl + i * 16 + 4 * (lane >> 4));
#pragma unroll
        for (int tg = 0; tg < MT; tg++) {
          y[tg].x = __fmul_rn(__fmul_rn((float)s[tg][0], sxv[tg]), swv.x);
          y[tg].y = __fmul_rn(__fmul_rn((float)s[tg][1], sxv[tg]), swv.y);
          y[tg].z = __fmul_rn(__fmul_rn((float)s[tg][2], sxv[tg]), swv.z);
          y[tg].w = __fmul_rn(__fmul_rn((float)s[tg][3], sxv[tg]), swv.w);
        }
      }
#pragma unroll
      for (int tg = 0; tg < MT; tg++) {
        const int tl = 16 * tg + (lane & 15);
        if (tl < mg && col < n) {
          const long o = (long)(h * mg + tl) * n + col;
          if constexpr (OUT == UWC_OUT_I32) {
            *reinterpret_cast<v4i*>(reinterpret_cast<i32*>(out) + o) = s[tg];
          } else if constexpr (OUT == UWC_OUT_F32) {
            *reinterpret_cast<float4*>(reinterpret_cast<float*>(out) + o) = y[tg];
          } else {
            const uint2 b = {sk_bf16_rne(y[tg].x) | (sk_bf16_rne(y[tg].y) << 16),
                             sk_bf16_rne(y[tg].z) | (sk_bf16_rne(y[tg].w) << 16)};
            *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + o) = b;
          }
        }
      }
    }
  }
}

// LDS bytes of the DMA-streamed form: ring, one group's X (rows of k + 16), partials
static size_t sd_lds_bytes(int ne, int npb, int xd, int mg, int k, int mt, int nmine_max) {
  const size_t xres = xd ? 0 : (((size_t)mg * (k + 16)) + 15) & ~(size_t)15;
  return (size_t)ne * (8 * xd + 16) * SD_PITCH + xres + (size_t)npb * 8 * mt * 1024 +
         (size_t)((nmine_max + 15) / 16) * 1024;
}

template <int MT, int NE, int NPB, int XD>
static void sd_launch(int out_mode, int G, size_t lds, hipStream_t s, const i8* X, const i8* W, int m, int n, int k,
                      int ts, const float* sx, const float* sw, void* out) {
  auto kern = skinny_dma_kernel<MT, NE, NPB, XD, UWC_OUT_F32>;
  if (out_mode == UWC_OUT_I32) kern = skinny_dma_kernel<MT, NE, NPB, XD, UWC_OUT_I32>;
  else if (out_mode == UWC_OUT_BF16) kern = skinny_dma_kernel<MT, NE, NPB, XD, UWC_OUT_BF16>;
  static bool attr[3] = {false, false, false};
  const int oi = out_mode == UWC_OUT_I32 ? 0 : out_mode == UWC_OUT_BF16 ? 1 : 2;
  if (!attr[oi]) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    attr[oi] = true;
  }
  hipLaunchKernelGGL(kern, dim3(G), dim3(640), lds, s, X, W, m, n, k, ts, sx, sw, out);
}

template <int MT, int XD>
static void sd_ne(int ne, int npb, int out_mode, int G, size_t lds, hipStream_t s, const i8* X, const i8* W, int m,
                  int n, int k, int ts, const float* sx, const float* sw, void* out) {
  if (npb == 2) {
    switch (ne) {
      case 4: sd_launch<MT, 4, 2, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
      case 5: sd_launch<MT, 5, 2, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
      default: sd_launch<MT, 6, 2, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
    }
  } else {
    switch (ne) {
      case 4: sd_launch<MT, 4, 1, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
      case 5: sd_launch<MT, 5, 1, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
      default: sd_launch<MT, 6, 1, XD>(out_mode, G, lds, s, X, W, m, n, k, ts, sx, sw, out); break;
    }
  }
}

// The DMA-streamed form's plan for (m, n, k), or false when it does not apply: token groups ts
// (1, else 2), X resident (xd = 0) or streamed (xd = 1, 2, 4: rows of 8 per entry), ring depth ne
// (4..6), partials buffers npb (2, else 1), grid, LDS bytes. Resident X is preferred; streaming
// takes the shapes whose group X does not fit beside a 4-entry ring.
struct SdPlan {
  int ts, xd, ne, npb, mt, grid;
  size_t lds;
};
static bool sd_plan(int m, int n, int k, SdPlan* p) {
  if (k % 1024 != 0 || n % 4 != 0 || m < 1 || m > 64) return false;
  const int grid = uwc_cu_count() & ~15;  // a multiple of 16: G / 8 is a multiple of ts
  if (grid < 16) return false;
  const int nblk = (n + 15) / 16;
  for (int stream = 0; stream <= 1; stream++)
    for (int ts = 1; ts <= 2; ts++) {
      if (m % ts) continue;
      const int mg = m / ts, mt = (mg + 15) / 16;
      const int xd = stream ? (mg <= 8 ? 1 : mg <= 16 ? 2 : mg <= 32 ? 4 : 0) : 0;
      if (stream && xd == 0) continue;
      // most tasks of a workgroup: tasks of the busiest XCD over its G / 8 workgroups
      const int nmine_max = ((nblk + 7) / 8 * ts + grid / 8 - 1) / (grid / 8);
      for (int npb = 2; npb >= 1; npb--)
        for (int ne = SD_MAX_NE; ne >= 4; ne--) {
          const size_t lds = sd_lds_bytes(ne, npb, xd, mg, k, mt, nmine_max);
          if (lds <= 160 * 1024) {
            // at least 81 KB: one workgroup per CU, so the dispatcher spreads them over every CU
            *p = SdPlan{ts, xd, ne, npb, mt, grid, std::max(lds, (size_t)81 * 1024)};
            return true;
          }
        }
    }
  return false;
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
  SdPlan sp;
  const bool vec_ok = ((uintptr_t)out & 15) == 0 && (out_mode == UWC_OUT_I32 || ((uintptr_t)sw & 15) == 0);
  if (vec_ok && sd_plan(m, n, k, &sp)) {
#define SD_GO(MT, XD) sd_ne<MT, XD>(sp.ne, sp.npb, out_mode, sp.grid, sp.lds, stream, X, W, m, n, k, sp.ts, sx, sw, out)
    if (sp.xd == 0) {
      switch (sp.mt) {
        case 1: SD_GO(1, 0); break;
        case 2: SD_GO(2, 0); break;
        case 3: SD_GO(3, 0); break;
        default: SD_GO(4, 0); break;
      }
    } else if (sp.xd == 1) {
      SD_GO(1, 1);
    } else if (sp.xd == 2) {
      SD_GO(1, 2);
    } else if (sp.mt == 1) {
      SD_GO(1, 4);
    } else {
      SD_GO(2, 4);
    }
#undef SD_GO
    return uwc_launch_status("skinny_dma_gemm");
  }
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
