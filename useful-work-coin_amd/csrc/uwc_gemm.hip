// gfx950 int8 x int8 -> int32 GEMM with the cuPOW transcript: C = A * B^T, A m x k, B n x k
// (both k-contiguous). One kernel serves the miner (FLAG_HASH: fold + BLAKE3 tile digests +
// win records; FLAG_DENOISE: exact low-rank correction) and the detrt linear (plain GEMM with
// an int32, bf16 or fp32-dequant epilogue).
//
// Semantics follow miner/ampere/uwc_ampere/kernels.cu:482-715 (noisy_gemm) and
// reference.py:111-125 (jackpot transcript); the design is CDNA4's own:
//   * workgroup tile 128 x 128 x 64, 4 wave64s in 2 x 2, each wave owns one 64 x 64 block;
//     v_mfma_i32_32x32x32_i8 (2 x 2 MFMA blocks per wave, 64 int32 accumulators per lane);
//   * the consensus hash tile (rows g + 8i, cols 2t + e + 8j inside a 64 x 64 block,
//     miner/ampere/uwc_ampere/pearl_glue.py:14-15) is spread by the MFMA C layout
//     (row = 8(e>>2) + 4(lane>>5) + (e&3), col = lane&31) over lane bits 0, 3, 4 and
//     accumulator index e>>2. Each fold XORs a lane's accumulators into 4 per-lane partials
//     (one per g&3) and folds them into per-lane partial messages; rotl13 and XOR are linear
//     over GF(2), so the cross-lane XOR of the partial messages, done once after the k loop,
//     equals the reference's per-fold tile XOR;
//   * k is reduced in a fixed order (k tiles ascending, 32 k per MFMA): int32 sums are exact,
//     so every tiling gives identical accumulators at every r boundary.
#include <stdarg.h>
#include <stdio.h>

#include "uwc_common.h"

#define G_BM 128
#define G_BN 128
#define G_BK 64
#define G_PITCH 80  // LDS bytes per tile row: 64 data + 16 pad, conflict-free 16-byte fragment reads
#define G_THREADS 256
#define G_TILE_BYTES (G_BM * G_PITCH)          // one operand tile in LDS
#define G_STAGE_BYTES (2 * G_TILE_BYTES)       // A + B
#define G_MSG_BYTES (4 * 4 * 16 * 64 * 4)      // 4 waves x 4 partials x 16 words x 64 lanes
#define G_LDS_BYTES (G_MSG_BYTES > 2 * G_STAGE_BYTES ? G_MSG_BYTES : 2 * G_STAGE_BYTES)

#define FLAG_HASH 1
#define FLAG_DENOISE 2
#define FLAG_TILE128 0x100  // force the 128 x 128 kernel (same results; for tests and small shapes)
// force configuration c of the plain DMA kernel (uwc_gemm_plain.hip) for a plain GEMM:
// FLAG_PLAIN | c << FLAG_PLAIN_SHIFT (same results; for tests and tuning)
#define FLAG_PLAIN 0x200
#define FLAG_PLAIN_SHIFT 12
#define FLAG_PLAIN_MASK (0xF << FLAG_PLAIN_SHIFT)
#define OUT_NONE 0
#define OUT_I32 1
#define OUT_BF16 2
#define OUT_F32 3
#define WIN_WORDS 10
#define DUMP_WORDS 24  // per tile: 16 message words + 8 digest words

struct GemmParams {
  const i8* A;
  const i8* B;
  int m, n, k, r;
  const i8* corrA;
  const i8* corrB;
  const i32* maxabs;
  int lmax;
  const u32* key;
  const u32* target;
  u32* wins;
  int max_wins;
  const float* a_scale;
  const float* b_scale;
  void* out;
  u32* dump;
  int ldc;  // output row stride in elements (n unless the GEMM writes a column slice)
};

// Global -> register prefetch of one 128 x 64 operand tile: 512 16-byte pieces, 2 per thread.
struct TileRegs {
  v4i a[2], b[2];
};

__device__ __forceinline__ v4i load16(const i8* base, long row, int rows, long ld, int col) {
  if (row < rows) return *reinterpret_cast<const v4i*>(base + row * ld + col);
  return v4i{0, 0, 0, 0};
}

__device__ __forceinline__ void tile_load(TileRegs& t, const i8* A, long lda, int arows, const i8* B, long ldb,
                                          int brows, int bm0, int bn0, int k0, int tid) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int idx = tid + i * G_THREADS, row = idx >> 2, c = idx & 3;
    t.a[i] = load16(A, (long)bm0 + row, arows, lda, k0 + c * 16);
    t.b[i] = load16(B, (long)bn0 + row, brows, ldb, k0 + c * 16);
  }
}

__device__ __forceinline__ void tile_store(const TileRegs& t, u8* stage, int tid) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int idx = tid + i * G_THREADS, row = idx >> 2, c = idx & 3;
    *reinterpret_cast<v4i*>(stage + row * G_PITCH + c * 16) = t.a[i];
    *reinterpret_cast<v4i*>(stage + G_TILE_BYTES + row * G_PITCH + c * 16) = t.b[i];
  }
}

// 64 k of MFMA work for one wave's 64 x 64 block from an LDS stage.
__device__ __forceinline__ void tile_mma(v16i acc[2][2], const u8* stage, int wm, int wn, int lane) {
  const u8* sA = stage + (wm * 64 + (lane & 31)) * G_PITCH + (lane >> 5) * 16;
  const u8* sB = stage + G_TILE_BYTES + (wn * 64 + (lane & 31)) * G_PITCH + (lane >> 5) * 16;
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    v4i a0 = *reinterpret_cast<const v4i*>(sA + ks * 32);
    v4i a1 = *reinterpret_cast<const v4i*>(sA + 32 * G_PITCH + ks * 32);
    v4i b0 = *reinterpret_cast<const v4i*>(sB + ks * 32);
    v4i b1 = *reinterpret_cast<const v4i*>(sB + 32 * G_PITCH + ks * 32);
    acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc[0][0], 0, 0, 0);
    acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, acc[0][1], 0, 0, 0);
    acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, acc[1][0], 0, 0, 0);
    acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc[1][1], 0, 0, 0);
  }
}

// Runs k tiles [kt_begin, kt_end) of a double-buffered pipeline whose stage (kt_begin & 1)
// already holds tile kt_begin. On return stage (kt_end & 1) holds tile kt_end (if < kt_total).
__device__ __forceinline__ void run_ktiles(v16i acc[2][2], u8* smem, const i8* A, long lda, int arows, const i8* B,
                                           long ldb, int brows, int bm0, int bn0, int kt_begin, int kt_end,
                                           int kt_total, int tid, int wm, int wn, int lane) {
  for (int kt = kt_begin; kt < kt_end; kt++) {
    TileRegs t;
    const bool more = kt + 1 < kt_total;
    if (more) tile_load(t, A, lda, arows, B, ldb, brows, bm0, bn0, (kt + 1) * G_BK, tid);
    tile_mma(acc, smem + (kt & 1) * G_STAGE_BYTES, wm, wn, lane);
    if (more) tile_store(t, smem + ((kt + 1) & 1) * G_STAGE_BYTES, tid);
    __syncthreads();
  }
}

__device__ __forceinline__ u32 xor3(u32 a, u32 b, u32 c) { return a ^ b ^ c; }

// Per-lane partial tile XOR: x[p] = XOR of this lane's accumulators with (e & 3) == p.
__device__ __forceinline__ void fold_partials(const v16i acc[2][2], u32 x[4]) {
#pragma unroll
  for (int p = 0; p < 4; p++) {
    u32 v = 0;
#pragma unroll
    for (int mb = 0; mb < 2; mb++)
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
        v = xor3(v, (u32)acc[mb][nb][p] ^ (u32)acc[mb][nb][4 + p], (u32)acc[mb][nb][8 + p] ^ (u32)acc[mb][nb][12 + p]);
    x[p] = v;
  }
}

__device__ __forceinline__ u32 rotl13(u32 x) { return __builtin_amdgcn_alignbit(x, x, 19); }

__device__ __forceinline__ u32 bf16_rne(float f) {
  const u32 u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Workgroup id -> (bm0, bn0). Consecutive ids are dispatched round-robin over the 8 XCDs;
// regrouping them gives each XCD a contiguous run, rastered in column groups of GROUP_M row
// tiles so neighbouring workgroups on one XCD share A and B tiles in that XCD's L2.
__device__ __forceinline__ void tile_coords(int m, int n, int& bm0, int& bn0) {
  const int npm = (m + G_BM - 1) / G_BM, npn = (n + G_BN - 1) / G_BN, total = npm * npn;
  int pid = blockIdx.x;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  constexpr int GROUP_M = 8;
  const int grp = GROUP_M * npn, gid = pid / grp, first = gid * GROUP_M;
  const int gsz = min(npm - first, GROUP_M), in = pid - gid * grp;
  bm0 = (first + in % gsz) * G_BM;
  bn0 = (in / gsz) * G_BN;
}

template <bool HASH, bool DENOISE, int OUT>
__global__ void __launch_bounds__(G_THREADS) noisy_gemm_kernel(GemmParams p) {
  __shared__ __attribute__((aligned(16))) u8 smem[G_LDS_BYTES];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wm = wave >> 1, wn = wave & 1;
  int bm0, bn0;
  tile_coords(p.m, p.n, bm0, bn0);
  const long k = p.k;
  const int KT = p.k / G_BK;

  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = v16i{};

  {
    TileRegs t;
    tile_load(t, p.A, k, p.m, p.B, k, p.n, bm0, bn0, 0, tid);
    tile_store(t, smem, tid);
    __syncthreads();
  }

  if constexpr (HASH) {
    u32 msg[4][16];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int w = 0; w < 16; w++) msg[q][w] = 0;
    const int tpc = p.r / G_BK, nchunks = p.k / p.r;
    int kt = 0;
    for (int c0 = 0; c0 < nchunks; c0 += 16) {
#pragma unroll
      for (int s = 0; s < 16; s++) {
        if (c0 + s < nchunks) {
          run_ktiles(acc, smem, p.A, k, p.m, p.B, k, p.n, bm0, bn0, kt, kt + tpc, KT, tid, wm, wn, lane);
          kt += tpc;
          u32 x[4];
          fold_partials(acc, x);
#pragma unroll
          for (int q = 0; q < 4; q++) msg[q][s] = rotl13(msg[q][s]) ^ x[q];
        }
      }
    }
    // Cross-lane combine of the partial messages through LDS (the pipeline buffers are free:
    // the last iteration ended with a barrier and loaded nothing).
    u32* ms = reinterpret_cast<u32*>(smem);
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int w = 0; w < 16; w++) ms[((wave * 4 + q) * 16 + w) * 64 + lane] = msg[q][w];
    __syncthreads();
    if (tid < 128) {
      // thread h digests tile (g, t) of wave wv's 64 x 64 block
      const int wv = tid >> 5, j = tid & 31, g = j >> 2, t = j & 3, q = g & 3;
      const int base = (g >> 2) * 32 + 2 * t;
      u32 mw[16];
#pragma unroll
      for (int w = 0; w < 16; w++) {
        const u32* src = ms + ((wv * 4 + q) * 16 + w) * 64 + base;
        u32 v = 0;
#pragma unroll
        for (int b34 = 0; b34 < 4; b34++) v ^= src[8 * b34] ^ src[8 * b34 + 1];
        mw[w] = v;
      }
      u32 key[8], h[8];
#pragma unroll
      for (int i = 0; i < 8; i++) key[i] = p.key[i];
      b3_keyed64(key, mw, h);
      const int row = bm0 + (wv >> 1) * 64 + g, col = bn0 + (wv & 1) * 64 + 2 * t;
      if (p.dump) {
        const long NB = p.n / 64;
        u32* d = p.dump + ((((long)(row >> 6) * 8 + g) * NB + (col >> 6)) * 4 + t) * DUMP_WORDS;
#pragma unroll
        for (int w = 0; w < 16; w++) d[w] = mw[w];
#pragma unroll
        for (int w = 0; w < 8; w++) d[16 + w] = h[w];
      }
      if (p.wins && u256_le(h, p.target)) {
        const u32 slot = atomicAdd(p.wins, 1u);
        if (slot < (u32)p.max_wins) {
          u32* rec = p.wins + 1 + slot * WIN_WORDS;
          rec[0] = row;
          rec[1] = col;
#pragma unroll
          for (int i = 0; i < 8; i++) rec[2 + i] = h[i];
        }
      }
    }
    __syncthreads();
  } else {
    run_ktiles(acc, smem, p.A, k, p.m, p.B, k, p.n, bm0, bn0, 0, KT, KT, tid, wm, wn, lane);
  }

  if constexpr (DENOISE) {
    // acc -= sum_li 128^li [X_li | EAL] [EBRt | Y_li]^T, Horner over limbs, exact mod 2^32
    // (kernels.cu:598-673). Operands: corrA (lmax, m, 2r), corrB (lmax, n, 2r) int8.
    const int mx = max(p.maxabs[0], p.maxabs[1]);
    int L = mx > 1040319 ? 4 : mx > 8127 ? 3 : mx > 63 ? 2 : 1;
    L = min(L, p.lmax);
    const long R2 = 2L * p.r;
    const int CKT = (int)(R2 / G_BK);
    v16i tmp[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) tmp[i][j] = v16i{};
    for (int li = L - 1; li >= 0; li--) {
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) tmp[i][j] = tmp[i][j] << 7;
      const i8* cA = p.corrA + (long)li * p.m * R2;
      const i8* cB = p.corrB + (long)li * p.n * R2;
      TileRegs t;
      tile_load(t, cA, R2, p.m, cB, R2, p.n, bm0, bn0, 0, tid);
      tile_store(t, smem, tid);
      __syncthreads();
      run_ktiles(tmp, smem, cA, R2, p.m, cB, R2, p.n, bm0, bn0, 0, CKT, CKT, tid, wm, wn, lane);
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] -= tmp[i][j];
  }

  if constexpr (OUT != OUT_NONE) {
    // lane holds col (lane & 31) of rows 8(e>>2) + 4(lane>>5) + (e&3) of each 32 x 32 block
#pragma unroll
    for (int mb = 0; mb < 2; mb++) {
#pragma unroll
      for (int nb = 0; nb < 2; nb++) {
        const int col = bn0 + wn * 64 + nb * 32 + (lane & 31);
        if (col >= p.n) continue;
        float bsc = 0.f;
        if constexpr (OUT == OUT_BF16 || OUT == OUT_F32) bsc = p.b_scale[col];
#pragma unroll
        for (int e = 0; e < 16; e++) {
          const int row = bm0 + wm * 64 + mb * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          if (row >= p.m) continue;
          const long o = (long)row * p.ldc + col;
          const int v = acc[mb][nb][e];
          if constexpr (OUT == OUT_I32) {
            reinterpret_cast<i32*>(p.out)[o] = v;
          } else {
            const float y = __fmul_rn(__fmul_rn((float)v, p.a_scale[row]), bsc);
            if constexpr (OUT == OUT_F32)
              reinterpret_cast<float*>(p.out)[o] = y;
            else
              reinterpret_cast<uint16_t*>(p.out)[o] = (uint16_t)bf16_rne(y);
          }
        }
      }
    }
  }
}

int uwc_noisy_gemm256(const int8_t* A, const int8_t* B, int m, int n, int k, int r, const int8_t* corrA,
                      const int8_t* corrB, const int32_t* maxabs, int lmax, const uint32_t* key,
                      const uint32_t* target, uint32_t* wins, int max_wins, const float* a_scale, const float* b_scale,
                      void* out, int out_mode, int flags, uint32_t* tile_dump, int ldc, hipStream_t stream);

int uwc_skinny_gemm(const int8_t* X, const int8_t* W, int m, int n, int k, const float* sx, const float* sw,
                    void* out, int out_mode, hipStream_t stream);
int uwc_plain_cfg_count();
bool uwc_plain_fits(int cfg, int m, int n, int k, int ldc, const void* out, int out_mode, const float* b_scale);
int uwc_gemm_plain(int cfg, const int8_t* A, const int8_t* B, int m, int n, int k, const float* a_scale,
                   const float* b_scale, void* out, int out_mode, int ldc, hipStream_t stream);

template <bool H, bool D>
static void launch_out(int out_mode, dim3 grid, hipStream_t s, const GemmParams& p) {
  switch (out_mode) {
    case OUT_NONE: hipLaunchKernelGGL((noisy_gemm_kernel<H, D, OUT_NONE>), grid, dim3(G_THREADS), 0, s, p); break;
    case OUT_I32: hipLaunchKernelGGL((noisy_gemm_kernel<H, D, OUT_I32>), grid, dim3(G_THREADS), 0, s, p); break;
    case OUT_BF16: hipLaunchKernelGGL((noisy_gemm_kernel<H, D, OUT_BF16>), grid, dim3(G_THREADS), 0, s, p); break;
    default: hipLaunchKernelGGL((noisy_gemm_kernel<H, D, OUT_F32>), grid, dim3(G_THREADS), 0, s, p); break;
  }
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The argument checks of uwc_noisy_gemm (status 0 or UWC_EINVAL with the message set).
static int gemm_check(const int8_t* A, const int8_t* B, int m, int n, int k, int r, const int8_t* corrA,
                      const int8_t* corrB, const int32_t* maxabs, int lmax, const uint32_t* key, const uint32_t* target,
                      uint32_t* wins, int max_wins, const float* a_scale, const float* b_scale, void* out, int out_mode,
                      int flags) {
  const bool hash = flags & FLAG_HASH, denoise = flags & FLAG_DENOISE;
  if (flags & ~(FLAG_HASH | FLAG_DENOISE | FLAG_TILE128 | FLAG_PLAIN | FLAG_PLAIN_MASK) ||
      ((flags & FLAG_PLAIN_MASK) && !(flags & FLAG_PLAIN)))
    return uwc_fail("uwc_noisy_gemm: unknown flags %d", flags);
  if (flags & FLAG_PLAIN) {
    const int cfg = (flags & FLAG_PLAIN_MASK) >> FLAG_PLAIN_SHIFT;
    if (hash || denoise || (flags & FLAG_TILE128))
      return uwc_fail("uwc_noisy_gemm: FLAG_PLAIN is for plain GEMMs without FLAG_TILE128 (flags %d)", flags);
    if (cfg >= uwc_plain_cfg_count()) return uwc_fail("uwc_noisy_gemm: plain configuration %d unknown", cfg);
    if (!uwc_plain_fits(cfg, m, n, k, n, out, out_mode, b_scale))
      return uwc_fail("uwc_noisy_gemm: plain configuration %d does not take m=%d n=%d k=%d", cfg, m, n, k);
  }
  if (!A || !B || m <= 0 || n <= 0 || k <= 0) return uwc_fail("uwc_noisy_gemm: empty or null operands (m=%d n=%d k=%d)", m, n, k);
  if (k % G_BK) return uwc_fail("uwc_noisy_gemm: k=%d must be a multiple of %d", k, G_BK);
  if (!aligned16(A) || !aligned16(B)) return uwc_fail("uwc_noisy_gemm: A and B must be 16-byte aligned");
  if (out_mode < OUT_NONE || out_mode > OUT_F32) return uwc_fail("uwc_noisy_gemm: unknown out_mode %d", out_mode);
  if (out_mode != OUT_NONE && !out) return uwc_fail("uwc_noisy_gemm: out is null for out_mode %d", out_mode);
  if ((out_mode == OUT_BF16 || out_mode == OUT_F32) && (!a_scale || !b_scale))
    return uwc_fail("uwc_noisy_gemm: a_scale and b_scale are required for out_mode %d", out_mode);
  if (hash || denoise) {
    if (m % G_BM || n % G_BN)
      return uwc_fail("uwc_noisy_gemm: mining needs m %% %d == 0 and n %% %d == 0 (m=%d n=%d)", G_BM, G_BN, m, n);
    if (r <= 0 || r % G_BK || k % r || (r & (r - 1)))
      return uwc_fail("uwc_noisy_gemm: r=%d must be a power of two, a multiple of %d and divide k=%d", r, G_BK, k);
  }
  if (hash && (!key || !target)) return uwc_fail("uwc_noisy_gemm: FLAG_HASH needs key and target");
  if (hash && wins && max_wins < 0) return uwc_fail("uwc_noisy_gemm: max_wins=%d < 0", max_wins);
  if (denoise) {
    if (!corrA || !corrB || !maxabs) return uwc_fail("uwc_noisy_gemm: FLAG_DENOISE needs corrA, corrB and maxabs");
    if (lmax < 1 || lmax > 4) return uwc_fail("uwc_noisy_gemm: lmax=%d outside 1..4", lmax);
    if (!aligned16(corrA) || !aligned16(corrB)) return uwc_fail("uwc_noisy_gemm: corrA/corrB must be 16-byte aligned");
  }
  return 0;
}

extern "C" int uwc_noisy_gemm(const int8_t* A, const int8_t* B, int m, int n, int k, int r, const int8_t* corrA,
                              const int8_t* corrB, const int32_t* maxabs, int lmax, const uint32_t* key,
                              const uint32_t* target, uint32_t* wins, int max_wins, const float* a_scale,
                              const float* b_scale, void* out, int out_mode, int flags, uint32_t* tile_dump,
                              hipStream_t stream) {
  if (int st = gemm_check(A, B, m, n, k, r, corrA, corrB, maxabs, lmax, key, target, wins, max_wins, a_scale, b_scale,
                          out, out_mode, flags))
    return st;
  const bool hash = flags & FLAG_HASH, denoise = flags & FLAG_DENOISE;
  const bool plain = !hash && !denoise;
  if (flags & FLAG_PLAIN)  // checked: a plain GEMM the forced configuration takes
    return uwc_gemm_plain((flags & FLAG_PLAIN_MASK) >> FLAG_PLAIN_SHIFT, A, B, m, n, k, a_scale, b_scale, out,
                          out_mode, n, stream);
  if (plain && m <= 64 && out_mode != OUT_NONE && !(flags & FLAG_TILE128))
    return uwc_skinny_gemm(A, B, m, n, k, a_scale, b_scale, out, out_mode, stream);
  // 256 x 256 tiles when hashing (one tiling per nonce shape), or for a plain GEMM when they keep
  // the CUs busy: at least one tile per CU and the last round of tiles at least 90% full (2048 x
  // 12288 gives 384 tiles on 256 CUs, a half-empty second round, and runs faster on the plain
  // kernel's 128 x 128 tiles).
  const int cus = uwc_cu_count();
  const long t256 = (long)(m / 256) * (n / 256), rounds256 = (t256 + cus - 1) / cus;
  const bool fills = t256 >= cus && t256 * 10 >= rounds256 * cus * 9;
  // the 256 x 256 DMA adds 32-bit lane offsets (255 k + 112) and its row stores 32-bit offsets
  // (31 ldc elements of 4 bytes): k and the output row stride stay below 2^24
  const bool k256 = k % 128 == 0 && k <= (1 << 24) && n <= (1 << 24);
  // the 256 x 256 epilogue writes 16-byte (8-byte for bf16) row segments: rows must start aligned
  const bool vec_out = out_mode == OUT_NONE || (aligned16(out) && n % 4 == 0);
  if (m % 256 == 0 && n % 256 == 0 && k256 && vec_out && !(flags & FLAG_TILE128) && (!plain || fills))
    return uwc_noisy_gemm256(A, B, m, n, k, r, corrA, corrB, maxabs, lmax, key, target, wins, max_wins, a_scale,
                             b_scale, out, out_mode, flags & ~FLAG_TILE128, tile_dump, n, stream);
  // A plain GEMM whose n is not a multiple of 256 (e.g. a vocabulary of 151936) but whose 256 x 256
  // tiles would fill the CUs: columns [0, n256) on 256 x 256 tiles, the last n - n256 on 128 x 128
  // tiles writing into the same rows (integer sums: the split cannot change a value).
  const int n256 = n / 256 * 256;
  if (plain && m % 256 == 0 && k256 && vec_out && n256 > 0 && n256 < n && !(flags & FLAG_TILE128) &&
      (long)(m / 256) * (n256 / 256) >= 256) {
    const int st = uwc_noisy_gemm256(A, B, m, n256, k, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0,
                                     a_scale, b_scale, out, out_mode, 0, nullptr, n, stream);
    if (st || out_mode == OUT_NONE) return st;
    const size_t es = out_mode == OUT_BF16 ? 2 : 4;
    GemmParams q{A, B + (long)n256 * k, m, n - n256, k, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0,
                 a_scale, b_scale ? b_scale + n256 : nullptr, static_cast<char*>(out) + n256 * es, nullptr, n};
    const dim3 g2(((m + G_BM - 1) / G_BM) * ((n - n256 + G_BN - 1) / G_BN));
    launch_out<false, false>(out_mode, g2, stream, q);
    return uwc_launch_status("noisy_gemm (column tail)");
  }
  // Any other plain GEMM of whole 128 x 128 tiles: the DMA-pipelined plain kernel with each
  // step's DMA spread over the next step's passes; a 4-step ring (one workgroup per CU) when there
  // is at most one tile per CU, else a 2-step ring (two workgroups per CU). Measured at the
  // Qwen3-1.7B layer linears (M = 2048): the first for o and down, the second for qkv and gate_up.
  if (plain && !(flags & FLAG_TILE128)) {
    const int cfg = (long)(m / 128) * (n / 128) <= cus ? 4 : 6;
    if (uwc_plain_fits(cfg, m, n, k, n, out, out_mode, b_scale))
      return uwc_gemm_plain(cfg, A, B, m, n, k, a_scale, b_scale, out, out_mode, n, stream);
  }
  GemmParams p{A, B, m, n, k, r, corrA, corrB, maxabs, lmax, key, target, wins, max_wins, a_scale, b_scale, out,
               hash ? tile_dump : nullptr, n};
  const dim3 grid(((m + G_BM - 1) / G_BM) * ((n + G_BN - 1) / G_BN));
  if (hash && denoise) launch_out<true, true>(out_mode, grid, stream, p);
  else if (hash) launch_out<true, false>(out_mode, grid, stream, p);
  else if (denoise) launch_out<false, true>(out_mode, grid, stream, p);
  else launch_out<false, false>(out_mode, grid, stream, p);
  return uwc_launch_status("noisy_gemm");
}

extern "C" int uwc_igemm_i32(const int8_t* A, const int8_t* B, int m, int n, int k, int32_t* C, hipStream_t stream) {
  return uwc_noisy_gemm(A, B, m, n, k, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr,
                        nullptr, C, OUT_I32, 0, nullptr, stream);
}

extern "C" int uwc_igemm_dequant_f32(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx,
                                     const float* sw, float* Y, hipStream_t stream) {
  return uwc_noisy_gemm(A, B, m, n, k, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, sx, sw, Y,
                        OUT_F32, 0, nullptr, stream);
}

int uwc_gemm256_residual(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx, const float* sw,
                         const float* x, float* Y, hipStream_t stream);
extern "C" int uwc_dequant_residual(const void* acc, const float* s, const float* sw, const float* x, int rows, int n,
                                    float* out, hipStream_t stream);

extern "C" int uwc_igemm_dequant_residual_f32(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx,
                                              const float* sw, const float* x, float* Y, hipStream_t stream) {
  const char* fn = "uwc_igemm_dequant_residual_f32";
  if (!x || !Y) return uwc_fail("%s: null x or Y", fn);
  if (int st = gemm_check(A, B, m, n, k, 0, nullptr, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, sx, sw, Y,
                          OUT_F32, 0))
    return st;
  const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)Y, bytes = (uintptr_t)m * (uintptr_t)n * 4;
  if (xa < ya + bytes && ya < xa + bytes) return uwc_fail("%s: Y overlaps x", fn);
  // the shapes uwc_noisy_gemm puts on 256 x 256 tiles with one workgroup per tile (at least one
  // tile per CU, the last round at least 90% full); their epilogue adds the residual
  const int cus = uwc_cu_count();
  const long t256 = (long)(m / 256) * (n / 256), rounds256 = (t256 + cus - 1) / cus;
  const bool fills = t256 >= cus && t256 * 10 >= rounds256 * cus * 9;
  const bool k256 = k % 128 == 0 && k <= (1 << 24) && n <= (1 << 24);
  if (m % 256 == 0 && n % 256 == 0 && k256 && fills && aligned16(Y) && aligned16(x) && n % 4 == 0)
    return uwc_gemm256_residual(A, B, m, n, k, sx, sw, x, Y, stream);
  // elsewhere: the dequantized product, then Y = fadd(x, Y) in place (each element read, then written)
  if (int st = uwc_igemm_dequant_f32(A, B, m, n, k, sx, sw, Y, stream)) return st;
  return uwc_dequant_residual(Y, nullptr, nullptr, x, m, n, Y, stream);
}

int uwc_noisy_gemm256_many(int count, const int8_t* const* A, const int8_t* B, int m, int n, int k, int r,
                           const int8_t* const* corrA, const int8_t* const* corrB, const int32_t* const* maxabs,
                           int lmax, const uint32_t* const* key, const uint32_t* target, uint32_t* const* wins,
                           int max_wins, void* const* out, uint32_t* const* tile_dump, hipStream_t stream);

#define GEMM_MANY_MAX 32  // items per split launch (the kernel's item table)

extern "C" int uwc_noisy_gemm_many(int count, const int8_t* const* A, const int8_t* B, int m, int n, int k, int r,
                                   const int8_t* const* corrA, const int8_t* const* corrB,
                                   const int32_t* const* maxabs, int lmax, const uint32_t* const* key,
                                   const uint32_t* target, uint32_t* const* wins, int max_wins, const float* a_scale,
                                   const float* b_scale, void* const* out, int out_mode, int flags,
                                   uint32_t* const* tile_dump, hipStream_t stream) {
  if (count < 0 || (count > 0 && (!A || !out))) return uwc_fail("uwc_noisy_gemm_many: count=%d or null A / out arrays", count);
  const bool hash = flags & FLAG_HASH, denoise = flags & FLAG_DENOISE;
  if ((hash && !key) || (denoise && (!corrA || !corrB || !maxabs)))
    return uwc_fail("uwc_noisy_gemm_many: the flags need key / corrA, corrB, maxabs arrays");
  bool split = count >= 2 && hash && denoise && out_mode == OUT_I32 && !(flags & FLAG_TILE128) && m % 256 == 0 &&
               n % 256 == 0 && k % 128 == 0 && k <= (1 << 24) && n <= (1 << 24);
  for (int i = 0; i < count; i++) {
    if (int st = gemm_check(A[i], B, m, n, k, r, denoise ? corrA[i] : nullptr, denoise ? corrB[i] : nullptr,
                            denoise ? maxabs[i] : nullptr, lmax, hash ? key[i] : nullptr, target,
                            wins ? wins[i] : nullptr, max_wins, a_scale, b_scale, out[i], out_mode, flags))
      return st;
    split = split && aligned16(out[i]);
  }
  if (!split) {  // one launch per item
    for (int i = 0; i < count; i++)
      if (int st = uwc_noisy_gemm(A[i], B, m, n, k, r, denoise ? corrA[i] : nullptr, denoise ? corrB[i] : nullptr,
                                  denoise ? maxabs[i] : nullptr, lmax, hash ? key[i] : nullptr, target,
                                  wins ? wins[i] : nullptr, max_wins, a_scale, b_scale, out[i], out_mode, flags,
                                  tile_dump ? tile_dump[i] : nullptr, stream))
        return st;
    return 0;
  }
  uint32_t* no_wins[GEMM_MANY_MAX] = {};
  for (int i0 = 0; i0 < count; i0 += GEMM_MANY_MAX) {
    const int c = count - i0 < GEMM_MANY_MAX ? count - i0 : GEMM_MANY_MAX;
    if (int st = uwc_noisy_gemm256_many(c, A + i0, B, m, n, k, r, corrA + i0, corrB + i0, maxabs + i0, lmax, key + i0,
                                        target, wins ? wins + i0 : no_wins, max_wins, out + i0,
                                        tile_dump ? tile_dump + i0 : nullptr, stream))
      return st;
  }
  return 0;
}
