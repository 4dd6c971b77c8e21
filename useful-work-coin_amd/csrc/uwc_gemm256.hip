// gfx950 noisy GEMM, large-tile variant for m % 256 == 0 and n % 256 == 0: the same contract
// as noisy_gemm_kernel (uwc_gemm.hip; miner/ampere/uwc_ampere/kernels.cu:482-715), built for
// throughput at the mining and detrt-prefill shapes.
//
//   * Workgroup tile 256 x 256, k step W_BK (128), 8 wave64s in 2 (M) x 4 (N); each wave owns
//     128 x 64 = two consensus 64 x 64 hash blocks, as 4 x 2 v_mfma_i32_32x32x32_i8 blocks
//     (128 int32 accumulators per lane, in VGPRs so the fold reads them directly).
//   * Operand tiles go HBM -> LDS with global_load_lds_dwordx4 (no VGPR staging) into a ring of
//     W_STAGES k steps (128 KiB): the ring's A tiles, then its B tiles, so that every fragment
//     read is a per-lane base register plus an immediate offset. One barrier per k step. The
//     main-loop DMA uses the scalar-base form: the tile window's address stays in SGPRs and each
//     lane adds a fixed 32-bit offset, so a k step costs no vector address arithmetic. A step's
//     refill goes out in three parts (W_DMA_SPREAD) so that the waves' MFMA issue is not stuck
//     behind a burst of DMA instructions.
//   * Software pipeline at k32-pass granularity: the six LDS fragments of pass p + 1 are read
//     while the eight MFMAs of pass p run (two fragment sets in registers). The step barrier and
//     the next DMA issue sit before the MFMAs of a step's last pass, whose fragments are already
//     in registers, so the barrier wait overlaps MFMA work.
//   * LDS rows are W_BK bytes; the 16-byte chunk c of row r sits at chunk c ^ swz(r), so the
//     32-row fragment reads are conflict-free with 32 or 64 banks. The swizzle is applied on the
//     global side (each lane of a DMA writes a fixed LDS slot and fetches the bytes that belong
//     there).
//   * Transposed C: the B fragment is the MFMA's A operand, so lane l holds row l & 31 of a
//     block and four consecutive columns per register group (16-byte epilogue stores, with the
//     non-temporal hint: the output is written once and would otherwise evict the A and B panels
//     the XCD's other tiles read from L2; 77.5 -> 76.9 us per nonce in the batched mining launch).
//   * Transcript fold every r along k: a lane XORs its accumulators into 4 partials (hash block
//     x bit 0 of the tile index) with 3-input v_bitop3 XORs, spread over a chunk's last pass
//     (blocks folded three MFMAs after their last MFMA of the chunk) and the next chunk's first
//     pass (the rest, before their first MFMA), then a reduce-scatter over lane bits 3 (DPP
//     row_ror:8 fused into v_xor) and 4 (v_permlane16_swap) leaves every lane with the full tile
//     XOR of exactly one tile, which it folds into that tile's 16-word message (message slots
//     are static: the chunk loop is unrolled over the 16 slots). After the k loop every lane
//     digests its own tile.
//   * Denoise in four passes over quarters of the wave's block (a 32-register Horner
//     accumulator), the corrections streamed through the same ring (or, when they fit, loaded
//     into it before the digest). The split kernel, when the corrections fill the ring exactly,
//     goes stage by stage instead (each stage's product shifted by its limb), so that stage 0 is
//     free for the next nonce's first k step while stage 1's MFMAs and the output hand-off run.
//   * SPLIT (the batched form): several nonces per launch on the same tiles; waves 0-3 issue the
//     DMA, waves 4-7 store every output (the others' through an LDS hand-off), so one nonce's
//     stores drain while the next computes (see the kernel).
#include "uwc_common.h"

// lambdas are always inlined: an out-of-line call would take the accumulator arrays' addresses
// (private memory) and load captured uniform values per lane
#define UWC_AI __attribute__((always_inline))
#define W_BM 256
#define W_BN 256
#ifndef W_BK
#define W_BK 128
#endif
#ifndef W_MULTI
#define W_MULTI 2  // plain int32 GEMMs of >= W_MULTI tiles per CU take the persistent multi-tile form
#endif
#ifndef W_STAGES
#define W_STAGES (W_BK == 64 ? 4 : 2)
#endif
#define W_CH (W_BK / 16)                    // 16-byte chunks per LDS row
#define W_KP (W_BK / 32)                    // k32 MFMA passes per k step
#define W_THREADS 512
#define W_TILE (W_BM * W_BK)                 // bytes of one operand tile
#define W_BOFF (W_STAGES * W_TILE)           // LDS byte offset of the ring's B tiles
#define W_LDS (2 * W_STAGES * W_TILE)        // the ring
#define W_LDS_HANDOFF (W_THREADS / 128 * 8192)  // the split kernels' hand-off slots (a quarter per loader)
static_assert(W_LDS + W_LDS_HANDOFF <= 160 * 1024, "LDS exceeds 160 KiB (gfx950 LDS per workgroup)");
#define W_WAVES (W_THREADS / 64)
#define W_SEGS_PER_WAVE (W_TILE / 1024 / W_WAVES)  // 1 KiB DMA segments per wave per operand per k step
#ifndef W_DB_PLAIN
#define W_DB_PLAIN 1  // two alternating fragment sets in the kernels without a transcript
#endif
#ifndef W_DMA_SPREAD
// Issue a k step's refill in three parts (after the barrier, before pass 0 and before pass 1 of
// the next step) instead of one burst: 64 DMA instructions per CU in one burst keep every wave
// blocked on the address unit, and its MFMAs queued behind them, for ~1600 cycles
#define W_DMA_SPREAD 1
#endif

#define FLAG_HASH 1
#define FLAG_DENOISE 2
#define OUT_NONE 0
#define OUT_I32 1
#define OUT_BF16 2
#define OUT_F32 3
#define OUT_F32R 4  // OUT_F32 plus an fp32 residual of the same layout (plain GEMMs only)
#define WIN_WORDS 10
#define DUMP_WORDS 24

// One item of a launch: a nonce's operand, corrections, seed, win records and output. Every item
// shares B, the shape, the target and the scales; a launch runs its items one after another on
// the same tiles.
#define G256_MAXB 32
struct Gemm256Item {
  const i8* A;
  const i8* corrA;
  const i8* corrB;
  const i32* maxabs;
  const u32* key;
  u32* wins;
  void* out;
  u32* dump;  // optional tile dump (messages and digests), NULL to skip
};

struct Gemm256Params {
  const i8* B;
  int m, n, k, r;
  int lmax;
  const u32* target;
  int max_wins;
  const float* a_scale;
  const float* b_scale;
  const float* res;  // OUT_F32R: the residual rows, row stride ldc
  int ldc;  // output row stride in elements
  int count;
  int tiles;  // > 0: the plain multi-tile form (item i is tile blockIdx.x + i * gridDim.x of it[0])
  Gemm256Item it[G256_MAXB];
};

// f(std::integral_constant<int, i>) for i = 0 .. N - 1, each i a compile-time constant.
template <int I, int N, class F>
__device__ __forceinline__ void static_for_(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for_<I + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_<0, N>(f);
}

// A word the launch only reads, written by an earlier launch (seeds, targets, maxabs), loaded
// through the constant address space: a scalar load, counted in lgkmcnt. A vector load would
// make the compiler wait on vmcnt, which in a split kernel's storer wave also counts the output
// stores still draining.
template <class T>
__device__ __forceinline__ T ld_uniform(const T* ptr, int i) {
  return ((const __attribute__((address_space(4))) T*)(uintptr_t)ptr)[i];
}

typedef const void __attribute__((address_space(1)))* gptr_t;
typedef void __attribute__((address_space(3)))* lptr_t;

// LDS tile rows are W_BK bytes; 16-byte chunk c of tile row r sits at chunk c ^ swz(r):
//   64-byte rows  (4 chunks): swz(r) = ((r >> 1) ^ (r >> 2)) & 3
//   128-byte rows (8 chunks): swz(r) = (r ^ (r >> 3)) & 7
// Either way 16 consecutive rows read at one logical chunk hit 16 distinct 16-byte bank groups
// (64 banks) and any 8 consecutive rows hit 8 distinct ones (32 banks).
__device__ __forceinline__ int swz(int r) {
  if constexpr (W_BK == 64) return ((r >> 1) ^ (r >> 2)) & 3;
  else return (r ^ (r >> 3)) & 7;
}

// A 1 KiB DMA segment holds 1024 / W_BK tile rows; lane i fills LDS bytes [16 i, 16 i + 16) of
// it: row RPS s + i / W_CH (RPS = rows per segment), physical chunk i % W_CH, so it fetches
// logical chunk (i % W_CH) ^ swz(row).
#define W_RPS (1024 / W_BK)

struct DmaLane {
  const i8* a;  // A + (bm0 + i / W_CH) * lda
  const i8* b;
  int rin, phys;
};

__device__ __forceinline__ DmaLane dma_lane(const i8* A, long lda, const i8* B, long ldb, int bm0, int bn0, int lane) {
  const int rin = lane / W_CH, phys = lane % W_CH;
  return DmaLane{A + (long)(bm0 + rin) * lda, B + (long)(bn0 + rin) * ldb, rin, phys};
}

// One wave-wide 16-byte-per-lane DMA: lane i's 16 bytes at g land at LDS byte lds + 16 i
// (lds is wave-uniform and goes in M0). Written as asm rather than the global_load_lds builtin
// so that the compiler's wait-count model does not see an LDS write in flight: with one pending
// it waits for every outstanding LDS read (lgkmcnt(0)) before each use of a fragment, instead
// of only for the reads that use needs. The kernel tracks these loads itself: wait_step waits
// on vmcnt and barriers before any stage is read, and the loads issue only after the barrier
// that ends every read of the stage they fill.
__device__ __forceinline__ void dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ u32 lds_addr(const u8* p) { return (u32)(uintptr_t)(lptr_t)p; }

// Issue this wave's DMA segments of one k step (segments SPL wave .. SPL wave + SPL - 1 of A and
// of B) into the LDS tiles at byte addresses lds_a, lds_b (wave-uniform).
template <int SPL>
__device__ __forceinline__ void dma_step(u32 lds_a, u32 lds_b, const DmaLane& d, long lda, long ldb, long k0, int wave) {
#pragma unroll
  for (int t = 0; t < SPL; t++) {
    const int s = SPL * wave + t;
    const int c = d.phys ^ swz(W_RPS * s + d.rin);
    const long off = (long)W_RPS * s;
    dma16(d.a + off * lda + k0 + c * 16, __builtin_amdgcn_readfirstlane(lds_a + s * 1024));
    dma16(d.b + off * ldb + k0 + c * 16, __builtin_amdgcn_readfirstlane(lds_b + s * 1024));
  }
}

// dma16 with a wave-uniform 64-bit base in SGPRs plus a 32-bit lane offset.
__device__ __forceinline__ void dma16s(u32 voff, const void* sbase, u32 lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}

// Lane byte offsets of the main loop's DMA segments within a 256-row window of a k-contiguous
// operand with row stride k (the same for A and B): segment s = SPL wave + t, tile row
// RPS s + i / W_CH, physical chunk i % W_CH = logical chunk (i % W_CH) ^ swz(row). SPL is the
// number of 1 KiB segments per loading wave per operand and k step: W_SEGS_PER_WAVE when every
// wave loads, twice that when only half of them do.
template <int SPL>
struct DmaOff {
  u32 v[SPL];
};

template <int SPL>
__device__ __forceinline__ DmaOff<SPL> dma_offsets(long k, int wave, int lane) {
  DmaOff<SPL> d;
  const int rin = lane / W_CH, phys = lane % W_CH;
#pragma unroll
  for (int t = 0; t < SPL; t++) {
    const int row = W_RPS * (SPL * wave + t) + rin;
    d.v[t] = (u32)((long)row * k + ((phys ^ swz(row)) << 4));
  }
  return d;
}

// Segments [T0, T1) of one k step of the main loop's DMA: a_win = A + bm0 k + k0 and
// b_win = B + bn0 k + k0 are wave-uniform (SGPRs).
template <int SPL, int T0, int T1>
__device__ __forceinline__ void dma_step_s(u32 lds_a, u32 lds_b, const DmaOff<SPL>& d, const i8* a_win, const i8* b_win,
                                           int wave) {
#pragma unroll
  for (int t = T0; t < T1; t++) {
    const u32 so = (u32)(SPL * wave + t) * 1024u;
    dma16s(d.v[t], a_win, lds_a + so);
    dma16s(d.v[t], b_win, lds_b + so);
  }
}

// Wait until at most `younger` of this wave's k steps are still loading (a loading wave, vm), then
// barrier. A wave that issues no DMA only takes the barrier: its vmcnt counts nothing but its
// own output stores, which it never needs to wait for.
template <int SPL>
__device__ __forceinline__ void wait_step(int younger, bool vm) {
  constexpr int per = 2 * SPL;  // DMA instructions per loading wave per k step
  static_assert((W_STAGES - 1) * per < 64, "vmcnt is 6 bits");
  if (vm) {
    if (younger >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * per) : "memory");
    else if (younger == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * per) : "memory");
    else if (younger == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(per) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ v4i lds16(const u8* p) { return *reinterpret_cast<const v4i*>(p); }

// Per-lane fragment offset within a tile for k32 pass kp and block parity par (the 32-row
// block index mb & 1 reaches swz through row bit 5 when rows are 128 bytes): row (lane & 31)
// of the block, logical chunk 2 kp + (lane >> 5).
__device__ __forceinline__ int frag_off(int lane, int kp, int par) {
  const int r = lane & 31, c = 2 * kp + (lane >> 5);
  return r * W_BK + ((c ^ swz(r + 32 * par)) << 4);
}

// One lane's LDS byte addresses of its fragment reads for the k32 passes of a step, in stage 0,
// for the wave's first 32-row (A) and 32-column (B) block. Stage st and block j add the
// immediate st W_TILE + 32 j W_BK. Even blocks use entry kp; odd blocks (row bit 5 set) use
// kp ^ 2 with 128-byte rows (swz then flips chunk bit 2) and kp with 64-byte rows (swz does not
// see row bit 5).
struct FragBase {
  u32 a[W_KP], b[W_KP];
};

__device__ __forceinline__ int par_kp(int kp, int par) {
  if constexpr (W_BK == 128) return par ? kp ^ 2 : kp;
  else return kp;
}

__device__ __forceinline__ FragBase frag_bases(u32 wsm_lds, int wm, int wn, int lane) {
  FragBase f;
#pragma unroll
  for (int kp = 0; kp < W_KP; kp++) {
    const u32 o = (u32)frag_off(lane, kp, 0);
    f.a[kp] = wsm_lds + (u32)(wm * 128 * W_BK) + o;
    f.b[kp] = wsm_lds + (u32)(W_BOFF + wn * 64 * W_BK) + o;
  }
  return f;
}

// The operand fragments of one k32 pass of the wave's 128 x 64 block.
struct Frag {
  v4i a[4], b[2];
};

typedef const v4i __attribute__((address_space(3)))* lds_v4i_t;
__device__ __forceinline__ v4i lds_at(u32 a) { return *(lds_v4i_t)(uintptr_t)a; }

__device__ __forceinline__ v4i frag_a(const FragBase& fb, int st, int kp, int mb) {
  return lds_at(fb.a[par_kp(kp, mb & 1)] + (u32)(st * W_TILE + mb * 32 * W_BK));
}
__device__ __forceinline__ v4i frag_b(const FragBase& fb, int st, int kp, int nb) {
  return lds_at(fb.b[par_kp(kp, nb & 1)] + (u32)(st * W_TILE + nb * 32 * W_BK));
}

__device__ __forceinline__ void frag_read(Frag& f, const FragBase& fb, int st, int kp) {
#pragma unroll
  for (int nb = 0; nb < 2; nb++) f.b[nb] = frag_b(fb, st, kp, nb);
#pragma unroll
  for (int mb = 0; mb < 4; mb++) f.a[mb] = frag_a(fb, st, kp, mb);
}

__device__ __forceinline__ u32 xor3(u32 a, u32 b, u32 c) { return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96); }

// XOR one 32 x 32 block's 16 accumulators into the lane's 2 partials of its hash block (the
// transposed C layout: lane l holds row l & 31 and, in register e, column 8 (e >> 2) + 4 (l >> 5)
// + (e & 3), so bit 1 of e is bit 0 of the tile index t): x[0] collects e & 2 == 0, x[1] the rest.
__device__ __forceinline__ void fold_block(const v16i& v, u32* x, bool first) {
  if (first) {
    x[0] = xor3(xor3(xor3(v[0], v[1], v[4]), v[5], v[8]), v[9], v[12]) ^ (u32)v[13];
    x[1] = xor3(xor3(xor3(v[2], v[3], v[6]), v[7], v[10]), v[11], v[14]) ^ (u32)v[15];
  } else {
    x[0] = xor3(xor3(xor3(xor3(x[0], v[0], v[1]), v[4], v[5]), v[8], v[9]), v[12], v[13]);
    x[1] = xor3(xor3(xor3(xor3(x[1], v[2], v[3]), v[6], v[7]), v[10], v[11]), v[14], v[15]);
  }
}

// The eight MFMAs of one pass, column half 0 first: block position pos = 4 nb + mb. With READ,
// f is refilled with the fragments of pass nkp of stage nst as the current ones retire: b[0]
// after the four half-0 MFMAs, a[mb] after MFMA (mb, 1), b[1] last; one fragment set stays in
// registers and each read still has several MFMAs to land before its first use in the next pass.
//
// The transcript fold of a chunk is spread over two passes so that neither carries all of its
// VALU work: in the chunk's last pass (TAIL) block pos - FOLD_LAG is XORed into the partials x
// right after MFMA pos (its accumulators became final FOLD_LAG MFMAs earlier), which covers
// blocks 0 .. 7 - FOLD_LAG; in the next chunk's first pass (HEAD) blocks 8 - FOLD_LAG .. 7 are
// XORed right before their first MFMA of the new chunk. Partials x[0..1] collect mb 0, 1 (hash
// block 0) and x[2..3] mb 2, 3; blocks 0 and 2 (the first of each in TAIL order) initialise them.
#define FOLD_LAG 3
template <bool HEAD, bool TAIL, bool READ>
__device__ __forceinline__ void pass_mma(v16i acc[4][2], Frag& f, u32 x[4], const FragBase& fb, int nst, int nkp) {
#pragma unroll
  for (int pos = 0; pos < 8; pos++) {
    const int mb = pos & 3, nb = pos >> 2;
    if (HEAD && pos >= 8 - FOLD_LAG) fold_block(acc[mb][nb], x + (mb >> 1) * 2, false);
    acc[mb][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[nb], f.a[mb], acc[mb][nb], 0, 0, 0);
    if (TAIL && pos >= FOLD_LAG) {
      const int q = pos - FOLD_LAG, qm = q & 3, qn = q >> 2;
      fold_block(acc[qm][qn], x + (qm >> 1) * 2, q == 0 || q == 2);
    }
    if (READ && pos == 3) f.b[0] = frag_b(fb, nst, nkp, 0);
    if (READ && pos >= 4) f.a[pos - 4] = frag_a(fb, nst, nkp, pos - 4);
  }
  if constexpr (READ) f.b[1] = frag_b(fb, nst, nkp, 1);
  // pin the interleave: [fold VALU,] MFMA [, fold VALU] [, read] per block position
#pragma unroll
  for (int pos = 0; pos < 8; pos++) {
    if (HEAD && pos >= 8 - FOLD_LAG) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    if (TAIL && pos >= FOLD_LAG) __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
    if (READ && pos >= 3) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
  }
  if constexpr (READ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
}

// The HEAD part of the fold without MFMAs: blocks 8 - FOLD_LAG .. 7 into x (after the k loop,
// for the last chunk, whose TAIL pass already folded the other blocks).
__device__ __forceinline__ void fold_head(const v16i acc[4][2], u32 x[4]) {
  static_for<FOLD_LAG>([&](auto ic) UWC_AI {
    constexpr int pos = 8 - FOLD_LAG + decltype(ic)::value, mb = pos & 3, nb = pos >> 2;
    fold_block(acc[mb][nb], x + (mb >> 1) * 2, false);
  });
}

// Double-buffered form of pass_mma for the kernels without a transcript: with READ, the six
// fragments of pass nkp go into nxt before the MFMAs on cur, so they have the whole pass to
// land. Costs a second fragment set (24 VGPRs).
template <bool READ>
__device__ __forceinline__ void pass_mma_db(v16i acc[4][2], const Frag& cur, Frag& nxt, const FragBase& fb, int nst,
                                            int nkp) {
  if constexpr (READ) frag_read(nxt, fb, nst, nkp);
#pragma unroll
  for (int mb = 0; mb < 4; mb++)
#pragma unroll
    for (int nb = 0; nb < 2; nb++)
      acc[mb][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.b[nb], cur.a[mb], acc[mb][nb], 0, 0, 0);
  if constexpr (READ) __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
  for (int i = 0; i < 8; i++) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
}

// Denoise k step for one quarter of the wave's block: M blocks 2h, 2h+1 of column half nb.
// The fragments of two passes are requested before their MFMAs, so each MFMA waits only for
// its own reads and the second pass's reads overlap the first pass's MFMAs.
__device__ __forceinline__ void step_mma_quarter(v16i tmp[2], const FragBase& fb, int st, int h, int nb) {
#pragma unroll
  for (int k2 = 0; k2 < W_KP; k2 += 2) {
    v4i a0[2], a1[2], b[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      b[j] = frag_b(fb, st, k2 + j, nb);
      a0[j] = frag_a(fb, st, k2 + j, 2 * h);
      a1[j] = frag_a(fb, st, k2 + j, 2 * h + 1);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      tmp[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[j], a0[j], tmp[0], 0, 0, 0);
      tmp[1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[j], a1[j], tmp[1], 0, 0, 0);
    }
  }
}

// a -= t << sh element by element (a vector shift by a scalar count would splat the count into
// a vector of registers), pinned where it stands: otherwise the subtraction is sunk to a's next
// use and t's registers stay live until then
__device__ __forceinline__ void sub_shl(v16i& a, const v16i& t, int sh) {
#pragma unroll
  for (int e = 0; e < 16; e++) {
    int x = a[e] - (t[e] << sh);
    asm volatile("" : "+v"(x));
    a[e] = x;
  }
}

__device__ __forceinline__ u32 rotl13(u32 x) { return __builtin_amdgcn_alignbit(x, x, 19); }

// Lane-permuted copy of x (DPP control CTRL). bound_ctrl with a zero old value lets the compiler
// fuse the permutation into the consuming v_xor as a DPP operand (every source lane is in range
// for the two controls used here, so the result is the plain permutation).
template <int CTRL>
__device__ __forceinline__ u32 dpp(u32 x) {
  return (u32)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF, true);
}

// Reduce-scatter of the 4 fold partials x[2 hm + tb] over lane bits 3, 4 (the lanes holding
// rows g + 8 i of one tile differ only there): afterwards the XOR of the one tile this lane owns,
// hash block hm = lane bit 3 and t bit 0 = lane bit 4, is keep ^ other.
__device__ __forceinline__ void fold_scatter(const u32 x[4], int lane, u32& keep, u32& other) {
  const bool b3 = (lane >> 3) & 1;
  u32 y[2];
#pragma unroll
  for (int tb = 0; tb < 2; tb++) {  // lane bit 3: keep hash block b3
    const u32 kp = b3 ? x[2 + tb] : x[tb], send = b3 ? x[tb] : x[2 + tb];
    y[tb] = kp ^ dpp<0x128>(send);  // row_ror:8 within a 16-lane row: partner lane ^ 8
  }
  // lane bit 4: v_permlane16_swap exchanges y[0] of the odd 16-lane rows with y[1] of the even
  // rows, so a lane of an even row ends with both partners' y[0] and one of an odd row with both
  // partners' y[1]
  const auto sw = __builtin_amdgcn_permlane16_swap(y[0], y[1], false, false);
  keep = sw[0];
  other = sw[1];
}

// msg = rotl13(msg) ^ (tile XOR), from the partials.
__device__ __forceinline__ void fold_into(u32& msg, const u32 x[4], int lane) {
  u32 keep, other;
  fold_scatter(x, lane, keep, other);
  msg = xor3(rotl13(msg), keep, other);
}

__device__ __forceinline__ u32 bf16_rne(float f) {
  const u32 u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Workgroup id -> tile: XCD-contiguous runs (ids are dispatched round-robin over 8 XCDs),
// rastered in groups of 4 tile rows.
__device__ __forceinline__ void tile256_of(int m, int n, int pid, int& bm0, int& bn0) {
  const int npm = m / W_BM, npn = n / W_BN, total = npm * npn;
  if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
  constexpr int GROUP_M = 4;
  const int grp = GROUP_M * npn, gid = pid / grp, first = gid * GROUP_M;
  const int gsz = min(npm - first, GROUP_M), in = pid - gid * grp;
  bm0 = (first + in % gsz) * W_BM;
  bn0 = (in / gsz) * W_BN;
}
__device__ __forceinline__ void tile256(int m, int n, int& bm0, int& bn0) { tile256_of(m, n, blockIdx.x, bm0, bn0); }

// SPLIT: the launch's items follow each other on the same tiles, and the output stores of item
// i drain while item i + 1 computes. On gfx9 a wave's vmcnt counts its stores as well as its
// loads, so a wave that waits on vmcnt for its LDS DMA cannot leave stores in flight. Waves
// 0 .. 3 (loaders, one per SIMD) therefore issue all the DMA and never store an output; waves
// 4 .. 7 (storers) issue no DMA, never wait on vmcnt, and store their own results and, through
// the idle ring, those of loader wave - 4 (64 sixteen-byte stores per lane and item).
template <bool HASH, bool DENOISE, int OUT, bool SPLIT = false>
__global__ void __launch_bounds__(W_THREADS) noisy_gemm256_kernel(Gemm256Params p) {
  extern __shared__ __attribute__((aligned(1024))) u8 wsm[];
  // the wave index is uniform: readfirstlane keeps everything derived from it scalar
  const int tid = threadIdx.x, lane0 = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  constexpr int SPL = SPLIT ? 2 * W_SEGS_PER_WAVE : W_SEGS_PER_WAVE;  // DMA segments per loading wave
  static_assert(SPL >= 4 && SPL % 4 == 0, "the refill spread takes halves and quarters of a wave's segments");
  const bool is_loader = !SPLIT || wave < W_WAVES / 2;
  int bm0, bn0;
  tile256(p.m, p.n, bm0, bn0);
  const long k = p.k;
  const int KT = p.k / W_BK;
  const u32 wsm_l = __builtin_amdgcn_readfirstlane(lds_addr(wsm));
  auto lds_a = [&](int st) UWC_AI { return wsm_l + (u32)(st * W_TILE); };           // stage st's A tile
  auto lds_b = [&](int st) UWC_AI { return wsm_l + (u32)(W_BOFF + st * W_TILE); };  // and its B tile
  const i8* b_win = p.B + (long)bn0 * k;
  // fragment sets: single set streamed (pass_mma) or two alternating sets (pass_mma_db)
  constexpr bool DB = !HASH && W_DB_PLAIN;
  using NoFold = std::integral_constant<int, 0>;

  // epilogue of one 32 x 32 MFMA block of wave (swm, swn): lane holds row (lane & 31) and, in
  // registers 4 j .. 4 j + 3, columns 8 j + 4 (lane >> 5) .. + 3: one 16-byte (I32, F32) or
  // 8-byte (BF16) store per j at a wave-uniform base plus a 32-bit lane offset. The host routes
  // outputs whose rows are not 16-byte aligned (ldc % 4 != 0) to the 128 x 128 kernel.
  auto store_block = [&](int lane, void* out, int swm, int swn, int mb, int nb, const v16i& v) UWC_AI {
    if constexpr (OUT != OUT_NONE) {
      constexpr int ES = OUT == OUT_BF16 ? 2 : 4;  // output element bytes
      const int row0 = bm0 + swm * 128 + mb * 32, col0 = bn0 + swn * 64 + nb * 32;
      const int lr = lane & 31, lc = 4 * (lane >> 5);
      u8* base = reinterpret_cast<u8*>(out) + ((long)row0 * p.ldc + col0) * ES;
      const u32 loff = (u32)(lr * p.ldc + lc) * ES;
      float asc = 0.f;
      if constexpr (OUT == OUT_BF16 || OUT == OUT_F32 || OUT == OUT_F32R) asc = p.a_scale[row0 + lr];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        u8* dst = base + loff + 8 * j * ES;
        if constexpr (OUT == OUT_I32) {
          uwc_store_nt(dst, v4i{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]});
        } else {
          float y[4];
#pragma unroll
          for (int i = 0; i < 4; i++)
            y[i] = __fmul_rn(__fmul_rn((float)v[4 * j + i], asc), p.b_scale[col0 + 8 * j + lc + i]);
          if constexpr (OUT == OUT_F32) {
            uwc_store_nt(dst, float4{y[0], y[1], y[2], y[3]});
          } else if constexpr (OUT == OUT_F32R) {
            const float4 x = uwc_load_nt(p.res + ((long)(row0 + lr) * p.ldc + col0 + 8 * j + lc));
            uwc_store_nt(dst, float4{__fadd_rn(x.x, y[0]), __fadd_rn(x.y, y[1]), __fadd_rn(x.z, y[2]),
                                     __fadd_rn(x.w, y[3])});
          } else {
            const uint2 w{bf16_rne(y[0]) | (bf16_rne(y[1]) << 16), bf16_rne(y[2]) | (bf16_rne(y[3]) << 16)};
            uwc_store_nt(dst, w);
          }
        }
      }
    }
  };

  // the single-item kernels compile without the item loop; the multi-tile form (plain GEMMs of at
  // least two tiles per workgroup) takes tiles blockIdx.x, blockIdx.x + gridDim.x, ... of one GEMM
  const bool multi = SPLIT && p.tiles > 0;
  const int count = SPLIT ? (multi ? (p.tiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : p.count) : 1;
  // One item, for a wave of role LOADER (a compile-time constant, so that neither role's code
  // carries the other's branches or registers; both take the same barriers in the same order).
  int pre = 0;  // ring stages 0 .. pre - 1 already hold (or are loading) this item's first k steps
  auto run_item = [&](int item, auto role) UWC_AI {
    constexpr bool loader = decltype(role)::value;
    if (multi) {
      tile256_of(p.m, p.n, (int)blockIdx.x + item * (int)gridDim.x, bm0, bn0);
      b_win = p.B + (long)bn0 * k;
    }
    const Gemm256Item& I = p.it[multi ? 0 : item];
    // The lane index through an opaque zero: everything derived from it is recomputed per item
    // instead of being hoisted out of the item loop and kept live across it.
    int z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z));
    const int lane = lane0 + z;
    const FragBase fbase = frag_bases(wsm_l, wm, wn, lane);
    const DmaOff<SPL> doff = dma_offsets<SPL>(k, wave, lane);
    v16i acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 2; j++) acc[i][j] = v16i{};
    const i8* a_win = I.A + (long)bm0 * k;  // + k0: this workgroup's operand windows
    // prologue: every stage of the ring loading (step 0 may already be, issued by the previous
    // item's denoise), then step 0 resident and its first pass read
    if constexpr (loader) {
#pragma unroll
      for (int s = 0; s < W_STAGES; s++)
        if (s < KT && s >= pre)
          dma_step_s<SPL, 0, SPL>(lds_a(s), lds_b(s), doff, a_win + s * W_BK, b_win + s * W_BK, wave);
    }
    pre = 0;
    wait_step<SPL>(min(KT - 1, W_STAGES - 1), loader);
    // transcript fold partials, carried from a chunk's TAIL pass to the next chunk's HEAD pass;
    // zero before chunk 0, so the HEAD pass of the first k step folds nothing into slot 15
    u32 fx[4];
#pragma unroll
    for (int i = 0; i < 4; i++) fx[i] = 0;
    Frag fb[DB ? 2 : 1];
    frag_read(fb[0], fbase, 0, 0);

    // One k step. Pass kp runs its MFMAs on the fragments in `cur` while reading those of pass
    // kp + 1. Before the last pass the wave waits for step kt + 1 (vmcnt + barrier: every wave
    // is then done reading step kt's stage) and the loaders refill that stage with step
    // kt + W_STAGES; the last pass reads the next step's first fragments (on the final step that
    // read of a resident stage is unused, which keeps the MFMA code free of branches). FM bit
    // kp: pass kp is the HEAD pass of a chunk (it finishes the fold of the chunk that ended with
    // the previous pass and folds it into m0 for kp == 0, else m1); FM bit 4 + kp: pass kp is the
    // TAIL pass of a chunk. The stage index ST == kt % W_STAGES is a compile-time constant, so
    // every LDS address of the step is a base register plus an immediate.
    auto step = [&](auto fm, auto stc, int kt, u32& m0, u32& m1) UWC_AI {
      constexpr int FM = decltype(fm)::value, ST = decltype(stc)::value;
      constexpr int H = SPL / 2, Q = SPL / 4;
      static_for<W_KP>([&](auto kpc) UWC_AI {
        constexpr int kp = decltype(kpc)::value;
        constexpr bool head = ((FM >> kp) & 1) != 0, tail = ((FM >> (4 + kp)) & 1) != 0;
        constexpr int nst = kp + 1 == W_KP ? (ST + 1) % W_STAGES : ST;
        constexpr int nkp = kp + 1 == W_KP ? 0 : kp + 1;
#if W_DMA_SPREAD
        // the refill of the previous step's stage, continued: the third quarter of the segments
        // before pass 0, the last quarter before pass 1 (the first half went out after the
        // previous step's barrier)
        if constexpr (kp < 2) {
          if (loader && kt >= 1 && kt - 1 + W_STAGES < KT) {
            constexpr int PST = (ST + W_STAGES - 1) % W_STAGES;
            const long k0 = (long)(kt - 1 + W_STAGES) * W_BK;
            dma_step_s<SPL, H + kp * Q, H + (kp + 1) * Q>(lds_a(PST), lds_b(PST), doff, a_win + k0, b_win + k0, wave);
          }
        }
#endif
        if constexpr (kp + 1 == W_KP) {
          if (kt + 1 < KT) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this stage's reads are complete
            wait_step<SPL>(min(KT - 2 - kt, W_STAGES - 2), loader);
            if (loader && kt + W_STAGES < KT) {
              const long k0 = (long)(kt + W_STAGES) * W_BK;
#if W_DMA_SPREAD
              dma_step_s<SPL, 0, H>(lds_a(ST), lds_b(ST), doff, a_win + k0, b_win + k0, wave);
#else
              dma_step_s<SPL, 0, SPL>(lds_a(ST), lds_b(ST), doff, a_win + k0, b_win + k0, wave);
#endif
            }
          }
        }
        if constexpr (DB) {
          static_assert(FM == 0, "the double-buffered passes carry no transcript fold");
          pass_mma_db<true>(acc, fb[kp & 1], fb[(kp + 1) & 1], fbase, nst, nkp);
        } else {
          pass_mma<head, tail, true>(acc, fb[0], fx, fbase, nst, nkp);
        }
        if constexpr (head) fold_into(kp == 0 ? m0 : m1, fx, lane);
      });
    };
    // step() for a k step whose stage is known only at run time
    auto step_rt = [&](auto fm, int kt, u32& m0, u32& m1) UWC_AI {
      static_for<W_STAGES>([&](auto stc) UWC_AI {
        if (kt % W_STAGES == decltype(stc)::value) step(fm, stc, kt, m0, m1);
      });
    };

    // Denoise setup (kernels.cu:598-673): acc -= sum_li 128^li [X_li | EAL] [EBRt | Y_li]^T, the
    // corr k steps running limb L-1 down to 0, each limb 2r / W_BK steps. CT steps in all.
    int L = 1, CPL = 1, CT = 1;
    long R2 = 0;
    if constexpr (DENOISE) {
      const int mx = max(ld_uniform(I.maxabs, 0), ld_uniform(I.maxabs, 1));
      L = min(mx > 1040319 ? 4 : mx > 8127 ? 3 : mx > 63 ? 2 : 1, p.lmax);
      R2 = 2L * p.r;
      CPL = (int)(R2 / W_BK);
      CT = L * CPL;
    }
    // next corr step to issue: global index ig, limb li, chunk kc
    int ig = 0, li = L - 1, kc = 0;
    auto cissue = [&]() UWC_AI {
      if constexpr (loader) {
        const DmaLane cl =
            dma_lane(I.corrA + (long)li * p.m * R2, R2, I.corrB + (long)li * p.n * R2, R2, bm0, bn0, lane);
        dma_step<SPL>(lds_a(ig % W_STAGES), lds_b(ig % W_STAGES), cl, R2, R2, (long)kc * W_BK, wave);
      }
      ig++;
      if (++kc == CPL) {
        kc = 0;
        li = li == 0 ? L - 1 : li - 1;
      }
    };

    u32 msg[16];
#pragma unroll
    for (int w = 0; w < 16; w++) msg[w] = 0;
    const int nchunks = p.k / p.r;
    if constexpr (HASH) {
      int kt = 0;
      u32 unused = 0;
      // The fold of chunk c ends in the first pass of chunk c + 1 (slot (c - 1) mod 16 for the
      // chunk starting at slot c). For chunk 0 that folds the all-zero partials into the
      // all-zero slot 15, which leaves it zero.
      using Head = std::integral_constant<int, 0x01>;
      using Tail = std::integral_constant<int, 0x80>;
      if (p.r == W_BK) {
        // one k step per chunk: an outer iteration is 16 k steps, so k step c0 + s sits in stage
        // s % W_STAGES
        static_assert(16 % W_STAGES == 0, "stage of an unrolled k step");
        for (int c0 = 0; c0 < nchunks; c0 += 16) {
          static_for<16>([&](auto sc) UWC_AI {
            constexpr int s = decltype(sc)::value;
            if (c0 + s < nchunks)
              step(std::integral_constant<int, 0x81>{}, std::integral_constant<int, s % W_STAGES>{}, c0 + s,
                   msg[(s + 15) & 15], unused);
          });
        }
      } else if (p.r > W_BK) {
        const int tpc = p.r / W_BK;
        for (int c0 = 0; c0 < nchunks; c0 += 16) {
#pragma unroll
          for (int s = 0; s < 16; s++) {
            if (c0 + s < nchunks) {
              step_rt(Head{}, kt++, msg[(s + 15) & 15], unused);
              for (int i = 1; i + 1 < tpc; i++) step_rt(NoFold{}, kt++, unused, unused);
              step_rt(Tail{}, kt++, unused, unused);
            }
          }
        }
      } else if constexpr (W_KP == 4) {
        // r = 64 = W_BK / 2: k step j holds chunks 2j (passes 0, 1) and 2j + 1 (passes 2, 3);
        // an outer iteration is 8 k steps, so k step c0 / 2 + s / 2 sits in stage
        // (s / 2) % W_STAGES
        static_assert(8 % W_STAGES == 0, "stage of an unrolled k step");
        for (int c0 = 0; c0 < nchunks; c0 += 16) {
          static_for<8>([&](auto jc) UWC_AI {
            constexpr int j = decltype(jc)::value, s = 2 * j;
            if (c0 + s < nchunks)
              step(std::integral_constant<int, 0xA5>{}, std::integral_constant<int, j % W_STAGES>{}, c0 / 2 + j,
                   msg[(s + 15) & 15], msg[s]);
          });
        }
      }
      // The ring is idle now: when every corr step fits it, start loading them so that their
      // latency hides behind the digest (every wave has finished its LDS reads at the barrier;
      // the k loop's last wait left no DMA in flight).
      if (DENOISE && CT <= W_STAGES) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        for (int t = 0; t < CT; t++) cissue();  // corr step t -> stage t
      }
      {  // the last chunk: its TAIL pass was the k loop's last pass
        u32 keep, other;
        fold_head(acc, fx);
        fold_scatter(fx, lane, keep, other);
        const int last = (nchunks - 1) & 15;
#pragma unroll
        for (int s = 0; s < 16; s++)
          if (s == last) msg[s] = xor3(rotl13(msg[s]), keep, other);
      }
      // Digests and wins before the outputs: a winning lane's atomic waits for its wave's
      // outstanding memory operations, which in a storer wave are then only the previous item's
      // output stores (drained during this item's k loop), not this item's.
      // every lane digests the tile it owns: hash block hb = lane bit 3, g = lane & 7,
      // t = 2 (lane >> 5) + lane bit 4
      const int hb = (lane >> 3) & 1, g = lane & 7, t = 2 * (lane >> 5) + ((lane >> 4) & 1);
      u32 key[8], h[8];
#pragma unroll
      for (int i = 0; i < 8; i++) key[i] = ld_uniform(I.key, i);
      b3_keyed64(key, msg, h);
      const int row = bm0 + wm * 128 + hb * 64 + g, col = bn0 + wn * 64 + 2 * t;
      if (I.dump) {
        const long NB = p.n / 64;
        u32* d = I.dump + ((((long)(row >> 6) * 8 + g) * NB + (col >> 6)) * 4 + t) * DUMP_WORDS;
#pragma unroll
        for (int w = 0; w < 16; w++) d[w] = msg[w];
#pragma unroll
        for (int w = 0; w < 8; w++) d[16 + w] = h[w];
      }
      u32 target[8];
#pragma unroll
      for (int i = 0; i < 8; i++) target[i] = ld_uniform(p.target, i);
      if (I.wins && u256_le(h, target)) {
        const u32 slot = atomicAdd(I.wins, 1u);
        if (slot < (u32)p.max_wins) {
          u32* rec = I.wins + 1 + slot * WIN_WORDS;
          rec[0] = row;
          rec[1] = col;
#pragma unroll
          for (int i = 0; i < 8; i++) rec[2 + i] = h[i];
        }
      }

    } else {
      u32 unused = 0;
      int kt = 0;
      for (; kt + W_STAGES <= KT; kt += W_STAGES)
        static_for<W_STAGES>([&](auto stc) UWC_AI { step(NoFold{}, stc, kt + decltype(stc)::value, unused, unused); });
      // the last KT % W_STAGES steps: kt is a multiple of W_STAGES here, so step kt + s sits in
      // stage s (a loop over step_rt instead made the compiler spill the DMA offsets, whose
      // reloads then wait for every DMA in flight)
      static_for<W_STAGES - 1>([&](auto sc) UWC_AI {
        constexpr int s = decltype(sc)::value;
        if (kt + s < KT) step(NoFold{}, sc, kt + s, unused, unused);
      });
    }

    // A finished quarter (blocks (2h, nb), (2h + 1, nb)): stored at once, or, in the split
    // kernel, stored by the storers, the loaders' through a hand-off slot past the ring: loader w
    // writes its quarter to slot w (block i, register group j, lane l at 16 ((4 i + j) 64 + l)),
    // storer w + 4 reads it and stores it as wave (0, w). Two barriers per quarter: the slot is
    // written, the slot is read. The loaders never store an output.
    // A quarter's two blocks through LDS, stored by rows. The slot holds blocks i = 0, 1 as
    // 16-byte pieces: register group j (columns 8 j + 4 hh .. + 3) of the MFMA layout's lane
    // hh 32 + rr (row rr) at piece (4 i + j) 64 + hh 32 + (rr ^ 2 (2 j + hh)). It is read back by
    // rows: for store instruction jj, lane l takes row 8 jj + l / 8, columns 4 (l % 8) .. + 3, so
    // each store writes 8 whole row segments of the block (the MFMA layout stored directly
    // writes 32 rows x 16 bytes per instruction, and a launch's output burst then drains slower:
    // 77.9 -> 75.9 us per nonce in the batched mining launch). The XOR spreads both the writes
    // (16 consecutive rows) and the row reads (2 rows x 8 pieces) of 16 lanes over 16 distinct
    // 16-byte bank groups.
    auto put = [&](u8* slot, const v16i& a0, const v16i& a1) UWC_AI {
      const int hh = lane >> 5, rr = lane & 31;
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const v16i& v = i ? a1 : a0;
          *reinterpret_cast<v4i*>(slot + ((4 * i + j) * 64 + hh * 32 + (rr ^ (2 * (2 * j + hh)))) * 16) =
              v4i{v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]};
        }
    };
    // block 2 h + i of wave row swm (column half nb of wave column wn), from the slot
    auto store_rows = [&](const u8* slot, int swm, int h, int nb, int i) UWC_AI {
      if constexpr (OUT != OUT_NONE) {
        constexpr int ES = OUT == OUT_BF16 ? 2 : 4;  // output element bytes
        const int j = (lane & 7) >> 1, hh = lane & 1;
        const int row0 = bm0 + swm * 128 + (2 * h + i) * 32, col = bn0 + wn * 64 + nb * 32 + 4 * (lane & 7);
        u8* base = reinterpret_cast<u8*>(I.out) + ((long)row0 * p.ldc + col) * ES;
        float4 sw{};
        if constexpr (OUT != OUT_I32) sw = float4{p.b_scale[col], p.b_scale[col + 1], p.b_scale[col + 2], p.b_scale[col + 3]};
        // the four LDS reads first, then the stores: read, wait, store in turn put an LDS round
        // trip in front of every one of a storer's 64 stores per item
        v4i xs[4];
        float ascs[4];
        float4 rs[4];  // OUT_F32R: the residual of the four row segments, loaded first
        if constexpr (OUT == OUT_F32R) {
#pragma unroll
          for (int jj = 0; jj < 4; jj++) rs[jj] = uwc_load_nt(p.res + ((long)(row0 + 8 * jj + (lane >> 3)) * p.ldc + col));
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int rr = 8 * jj + (lane >> 3);
          xs[jj] = *reinterpret_cast<const v4i*>(slot + ((4 * i + j) * 64 + hh * 32 + (rr ^ (2 * (2 * j + hh)))) * 16);
          if constexpr (OUT != OUT_I32) ascs[jj] = p.a_scale[row0 + rr];
        }
#pragma unroll
        for (int jj = 0; jj < 4; jj++) {
          const int rr = 8 * jj + (lane >> 3);
          const v4i x = xs[jj];
          u8* dst = base + (u32)(rr * p.ldc * ES);  // < 2^32: 32 rows of at most 2^24 elements
          if constexpr (OUT == OUT_I32) {
            uwc_store_nt(dst, x);
          } else {
            const float asc = ascs[jj];
            const float y0 = __fmul_rn(__fmul_rn((float)x[0], asc), sw.x);
            const float y1 = __fmul_rn(__fmul_rn((float)x[1], asc), sw.y);
            const float y2 = __fmul_rn(__fmul_rn((float)x[2], asc), sw.z);
            const float y3 = __fmul_rn(__fmul_rn((float)x[3], asc), sw.w);
            if constexpr (OUT == OUT_F32) {
              uwc_store_nt(dst, float4{y0, y1, y2, y3});
            } else if constexpr (OUT == OUT_F32R) {
              uwc_store_nt(dst, float4{__fadd_rn(rs[jj].x, y0), __fadd_rn(rs[jj].y, y1), __fadd_rn(rs[jj].z, y2),
                                       __fadd_rn(rs[jj].w, y3)});
            } else {
              uwc_store_nt(dst, uint2{bf16_rne(y0) | (bf16_rne(y1) << 16), bf16_rne(y2) | (bf16_rne(y3) << 16)});
            }
          }
        }
      }
    };

    // A finished quarter (blocks (2h, nb), (2h + 1, nb)). Without SPLIT: with DENOISE the ring
    // holds the corrections while the quarters finish, so the blocks are stored directly;
    // otherwise through this wave's own 16 KiB of the idle ring (the caller's barrier ends the k
    // loop's reads of it). In the split kernel the storers store everything, the loaders'
    // quarters through a hand-off slot past the ring: loader w puts its quarter in slot w, storer
    // w + 4 stores it as wave (0, w), then puts and stores its own through the same slot. Two
    // barriers per quarter: the slot is written, the slot is done with. The loaders never store
    // an output.
    auto quarter_done = [&](int h, int nb, const v16i& v0, const v16i& v1) UWC_AI {
      if constexpr (!SPLIT) {
        if constexpr (DENOISE) {
          store_block(lane, I.out, wm, wn, 2 * h, nb, v0);
          store_block(lane, I.out, wm, wn, 2 * h + 1, nb, v1);
        } else if constexpr (OUT != OUT_NONE) {
          u8* slot = wsm + wave * 16384;
          put(slot, v0, v1);
          store_rows(slot, wm, h, nb, 0);
          store_rows(slot, wm, h, nb, 1);
        }
      } else {
        u8* slot = wsm + W_LDS + (wave & 3) * 8192;
        if constexpr (loader) put(slot, v0, v1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if constexpr (!loader) {
          // the loader's quarter, then this wave's own through the same slot (a wave's LDS
          // operations execute in order: the writes follow the reads they overwrite)
          store_rows(slot, wm - 1, h, nb, 0);
          store_rows(slot, wm - 1, h, nb, 1);
          put(slot, v0, v1);
          store_rows(slot, wm, h, nb, 0);
          store_rows(slot, wm, h, nb, 1);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
      }
    };

    if constexpr (DENOISE) {
      // Four passes over quarters of the wave's block keep the Horner accumulator at 32
      // registers; each quarter is final as soon as its pass ends. When all CT corr steps fit in
      // the ring (L * 2r <= W_STAGES * W_BK: the mining shapes) they are loaded once (the hashing
      // kernels issued them before the digest) and the four passes read them without further
      // barriers; otherwise they stream through the ring continuously across the passes (global
      // step g is corr step g mod CT).
      const int GT = 4 * CT;
      if (CT <= W_STAGES) {
        if constexpr (!HASH) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the k loop's last fragment reads
          __builtin_amdgcn_s_barrier();
          for (int t = 0; t < CT; t++) cissue();  // corr step t -> stage t
        }
        if constexpr (loader) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // also drains the hash phase's stores
        __builtin_amdgcn_s_barrier();
        if constexpr (SPLIT && W_STAGES == 2) {
          if (CT == W_STAGES) {
            // Stage by stage instead of quarter by quarter: corr stage t belongs to limb
            // L - 1 - t / CPL, and acc - sum_t (P_t << 7 li(t)) equals the Horner form mod 2^32.
            // Once every wave has read stage 0 it takes the next item's k step 0, whose latency
            // then hides behind stage 1's MFMAs and the output hand-off.
            const int sh0 = 7 * (L - 1), sh1 = 7 * (L - 1 - 1 / CPL);
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const int h = q >> 1, nb = q & 1;
              v16i tmp[2] = {v16i{}, v16i{}};
              step_mma_quarter(tmp, fbase, 0, h, nb);
              sub_shl(acc[2 * h][nb], tmp[0], sh0);
              sub_shl(acc[2 * h + 1][nb], tmp[1], sh0);
              // one quarter's fragments live at a time: the scheduler would otherwise hoist all
              // four quarters' reads and spill
              __builtin_amdgcn_sched_barrier(0);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // every read of stage 0 is complete
            __builtin_amdgcn_s_barrier();
            if (item + 1 < count) {
              if constexpr (loader) {
                // the offsets recomputed from an opaque lane index, so that the k loop's copy
                // is not kept live across the digest
                int z2;
                asm volatile("v_mov_b32 %0, 0" : "=v"(z2));
                const DmaOff<SPL> doff2 = dma_offsets<SPL>(k, wave, lane0 + z2);
                dma_step_s<SPL, 0, SPL>(lds_a(0), lds_b(0), doff2, p.it[item + 1].A + (long)bm0 * k, b_win, wave);
              }
              pre = 1;
            }
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const int h = q >> 1, nb = q & 1;
              v16i tmp[2] = {v16i{}, v16i{}};
              step_mma_quarter(tmp, fbase, 1, h, nb);
              sub_shl(acc[2 * h][nb], tmp[0], sh1);
              sub_shl(acc[2 * h + 1][nb], tmp[1], sh1);
              quarter_done(h, nb, acc[2 * h][nb], acc[2 * h + 1][nb]);
            }
            return;
          }
        }
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int h = q >> 1, nb = q & 1;
          v16i tmp[2] = {v16i{}, v16i{}};
          for (int t = 0, c = 0; t < CT; t++) {
            if (c == 0) {
              tmp[0] = tmp[0] << 7;
              tmp[1] = tmp[1] << 7;
            }
            if (++c == CPL) c = 0;
            step_mma_quarter(tmp, fbase, t, h, nb);
          }
          quarter_done(h, nb, acc[2 * h][nb] - tmp[0], acc[2 * h + 1][nb] - tmp[1]);
        }
      } else {
        if constexpr (loader) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // gfx9 counts stores in vmcnt
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // every wave is done reading the ring
#pragma unroll
        for (int g = 0; g < W_STAGES - 1; g++)
          if (g < GT) cissue();
        int g = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int h = q >> 1, nb = q & 1;
          v16i tmp[2] = {v16i{}, v16i{}};
          for (int t = 0, c = 0; t < CT; t++, g++) {
            wait_step<SPL>(min(GT - 1 - g, W_STAGES - 2), loader);
            if (ig < GT) cissue();
            if (c == 0) {
              tmp[0] = tmp[0] << 7;
              tmp[1] = tmp[1] << 7;
            }
            if (++c == CPL) c = 0;
            step_mma_quarter(tmp, fbase, g % W_STAGES, h, nb);
          }
          quarter_done(h, nb, acc[2 * h][nb] - tmp[0], acc[2 * h + 1][nb] - tmp[1]);
        }
      }
    } else {
      if constexpr (!SPLIT) {  // every wave is done reading the ring before it takes a slot of it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
      } else {
        // every wave is done reading the ring: the loaders start the next tile's first k steps,
        // whose latency then hides behind the output hand-off (the hand-off slots are past the
        // ring); its window and the DMA offsets are recomputed here rather than kept live
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (multi && item + 1 < count) {
          if constexpr (loader) {
            int nbm0, nbn0;
            tile256_of(p.m, p.n, (int)blockIdx.x + (item + 1) * (int)gridDim.x, nbm0, nbn0);
            int z2;
            asm volatile("v_mov_b32 %0, 0" : "=v"(z2));
            const DmaOff<SPL> doff2 = dma_offsets<SPL>(k, wave, lane0 + z2);
            const i8* na = I.A + (long)nbm0 * k;
            const i8* nb = p.B + (long)nbn0 * k;
#pragma unroll
            for (int s = 0; s < W_STAGES; s++)
              if (s < KT) dma_step_s<SPL, 0, SPL>(lds_a(s), lds_b(s), doff2, na + s * W_BK, nb + s * W_BK, wave);
          }
          pre = W_STAGES;
        }
      }
#pragma unroll
      for (int q = 0; q < 4; q++) quarter_done(q >> 1, q & 1, acc[2 * (q >> 1)][q & 1], acc[2 * (q >> 1) + 1][q & 1]);
    }

    if constexpr (!SPLIT) {
      if (item + 1 < count) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the next prologue refills the ring
        __builtin_amdgcn_s_barrier();
      }
    }

  };
  for (int item = 0; item < count; item++) {
    if (!SPLIT || is_loader) run_item(item, std::true_type{});
    else run_item(item, std::false_type{});
  }
}

template <bool H, bool D, int OUT, bool SPLIT = false>
static void go256(dim3 grid, hipStream_t s, const Gemm256Params& p) {
  auto kern = noisy_gemm256_kernel<H, D, OUT, SPLIT>;
  constexpr int lds = W_LDS + (SPLIT ? W_LDS_HANDOFF : 0);
  static bool attr = false;  // one attribute call per instantiation (the library is process-wide)
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    attr = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(W_THREADS), lds, s, p);
}

template <bool H, bool D>
static void out256(int out_mode, dim3 grid, hipStream_t s, const Gemm256Params& p) {
  switch (out_mode) {
    case OUT_NONE: go256<H, D, OUT_NONE>(grid, s, p); break;
    case OUT_I32: go256<H, D, OUT_I32>(grid, s, p); break;
    case OUT_BF16: go256<H, D, OUT_BF16>(grid, s, p); break;
    default: go256<H, D, OUT_F32>(grid, s, p); break;
  }
}

// Called by uwc_noisy_gemm after argument checks when m % 256 == 0 and n % 256 == 0; ldc is the
// output row stride (n, or wider when this GEMM writes the first n columns of a wider output).
int uwc_noisy_gemm256(const int8_t* A, const int8_t* B, int m, int n, int k, int r, const int8_t* corrA,
                      const int8_t* corrB, const int32_t* maxabs, int lmax, const uint32_t* key,
                      const uint32_t* target, uint32_t* wins, int max_wins, const float* a_scale, const float* b_scale,
                      void* out, int out_mode, int flags, uint32_t* tile_dump, int ldc, hipStream_t stream) {
  const bool hash = flags & FLAG_HASH, denoise = flags & FLAG_DENOISE;
  Gemm256Params p{};
  p.B = B;
  p.m = m, p.n = n, p.k = k, p.r = r;
  p.lmax = lmax;
  p.target = target;
  p.max_wins = max_wins;
  p.a_scale = a_scale;
  p.b_scale = b_scale;
  p.ldc = ldc;
  p.count = 1;
  p.it[0] = Gemm256Item{A, corrA, corrB, maxabs, key, wins, out, hash ? tile_dump : nullptr};
  const dim3 grid((m / W_BM) * (n / W_BN));
  // A plain int32 GEMM of at least W_MULTI tiles per CU: one persistent workgroup per CU takes
  // its tiles in turn on the split-role kernel, so a tile's output stores drain while the next
  // one computes and the next tile's first k steps load during the hand-off. Measured against one
  // workgroup per tile: 8192 x 151808 x 2048 (74 tiles per CU) 2942 -> 2813 us, 8192 x 12288 x
  // 2048 (6) 240 -> 233 us, and at 2-3 tiles per CU (graph-replayed, interleaved, outputs equal)
  // 8192 x 4096 x 2048 83.7 -> 77.9 us, 8192 x 4096 x 4096 130.0 -> 126.0, 8192 x 6144 x 4096
  // 184.3 -> 182.0, 8192 x 4096 x 14336 375.5 -> 369.0 (an earlier build of this form had been
  // slower at 2 tiles per CU). The fp32 dequant epilogue, which only the 4 storer waves run in this
  // form, is 1.5-3% slower at the prefill shapes (8192 x 28672 x 4096 802 -> 815 us), so it keeps
  // one workgroup per tile.
  const int G = uwc_cu_count() & ~7;
  const long tiles = (long)(m / W_BM) * (n / W_BN);
  if (W_MULTI > 0 && !hash && !denoise && out_mode == OUT_I32 && G >= 8 && tiles >= (long)W_MULTI * G &&
      tiles <= 0x7FFFFFFFL) {
    p.tiles = (int)tiles;
    p.count = 0;
    go256<false, false, OUT_I32, true>(dim3(G), stream, p);
    return uwc_launch_status("noisy_gemm256 (plain, multi-tile)");
  }
  if (hash && denoise) out256<true, true>(out_mode, grid, stream, p);
  else if (hash) out256<true, false>(out_mode, grid, stream, p);
  else if (denoise) out256<false, true>(out_mode, grid, stream, p);
  else out256<false, false>(out_mode, grid, stream, p);
  return uwc_launch_status("noisy_gemm256");
}

// Y = x + fmul(fmul(f32(A B^T), sx[i]), sw[j]) on 256 x 256 tiles, one workgroup per tile: the
// fp32 dequant epilogue with the residual added before the store (the same two roundings and the
// same add as a separate residual pass, without writing and rereading the dequantized rows).
// Called by uwc_igemm_dequant_residual_f32 for the shapes uwc_noisy_gemm puts on these tiles.
int uwc_gemm256_residual(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx, const float* sw,
                         const float* x, float* Y, hipStream_t stream) {
  Gemm256Params p{};
  p.B = B;
  p.m = m, p.n = n, p.k = k;
  p.a_scale = sx;
  p.b_scale = sw;
  p.res = x;
  p.ldc = n;
  p.count = 1;
  p.it[0] = Gemm256Item{A, nullptr, nullptr, nullptr, nullptr, nullptr, Y, nullptr};
  go256<false, false, OUT_F32R>(dim3((m / W_BM) * (n / W_BN)), stream, p);
  return uwc_launch_status("noisy_gemm256 (dequant + residual)");
}

// `count` (1 .. G256_MAXB) hashed, denoised GEMMs with int32 outputs sharing B in one launch, each
// equal to its own uwc_noisy_gemm256 call: the split-role kernel, whose output stores of one item
// drain while the next computes. Called by uwc_noisy_gemm_many after argument checks.
int uwc_noisy_gemm256_many(int count, const int8_t* const* A, const int8_t* B, int m, int n, int k, int r,
                           const int8_t* const* corrA, const int8_t* const* corrB, const int32_t* const* maxabs,
                           int lmax, const uint32_t* const* key, const uint32_t* target, uint32_t* const* wins,
                           int max_wins, void* const* out, uint32_t* const* tile_dump, hipStream_t stream) {
  if (count < 1 || count > G256_MAXB) return uwc_fail("uwc_noisy_gemm256_many: count=%d outside 1..%d", count, G256_MAXB);
  Gemm256Params p{};
  p.B = B;
  p.m = m, p.n = n, p.k = k, p.r = r;
  p.lmax = lmax;
  p.target = target;
  p.max_wins = max_wins;
  p.ldc = n;
  p.count = count;
  for (int i = 0; i < count; i++)
    p.it[i] = Gemm256Item{A[i], corrA[i], corrB[i], maxabs[i], key[i], wins[i], out[i], tile_dump ? tile_dump[i] : nullptr};
  go256<true, true, OUT_I32, true>(dim3((m / W_BM) * (n / W_BN)), stream, p);
  return uwc_launch_status("noisy_gemm256 (split, batched)");
}
