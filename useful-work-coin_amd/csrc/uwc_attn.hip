// detrt's exact causal attention on gfx950, bit-identical to the CPU reference
// (runtime/detrt/stage.py:171-196, runtime/detrt/qwen3.py:255-282; CUDA twin
// runtime/detgpu/kernels.py:196-633):
//
//   s_ij  = ((f32(q_i . k_j) * qs_i) * ks_j) * (1 / sqrt(hd))          exact int dot product
//   e_ij  = det_exp(s_ij - max_j s_ij)                                  j <= i, else 0
//   den_i = exact_rowsum(e_i)                                           int64 fixed point
//   pv_ij = (e_ij / den_i) * vs_j,  sp_i = max(max_j pv_ij, 1e-30) / 16383
//   p_ij  = clamp(rint(pv_ij / sp_i), 0, 16383) = 128 hi + lo
//   o_id  = f32(sum_j p_ij v_jd) * sp_i                                 exact int64 sum
//
// The design is MI355X-first rather than a row-per-block port:
//   * a wave owns 16 queries of one head; both products run on v_mfma_i32_16x16x64_i8:
//     scores as S^T = K Q^T (A = 16 keys, B = the wave's 16 queries, held in registers), the
//     output as O^T = V^T P^T with P's two 7-bit limbs as int8 B operands (int32 accumulators
//     stay exact: 127 * 127 * T < 2^31 for T <= 131072);
//   * the C registers of the four 16x16 score blocks of a 64-key tile are, lane by lane, the
//     16 keys of one query that the P x V MFMA needs as its k slots (keys 16 b + 4 g + i for lane
//     group g), so P never leaves registers; V^T is stored with its keys in that order
//     (qkv_post / v_transpose write it so), one 16-byte load (in the stored form one LDS read
//     from a ring the workgroup fills) per lane and dim block;
//   * the three row statistics (max, exact sum, max of the scaled probabilities) each need the
//     previous one over the whole causal row: sweep 1 finds the max, sweep 2 the exact sum and,
//     from per-lane candidates, the third statistic (sweep 3, a pass over the keys of its own,
//     runs only for waves with a near tie), sweep 4 quantizes P and runs P x V; the scores are
//     recomputed on the matrix cores rather than stored as T x T rows, and the exponentials of
//     sweep 2 are kept in a scratch for sweep 4 (uwc_attention_ws), which also runs sweep 1 as
//     a kernel of its own whose workgroups share each key tile through LDS (attn_rowmax_kernel);
//   * workgroups are mapped so that each XCD owns whole kv heads, whose K and V then stay in its
//     L2 (at_block);
//   * exp rows have max exactly det_exp(0) = 1 and every term below 2, so exact_rowsum's
//     scale is the constant 2^41 (L = 20 for MAX_KEYS = 2^20): a term is rint(e * 2^41) < 2^42;
//   * the divisions by the row constants den and sp are products with their float64
//     reciprocals (exact after rounding to float32, see at_div).
// Row statistics are per lane partials combined across the 4 lane groups (xor 16, 32); all
// reductions are max or exact integer sums, so the key split cannot change a bit.
#include <type_traits>

#include "uwc_rows.h"

#define AT_PLEVELS 16383.0f
// lambdas are always inlined: an out-of-line call would take the address of the register arrays
// they capture (private memory)
#define AT_AI __attribute__((always_inline))
typedef void __attribute__((address_space(3)))* s2_lptr_at;

// One wave-wide DMA into LDS at lds + 16 lane (dwordx4) or lds + 4 lane (dword); lds is
// wave-uniform (M0). Such loads count in vmcnt only, so the kernels wait for them with explicit
// vmcnt counts and a workgroup barrier before another wave reads the data.
__device__ __forceinline__ void at_dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
// the same with the non-temporal hint (data read once: the stored exponentials)
__device__ __forceinline__ void at_dma16_nt(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds) : "memory", "m0");
}
__device__ __forceinline__ void at_dma4(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void at_waitv() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// LDS barrier: this wave's LDS operations done, then every wave's (global memory is not fenced)
__device__ __forceinline__ void at_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }


__device__ __forceinline__ v4i at_zero4() { return v4i{0, 0, 0, 0}; }

// The chunk (four 16-byte slots) of row r (0..15) in a 16-row block of the P x V sweep's V ring:
// 4 ((r >> 1) & 3) + 2 (r & 1) + (r >> 3)
__host__ __device__ constexpr int at_vchunk(int r) { return 4 * ((r >> 1) & 3) + 2 * (r & 1) + (r >> 3); }

// round_half_even(e * 2^41) for 0 <= e < 2, as a float64 integer (exact: e * 2^41 is a float32
// scaled by a power of two, its rounding to an integer is a float32 integer below 2^42).
__device__ __forceinline__ double at_fix41(float e) { return (double)rintf(__fmul_rn(e, 0x1p41f)); }

// det_exp(z) for z <= 0 or z = -inf (the attention's s - max): the overflow and NaN branches of
// dx_exp cannot trigger, the rest is dx_exp's op sequence. With UNDER false (tiles without masked
// keys, where z is finite) det_exp's underflow rule (t < -126 gives 0) is left out: ldexp then
// returns p 2^n < 2^-126 (a subnormal or 0) where det_exp gives 0, and no result of the kernel
// can tell them apart: the fixed-point term rint(e 2^41) is 0 for both, such a key's product e vs
// is far below the best product of its lane and row (at least 1e-8/127 times the row's max key,
// whose e is 1), so it is never a candidate, and its quantized probability rounds to 0 (pv / sp
// stays below 2^-126 16383 (vs / max vs)). Three VALU operations fewer per score element.
template <bool UNDER = true>
__device__ __forceinline__ float at_exp(float z) {
  float t = __fmul_rn(z, DX_LOG2E);
  bool under = false;
  if constexpr (UNDER) {
    under = t < -126.0f;
    if (under) t = 0.0f;
  }
  const float n = floorf(t);
  const float f = __fsub_rn(t, n);
  float p = DX_E7;
  p = __fadd_rn(__fmul_rn(p, f), DX_E6);
  p = __fadd_rn(__fmul_rn(p, f), DX_E5);
  p = __fadd_rn(__fmul_rn(p, f), DX_E4);
  p = __fadd_rn(__fmul_rn(p, f), DX_E3);
  p = __fadd_rn(__fmul_rn(p, f), DX_E2);
  p = __fadd_rn(__fmul_rn(p, f), DX_E1);
  p = __fadd_rn(__fmul_rn(p, f), DX_E0);
  // p * 2^n with -126 <= n <= 0 and p >= 1 is a normal number, so the product is exact and
  // equals ldexp(p, n), one instruction instead of building 2^n and multiplying
  const float r = __builtin_amdgcn_ldexpf(p, (int)n);
  if constexpr (UNDER) return under ? 0.0f : r;
  else return r;
}

// x / d correctly rounded to float32, for float32 x and a per-row divisor given as
// rd = 1.0 / (double)d (correctly rounded in float64): the float64 product is within 2^-52
// (relative) of x / d, while a float32 quotient of two float32 values is never a rounding tie and
// lies more than 2^-49 (relative) from every float32 midpoint, so rounding the product to float32
// gives the correctly rounded quotient.
__device__ __forceinline__ float at_div(float x, double rd) { return (float)((double)x * rd); }

__device__ __forceinline__ float at_max_groups(float v) {
  v = fmaxf(v, __shfl_xor(v, 16, 64));
  return fmaxf(v, __shfl_xor(v, 32, 64));
}

__device__ __forceinline__ u64 at_sum_groups(u64 v) {
#pragma unroll
  for (int s = 16; s <= 32; s <<= 1) {
    const u32 lo = (u32)__shfl_xor((int)(u32)v, s, 64), hi = (u32)__shfl_xor((int)(u32)(v >> 32), s, 64);
    v += ((u64)hi << 32) | lo;
  }
  return v;
}

// The scales of one 64-key tile (keys kt*64 .. +63, clamped to T - 1) staged through the wave's
// own LDS slot; lane group g then reads keys 16 b + 4 g .. + 3 of block b as one float4. LDS
// operations of a wave complete in order, so no barrier is involved.
__device__ __forceinline__ void at_stage_scales(const float* __restrict__ sc, u32 base, int stride, int k0, int T,
                                                float* slot, int lane, float4 out[4]) {
  const int j = min(k0 + lane, T - 1);
  slot[lane] = sc[base + (u32)j * (u32)stride];
  __builtin_amdgcn_wave_barrier();
  const int g = lane >> 4;
#pragma unroll
  for (int b = 0; b < 4; b++) out[b] = *reinterpret_cast<const float4*>(slot + 16 * b + 4 * g);
  __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float at_get(const float4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// Block id -> (q tile, head, sequence). Workgroups are dispatched round-robin over the 8 XCDs
// (id % 8). When the (sequence, kv head) units split evenly over them, XCD x takes units x,
// x + 8, ..., so every key and value tile an XCD reads belongs to its own units: at T = 8192 one
// kv head's K and V (1 MiB each) stay in the XCD's 4 MB L2, where the plain order had every XCD
// read all 8 kv heads' 8 MiB from the Infinity Cache for each 16-query wave. Within an XCD the
// longest rows (highest q tile) go first.
__device__ __forceinline__ void at_block(int id, int ntiles, int H, int Hkv, int B, int& qt, int& h, int& bseq) {
  const int G = H / Hkv, units = B * Hkv;
  if (units % 8 == 0) {
    const int x = id & 7, j = id >> 3;
    const int per_tile = units / 8 * G;  // this XCD's blocks of one q tile
    qt = ntiles - 1 - j / per_tile;
    const int r = j % per_tile, u = x + 8 * (r / G);
    h = (u % Hkv) * G + r % G;
    bseq = u / Hkv;
  } else {
    qt = ntiles - 1 - id % ntiles;
    h = (id / ntiles) % H;
    bseq = id / (ntiles * H);
  }
}

// Exp tiles of the stored form: wave block wq (queries 16 wq .. + 15) of a (sequence, head) owns
// tiles 0 .. wq / 4 (its key tiles), the blocks' tiles back to back: block wq starts at tile
// (a + 1)(2 a + b) for wq = 4 a + b, and a (sequence, head) holds at_tiles(Tp) of them.
__host__ __device__ constexpr u64 at_tile0(u64 wq) { return (wq / 4 + 1) * (2 * (wq / 4) + wq % 4); }
__host__ __device__ constexpr u64 at_tiles(u64 Tp) { return at_tile0(Tp / 16); }

// Without ES the kernel runs the four sweeps, recomputing the scores and det_exp in each.
// ES (exp stored, uwc_attention_ws) runs after attn_rowmax_kernel, which leaves each row's max
// of y = fl(fl(acc qs) ks) in rows (B T H floats, index (b T + q) H + h; a max in any order is
// the same number). Sweep 2 writes every e_ij it computes to escr (one 4 KiB tile per wave and
// key tile, 16 floats per lane as four float4 at lane and piece offsets), and sweeps 3 and 4
// read them back instead of recomputing the scores and det_exp (about two thirds of the VALU
// work per score element); the same values go through the same operations, so both forms give
// the same bits. The scratch (2.2 GB at T = 8192, 16 heads) is written and read with the
// non-temporal hint: cached normally, its stream evicted the XCD's K and V from L2. Sweep 4 of
// the stored form feeds every operand through LDS (DMA rings, see there). The workgroups of
// one launch are at different sweeps at any time (their causal rows differ in length), so one
// workgroup's VALU-bound sums overlap another's memory-bound P x V on the same CU.
template <int HD, bool ES>
__global__ void __launch_bounds__(256, ES ? 3 : HD == 128 ? 2 : 3)
    attention_kernel(const i8* __restrict__ qq, const float* __restrict__ qs, const i8* __restrict__ kq,
                     const float* __restrict__ ks, const i8* __restrict__ vt, const float* __restrict__ vs, int T,
                     int Tp, int H, int Hkv, float inv_sqrt, float* __restrict__ o, float* __restrict__ escr,
                     const float* __restrict__ rows) {
  constexpr int NC = (HD + 63) / 64;  // 64-dim chunks of the score product
  constexpr int ND = HD / 16;         // 16-dim blocks of the output
  __shared__ __attribute__((aligned(16))) float at_slot[4][2][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 15, g = lane >> 4;
  int qt, h, bseq;
  at_block((int)blockIdx.x, Tp / 64, H, Hkv, (int)(gridDim.x / (u32)(Tp / 64 * H)), qt, h, bseq);
  const int q0 = qt * 64 + wave * 16;
  // whole waves only (the stored form keeps every wave: its sweep 4 has workgroup barriers; a
  // wave past T computes clamped rows and stores nothing)
  if (!ES && q0 >= T) return;
  const int hk = h / (H / Hkv);
  // 32-bit offsets: the host checks B * T * max(H, Hkv) * HD < 2^31
  const u32 nb = (u32)(bseq * T);
  const int qi = q0 + ql, qc = min(qi, T - 1);
  const float my_qs = qs[(nb + qc) * (u32)H + h];
  float* sk_slot = at_slot[wave][0];
  float* sv_slot = at_slot[wave][1];
  const u32 sc_base = nb * (u32)Hkv + hk;  // ks / vs index of key j: sc_base + j * Hkv

  v4i qf[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int d0 = 64 * c + 16 * g;
    qf[c] = d0 < HD ? *reinterpret_cast<const v4i*>(qq + ((nb + qc) * (u32)H + h) * HD + d0) : at_zero4();
  }
  const int kmax = min(T, q0 + 16);  // keys any query of the wave sees
  const int nkt = (kmax + 63) / 64;
  const i8* kbase = kq + (size_t)hk * HD;
  // stored form: this wave's exp tiles (tile kt at + 1024 kt floats, piece b at + 256 b)
  float* ewave = nullptr;
  if constexpr (ES)
    ewave = escr + ((u64)(bseq * H + h) * at_tiles((u64)Tp) + at_tile0((u64)(q0 >> 4))) * 1024 + lane * 4;

  // integer scores of key tile kt: acc[b][i] = q_qi . k_j, j = 64 kt + 16 b + 4 g + i
  auto iscores = [&](int kt, v4i acc[4]) {
#pragma unroll
    for (int b = 0; b < 4; b++) {
      acc[b] = at_zero4();
      const int kr = min(kt * 64 + 16 * b + ql, T - 1);
      const i8* kp = kbase + (nb + kr) * (u32)(Hkv * HD);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int d0 = 64 * c + 16 * g;
        const v4i kf = d0 < HD ? *reinterpret_cast<const v4i*>(kp + d0) : at_zero4();
        acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, qf[c], acc[b], 0, 0, 0);
      }
    }
  };
  // scores as floats. Tiles below nfull hold only keys <= q0 (the wave's first query) and < T and
  // need no mask; in the others masked entries are -inf. MASK is a compile-time flag: the sweeps
  // run the full tiles, then the one diagonal tile.
  const int nfull = (q0 + 1) / 64;
  auto scores = [&](int kt, float S[4][4], float4 skv[4], auto mask) {
    constexpr bool MASK = decltype(mask)::value;
    v4i acc[4];
    iscores(kt, acc);
    at_stage_scales(ks, sc_base, Hkv, kt * 64, T, sk_slot, lane, skv);
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float s = __fmul_rn(__fmul_rn(__fmul_rn((float)acc[b][i], my_qs), at_get(skv[b], i)), inv_sqrt);
        if constexpr (MASK) {
          const int j = kt * 64 + 16 * b + 4 * g + i;
          S[b][i] = (j <= qi && j < T) ? s : -__int_as_float(0x7f800000);
        } else {
          S[b][i] = s;
        }
      }
  };
  auto sweep = [&](auto body) {
    for (int kt = 0; kt < nfull; kt++) body(kt, std::false_type{});
    for (int kt = nfull; kt < nkt; kt++) body(kt, std::true_type{});
  };
  // over tiles 0 .. nkt - 1 with loads two tiles ahead: prefetch(kt, slot) loads tile kt into
  // register set slot, body(kt, slot) uses it (slot is a compile-time 0 or 1)
  auto pipelined = [&](auto prefetch, auto body) AT_AI {
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if (nkt > 0) prefetch(0, S0{});
    if (nkt > 1) prefetch(1, S1{});
    for (int kt = 0; kt < nkt; kt += 2) {
      body(kt, S0{});
      if (kt + 2 < nkt) prefetch(kt + 2, S0{});
      if (kt + 1 < nkt) {
        body(kt + 1, S1{});
        if (kt + 3 < nkt) prefetch(kt + 3, S1{});
      }
    }
  };
  // The K fragments and the key scale of one 64-key tile, fetched two tiles ahead of their use in
  // sweeps 1 and 2 (each tile's loads then overlap the previous tiles' work instead of stalling
  // the wave: with two waves per SIMD a wave's own loads are its main wait)
  struct KTile {
    v4i kf[4][NC];
    float ks, vs;
  };
  auto kfetch = [&](int kt, KTile& t) AT_AI {
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int kr = min(kt * 64 + 16 * b + ql, T - 1);
      const i8* kp = kbase + (nb + kr) * (u32)(Hkv * HD);
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int d0 = 64 * c + 16 * g;
        t.kf[b][c] = d0 < HD ? *reinterpret_cast<const v4i*>(kp + d0) : at_zero4();
      }
    }
    t.ks = ks[sc_base + (u32)min(kt * 64 + lane, T - 1) * (u32)Hkv];
    t.vs = vs[sc_base + (u32)min(kt * 64 + lane, T - 1) * (u32)Hkv];
  };
  // scores(kt, ...) from a fetched tile: the same MFMAs, scales and mask
  auto scores_t = [&](int kt, const KTile& t, float S[4][4], auto mask, auto noinv) AT_AI {
    constexpr bool MASK = decltype(mask)::value, NOINV = decltype(noinv)::value;
    float4 skv[4];
    sk_slot[lane] = t.ks;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < 4; b++) skv[b] = *reinterpret_cast<const float4*>(sk_slot + 16 * b + 4 * g);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < 4; b++) {
      v4i acc = at_zero4();
#pragma unroll
      for (int c = 0; c < NC; c++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(t.kf[b][c], qf[c], acc, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float y = __fmul_rn(__fmul_rn((float)acc[i], my_qs), at_get(skv[b], i));
        const float sv = NOINV ? y : __fmul_rn(y, inv_sqrt);
        if constexpr (MASK) {
          const int j = kt * 64 + 16 * b + 4 * g + i;
          S[b][i] = (j <= qi && j < T) ? sv : -__int_as_float(0x7f800000);
        } else {
          S[b][i] = sv;
        }
      }
    }
  };
  // a sweep over the key tiles with the tiles fetched two ahead; full tiles unmasked. With noinv
  // the scores are left without the final factor 1 / sqrt(hd) (sweep 1's max needs no more)
  auto ksweep = [&](auto body, auto noinv) AT_AI {
    KTile kb[2];
    pipelined([&](int kt, auto sl) AT_AI { kfetch(kt, kb[decltype(sl)::value]); },
              [&](int kt, auto sl) AT_AI {
                float S[4][4];
                if (kt < nfull) {
                  scores_t(kt, kb[decltype(sl)::value], S, std::false_type{}, noinv);
                  body(kt, S, kb[decltype(sl)::value], std::false_type{});
                } else {
                  scores_t(kt, kb[decltype(sl)::value], S, std::true_type{}, noinv);
                  body(kt, S, kb[decltype(sl)::value], std::true_type{});
                }
              });
  };

  // sweep 1: row max. A score is fl(y * inv) with y = fl(fl(acc * qs) * ks) and inv > 0, a
  // monotone function of y, so the max score is fl(max_j y_j * inv) (-inf for an empty row too)
  float mx = -__int_as_float(0x7f800000);
  // a padding query (qi >= T) sees keys 0 .. T - 1, as query T - 1 does
  const u32 ridx = (nb + qc) * (u32)H + h;
  if constexpr (ES) {
    mx = __fmul_rn(rows[ridx], inv_sqrt);
  } else {
    ksweep([&](int, const float (&Y)[4][4], const KTile&, auto) AT_AI {
#pragma unroll
      for (int b = 0; b < 4; b++)
#pragma unroll
        for (int i = 0; i < 4; i++) mx = fmaxf(mx, Y[b][i]);
    }, std::true_type{});
    mx = __fmul_rn(at_max_groups(mx), inv_sqrt);
  }

  // stored form: tile loads for sweeps 3 and 4, and the V scales of a tile (lane's key
  // 64 kt + lane, staged through the wave's LDS slot as at_stage_scales does)
  auto eload = [&](int kt, float4 (&ev)[4]) AT_AI {
#pragma unroll
    for (int b = 0; b < 4; b++) ev[b] = uwc_load_nt(ewave + kt * 1024 + b * 256);
  };
  auto vsload = [&](int kt) AT_AI { return vs[sc_base + (u32)min(kt * 64 + lane, T - 1) * (u32)Hkv]; };
  auto vsstage = [&](float v, float4 out[4]) AT_AI {
    sv_slot[lane] = v;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < 4; b++) out[b] = *reinterpret_cast<const float4*>(sv_slot + 16 * b + 4 * g);
    __builtin_amdgcn_wave_barrier();
  };
  // sweep 2: exact denominator (fixed point at 2^41); masked entries give det_exp(-inf) = 0.
  // A tile's 16 terms per lane sum exactly in float64 (< 2^46), then join a u64 total.
  //
  // Sweep 3's statistic pm = max_j fl(fl(e_j / den) vs_j) is found here from candidates: every
  // lane keeps the largest fp32 product p1 = fl(e vs) of its keys with that key's e and vs, and
  // the largest product p2 among its other keys. With q_j = fl(e_j / den) and pv_j = fl(q_j vs_j),
  // pv_j lies within a factor (1 +- 2^-24)^2 of e_j vs_j / den, and fl(e vs) within (1 +- 2^-24)
  // of e vs; so a key whose product is at most p1 (1 - 2^-21) cannot have a larger pv than the
  // lane's best key (products are normal numbers: the best is at least vs >= 1e-8 / 127, and a
  // key whose product underflows is far below it). When every lane of the wave has
  // p2 <= fl(p1 (1 - 2^-16)) (stricter than needed), pm is the max over the lanes' best keys of
  // their pv, the same bits sweep 3 gives; otherwise (a near tie, e.g. repeated keys) the wave
  // runs sweep 3.
  u64 dsum = 0;
  float p1 = -1.f, p2 = -1.f, e1 = 0.f, v1 = 0.f;
  ksweep([&](int kt, const float (&S)[4][4], const KTile& t, auto mask) AT_AI {
    float4 svv[4];
    sv_slot[lane] = t.vs;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int b = 0; b < 4; b++) svv[b] = *reinterpret_cast<const float4*>(sv_slot + 16 * b + 4 * g);
    __builtin_amdgcn_wave_barrier();
    double part = 0.0;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      float e[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        e[i] = at_exp<decltype(mask)::value>(__fsub_rn(S[b][i], mx));
        part += at_fix41(e[i]);
        const float vsj = at_get(svv[b], i), pr = __fmul_rn(e[i], vsj);
        const bool nb = pr > p1;
        p2 = nb ? p1 : fmaxf(p2, pr);
        p1 = nb ? pr : p1;
        e1 = nb ? e[i] : e1;
        v1 = nb ? vsj : v1;
      }
      if constexpr (ES) uwc_store_nt(ewave + kt * 1024 + b * 256, float4{e[0], e[1], e[2], e[3]});
    }
    dsum += (u64)part;
  }, std::false_type{});
  dsum = at_sum_groups(dsum);
  const float den = (float)ldexp((double)dsum, -41);
  const double rden = 1.0 / (double)den;

  // sweep 3: max of the V-scaled probabilities, only for waves with a near tie (see sweep 2)
  float pm = 0.f;
  const bool near_tie = p2 > __fmul_rn(p1, 0x1.fffep-1f);
  if (__ballot(near_tie) == 0) {
    pm = fmaxf(0.f, __fmul_rn(at_div(e1, rden), v1));
  } else if constexpr (ES) {
    float4 eb[2][4];
    float vb[2];
    pipelined(
        [&](int kt, auto sl) AT_AI {
          eload(kt, eb[decltype(sl)::value]);
          vb[decltype(sl)::value] = vsload(kt);
        },
        [&](int, auto sl) AT_AI {
          constexpr int L = decltype(sl)::value;
          float4 svv[4];
          vsstage(vb[L], svv);
#pragma unroll
          for (int b = 0; b < 4; b++)
#pragma unroll
            for (int i = 0; i < 4; i++) pm = fmaxf(pm, __fmul_rn(at_div(at_get(eb[L][b], i), rden), at_get(svv[b], i)));
        });
  } else sweep([&](int kt, auto mask) {
    float S[4][4];
    float4 skv[4], svv[4];
    scores(kt, S, skv, mask);
    at_stage_scales(vs, sc_base, Hkv, kt * 64, T, sv_slot, lane, svv);
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float e = at_exp(__fsub_rn(S[b][i], mx));
        pm = fmaxf(pm, __fmul_rn(at_div(e, rden), at_get(svv[b], i)));
      }
  });
  pm = at_max_groups(pm);
  const float sp = __fdiv_rn(fmaxf(pm, 1e-30f), AT_PLEVELS);
  const double rsp = 1.0 / (double)sp;

  // sweep 4: 14-bit probabilities as two 7-bit limbs, O^T = V^T P^T on the matrix cores
  v4i ohi[ND], olo[ND];
#pragma unroll
  for (int d = 0; d < ND; d++) ohi[d] = olo[d] = at_zero4();
  const i8* vbase = vt + (size_t)(bseq * Hkv + hk) * HD * Tp;
  // P of one tile from its exp values e[b][i] and V scales, times the tile's V rows (vf[d])
  auto pv_tile = [&](const float (&e)[4][4], const float4 (&svv)[4], const v4i (&vf)[ND]) AT_AI {
    v4i bhi, blo;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      u32 ph = 0, pl = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float pv = __fmul_rn(at_div(e[b][i], rden), at_get(svv[b], i));
        const int p = (int)fminf(fmaxf(rintf(at_div(pv, rsp)), 0.0f), AT_PLEVELS);
        ph |= (u32)(p >> 7) << (8 * i);
        pl |= (u32)(p & 127) << (8 * i);
      }
      bhi[b] = (int)ph;
      blo[b] = (int)pl;
    }
#pragma unroll
    for (int d = 0; d < ND; d++) {
      ohi[d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[d], bhi, ohi[d], 0, 0, 0);
      olo[d] = __builtin_amdgcn_mfma_i32_16x16x64_i8(vf[d], blo, olo[d], 0, 0, 0);
    }
  };
  auto vload = [&](int kt, v4i (&vf)[ND]) AT_AI {
#pragma unroll
    for (int d = 0; d < ND; d++)
      vf[d] = *reinterpret_cast<const v4i*>(vbase + (u32)(16 * d + ql) * (u32)Tp + kt * 64 + 16 * g);
  };
  if constexpr (ES) {
    // Sweep 4 with every load a DMA into LDS: the wave's own exponentials (4 KiB a tile) into
    // its slot of a 2-stage ring, the tile's V^T rows (64 keys of every dim, the same for the
    // four waves: each DMAs a quarter) and V scales (a quarter each) into shared rings. Loaded per
    // wave into registers, the 13 vector-memory instructions of a wave and tile (8 of them for
    // V tiles the workgroup's four waves all read) bound the sweep at the CU's rate for such
    // instructions; here a wave issues 7 DMAs a tile. No compiler-issued global load remains in
    // the loop, so every wait count is static. The V tile is HD / 16
    // blocks of 16 rows x 64 key bytes (1 KiB, 64 slots of 16 bytes); row r of block d sits in
    // chunk at_vchunk(r) of four slots (its 64 bytes, so four consecutive DMA lanes read one
    // row segment), piece p at slot p ^ ((r >> 1) & 3) of the chunk. A fragment read (lane
    // group g reads piece g of the block's 16 rows) then gives every lane the slot residue
    // (mod 16) the row-max ring's reads give it, a pattern measured free of bank conflicts
    // (the earlier slot 4 r + (p ^ ((r >> 2) & 3)), distinct residues in each 16-lane group,
    // measured 2-way).
    constexpr int VT = HD * 64;                   // bytes of a V tile
    constexpr int VS = VT / 16 / 4;               // its 16-byte slots per wave
    constexpr int VD = VS >= 64 ? VS / 64 : 1;    // V DMAs per wave and tile
    constexpr int VL = VS >= 64 ? 64 : VS;        // lanes active in each
    static_assert(VD * VL * 4 * 16 == VT, "V tile split over the four waves");
    // two ring stages, so that three workgroups (at three waves per SIMD) fit a CU's LDS
    constexpr int NS = 2;
    static_assert(NS == 2, "the loop's wait assumes one tile in flight");
    __shared__ __attribute__((aligned(16))) u8 ering[NS][4][4096];
    __shared__ __attribute__((aligned(16))) u8 vring[NS][VT];
    __shared__ __attribute__((aligned(16))) float sring[NS][64];
    const u32 er0 = (u32)(uintptr_t)(s2_lptr_at)ering[0][0], vr0 = (u32)(uintptr_t)(s2_lptr_at)vring[0];
    const u32 sr0 = (u32)(uintptr_t)(s2_lptr_at)sring[0];
    // the row constants are final before the loop (the compiler's waits for the loads they
    // come from stay out of it)
    asm volatile("" ::"v"(rden), "v"(rsp));
    // the wave's stores of its exponentials (sweep 2) are done before its DMAs read them
    at_waitv<0>();
    auto issue = [&](int kt) AT_AI {
      const int st = kt % NS;
#pragma unroll
      for (int b = 0; b < 4; b++)
        at_dma16_nt(ewave + kt * 1024 + b * 256,
                    __builtin_amdgcn_readfirstlane(er0 + (u32)((st * 4 + wave) * 4096 + b * 1024)));
#pragma unroll
      for (int u = 0; u < VD; u++) {
        const int s16 = (wave * VD + u) * VL + lane, c = (s16 >> 2) & 15;
        const int r = ((c & 1) << 3) | ((c >> 2) << 1) | ((c >> 1) & 1);  // at_vchunk(r) = c
        const int row = 16 * (s16 >> 6) + r, p = (s16 & 3) ^ ((r >> 1) & 3);
        const i8* src = vbase + (u32)row * (u32)Tp + kt * 64 + 16 * p;
        const u32 dst = __builtin_amdgcn_readfirstlane(vr0 + (u32)(st * VT + (wave * VD + u) * VL * 16));
        if (VL == 64 || lane < VL) at_dma16(src, dst);
      }
      const float* ssrc = vs + sc_base + (u32)min(kt * 64 + wave * 16 + (lane & 15), T - 1) * (u32)Hkv;
      if (lane < 16) at_dma4(ssrc, __builtin_amdgcn_readfirstlane(sr0 + (u32)(st * 256 + wave * 64)));
    };
    for (int t = 0; t < NS - 1; t++)
      if (t < nkt) issue(t);
    for (int kt = 0; kt < nkt; kt++) {
      at_waitv<0>();  // tile kt's DMAs done (with two stages no other tile is in flight)
      at_lds_barrier();  // tile kt is in LDS; every wave is done with tile kt - 1's stage
      if (kt + NS - 1 < nkt) issue(kt + NS - 1);
      const int st = kt % NS;
      float e[4][4];
      float4 svv[4];
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const float4 x = *reinterpret_cast<const float4*>(ering[st][wave] + b * 1024 + lane * 16);
        e[b][0] = x.x, e[b][1] = x.y, e[b][2] = x.z, e[b][3] = x.w;
        svv[b] = *reinterpret_cast<const float4*>(&sring[st][16 * b + 4 * g]);
      }
      v4i vf[ND];
#pragma unroll
      for (int d = 0; d < ND; d++)
        vf[d] = *reinterpret_cast<const v4i*>(vring[st] + 16 * (64 * d + 4 * at_vchunk(ql) + (g ^ ((ql >> 1) & 3))));
      pv_tile(e, svv, vf);
    }
  } else sweep([&](int kt, auto mask) {
    float S[4][4];
    float4 skv[4], svv[4];
    scores(kt, S, skv, mask);
    at_stage_scales(vs, sc_base, Hkv, kt * 64, T, sv_slot, lane, svv);
    float e[4][4];
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) e[b][i] = at_exp(__fsub_rn(S[b][i], mx));
    v4i vf[ND];
    vload(kt, vf);
    pv_tile(e, svv, vf);
  });
  if (qi >= T) return;
  // lane holds dims 16 d + 4 g + i of query qi
  float* orow = o + ((nb + qi) * (u32)H + h) * HD;
#pragma unroll
  for (int d = 0; d < ND; d++) {
    float4 r;
    float* rr = reinterpret_cast<float*>(&r);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const long long a = ((long long)ohi[d][i] << 7) + (long long)olo[d][i];
      rr[i] = __fmul_rn((float)a, sp);
    }
    *reinterpret_cast<float4*>(orow + 16 * d + 4 * g) = r;
  }
}

// ------------------------------------------------------------------ sweep 1 alone
// The row max of y = fl(fl(acc qs) ks) over each query's causal keys, for the stored-exp form.
// Inside the full kernel (two waves per SIMD) this sweep waited on its K loads most of the time:
// every wave fetched each 64-key tile itself, 16 half-used 128-byte lines per load instruction.
// Here the 4 HPW waves of a workgroup (64 queries of each of HPW heads that share one kv head,
// so the same key tiles) share each tile: it is DMA'd once into an LDS ring of NS tiles
// (global_load_lds_dwordx4, each lane 16 bytes, eight consecutive lanes one whole 128-byte key
// row), every wave issuing the same number of DMAs per tile so that its wait counts are static,
// and read back in the MFMA operand layout. The 16-byte pieces of key row m sit at piece
// p ^ swz(m) so that the 16 lanes of a read (rows 16 b .. + 15, one piece) hit 16 distinct bank
// groups. The tiles' DMAs from L2 bound this kernel (one head per workgroup ran no faster with
// a third less VALU work), so the heads of a kv head share them: Qwen3-1.7B (2 heads per kv
// head) moves half the key bytes per score.
template <int HD>
__host__ __device__ constexpr int at_swz(int m) {
  return (m / (16 / (HD / 16))) & (HD / 16 - 1);
}

template <int HD, int NS, int HPW>
__global__ void __launch_bounds__(256 * HPW) attn_rowmax_kernel(const i8* __restrict__ qq, const float* __restrict__ qs,
                                                                const i8* __restrict__ kq, const float* __restrict__ ks,
                                                                int T, int Tp, int H, int Hkv, float* __restrict__ rmax) {
  constexpr int NC = (HD + 63) / 64;
  constexpr int PR = HD / 16;                     // 16-byte pieces per key row
  constexpr int TILE = 64 * HD;                   // bytes of one 64-key tile
  constexpr int W = 4 * HPW;                      // waves of the workgroup
  constexpr int KS = TILE / 16 / W;               // 16-byte slots of a tile per wave
  constexpr int KD = KS >= 64 ? KS / 64 : 1;      // K DMAs per wave and tile
  constexpr int KL = KS >= 64 ? 64 : KS;          // lanes active in each
  constexpr int SL = 64 / W;                      // key scales per wave and tile
  constexpr int NW = (NS - 2) * (KD + 1);         // DMAs of the tiles a wait leaves in flight
  static_assert(KS >= 1 && SL >= 1 && KD * KL * W * 16 == TILE, "tile split over the waves");
  __shared__ __attribute__((aligned(16))) u8 kring[NS][TILE];
  __shared__ __attribute__((aligned(16))) float sring[NS][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ql = lane & 15, g = lane >> 4;
  int qt, hg, bseq;
  at_block((int)blockIdx.x, Tp / 64, H / HPW, Hkv, (int)(gridDim.x / (u32)(Tp / 64 * (H / HPW))), qt, hg, bseq);
  // every wave runs every tile and barrier (a wave past T computes clamped rows and stores nothing)
  const int h = hg * HPW + (wave >> 2);
  const int q0 = qt * 64 + (wave & 3) * 16;
  const int hk = h / (H / Hkv);
  const u32 nb = (u32)(bseq * T);
  const int qi = q0 + ql, qc = min(qi, T - 1);
  const float my_qs = qs[(nb + qc) * (u32)H + h];
  v4i qf[NC];
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const int d0 = 64 * c + 16 * g;
    qf[c] = d0 < HD ? *reinterpret_cast<const v4i*>(qq + ((nb + qc) * (u32)H + h) * HD + d0) : at_zero4();
  }
  // the compiler waits for these loads here (asm inputs), so that it places no vmcnt wait for them
  // inside the tile loop, where any vmcnt wait would also drain the ring's DMAs
#pragma unroll
  for (int c = 0; c < NC; c++) asm volatile("" ::"v"(qf[c]));
  asm volatile("" ::"v"(my_qs));
  const int nkt = qt + 1;  // key tiles 0 .. qt; tile qt holds the diagonal
  const i8* kbase = kq + (size_t)hk * HD;
  const u32 sc_base = nb * (u32)Hkv + hk;
  const u32 kr0 = (u32)(uintptr_t)(s2_lptr_at)kring[0], sr0 = (u32)(uintptr_t)(s2_lptr_at)sring[0];
  auto issue = [&](int kt) AT_AI {
    const int st = kt % NS;
#pragma unroll
    for (int u = 0; u < KD; u++) {
      const int s16 = (wave * KD + u) * KL + lane;  // 16-byte slot of the tile
      const int m = s16 / PR, p = (s16 % PR) ^ at_swz<HD>(m);
      const i8* src = kbase + (nb + (u32)min(kt * 64 + m, T - 1)) * (u32)(Hkv * HD) + 16 * p;
      const u32 dst = __builtin_amdgcn_readfirstlane(kr0 + (u32)(st * TILE + (wave * KD + u) * KL * 16));
      if (KL == 64 || lane < KL) at_dma16(src, dst);
    }
    const float* ssrc = ks + sc_base + (u32)min(kt * 64 + wave * SL + (lane & (SL - 1)), T - 1) * (u32)Hkv;
    const u32 sdst = __builtin_amdgcn_readfirstlane(sr0 + (u32)(st * 256 + wave * SL * 4));
    if (lane < SL) at_dma4(ssrc, sdst);
  };
#pragma unroll
  for (int t = 0; t < NS - 1; t++)
    if (t < nkt) issue(t);
  float mx = -__int_as_float(0x7f800000);
  for (int kt = 0; kt < nkt; kt++) {
    if (kt + NS - 2 < nkt) at_waitv<NW>();
    else at_waitv<0>();
    at_lds_barrier();  // tile kt is in LDS; every wave is done with tile kt - 1's stage
    if (kt + NS - 1 < nkt) issue(kt + NS - 1);
    const int st = kt % NS;
    const u8* tile = kring[st];
    float4 skv[4];
#pragma unroll
    for (int b = 0; b < 4; b++) skv[b] = *reinterpret_cast<const float4*>(&sring[st][16 * b + 4 * g]);
    // tiles below qt hold only keys below the wave's first query: no mask; tile qt masks
    auto tile_max = [&](auto mask) AT_AI {
#pragma unroll
      for (int b = 0; b < 4; b++) {
        v4i acc = at_zero4();
        const int m = 16 * b + ql;
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const int p = 4 * c + g;
          const v4i kf =
              p < PR ? *reinterpret_cast<const v4i*>(tile + 16 * (m * PR + (p ^ at_swz<HD>(m)))) : at_zero4();
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, qf[c], acc, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float y = __fmul_rn(__fmul_rn((float)acc[i], my_qs), at_get(skv[b], i));
          if constexpr (decltype(mask)::value) {
            const int j = kt * 64 + 16 * b + 4 * g + i;
            mx = fmaxf(mx, (j <= qi && j < T) ? y : -__int_as_float(0x7f800000));
          } else {
            mx = fmaxf(mx, y);
          }
        }
      }
    };
    if (kt < qt) tile_max(std::false_type{});
    else tile_max(std::true_type{});
  }
  mx = at_max_groups(mx);
  if (g == 0 && qi < T) rmax[(nb + qi) * (u32)H + h] = mx;
}

// The scratch of uwc_attention_ws: the exponentials' tiles, then the row maxima (one float per
// query and head) from a 256-byte boundary.
static u64 at_exp_bytes(int B, int T, int H) {
  const u64 Tp = ((u64)T + 63) / 64 * 64;
  return (u64)B * (u64)H * at_tiles(Tp) * 4096;
}

extern "C" uint64_t uwc_attention_scratch_bytes(int B, int T, int H) {
  if (B <= 0 || T <= 0 || H <= 0) return 0;
  return at_exp_bytes(B, T, H) + ((u64)B * (u64)T * (u64)H * 4 + 255) / 256 * 256;
}

static int attention_go(const char* fn, const int8_t* qq, const float* qs, const int8_t* kq, const float* ks,
                        const int8_t* vt, const float* vs, int B, int T, int H, int Hkv, int hd, float inv_sqrt_hd,
                        float* o, float* escratch, uint64_t escratch_bytes, hipStream_t stream) {
  if (!qq || !qs || !kq || !ks || !vt || !vs || !o) return uwc_fail("%s: null arguments", fn);
  if (B < 0 || T <= 0 || T > 131072 || H <= 0 || Hkv <= 0 || H % Hkv)
    return uwc_fail("%s: bad B=%d T=%d H=%d Hkv=%d (T <= 131072)", fn, B, T, H, Hkv);
  if (hd != 32 && hd != 64 && hd != 128) return uwc_fail("%s: head_dim %d not in {32, 64, 128}", fn, hd);
  if (((uintptr_t)qq | (uintptr_t)kq | (uintptr_t)vt) & 15) return uwc_fail("%s: qq, kq, vt must be 16-byte aligned", fn);
  if ((uintptr_t)o & 15) return uwc_fail("%s: o must be 16-byte aligned", fn);
  if (B == 0) return UWC_OK;
  if (B > 65535 || H > 65535) return uwc_fail("%s: B and H must be <= 65535", fn);
  if ((int64_t)B * T * (H > Hkv ? H : Hkv) * hd >= (1LL << 31))
    return uwc_fail("%s: B * T * H * hd must be below 2^31 (32-bit offsets)", fn);
  const int Tp = ((T + 63) / 64) * 64;
  const dim3 grid((unsigned)((long)(Tp / 64) * H * B));
  if (escratch) {
    if (escratch_bytes < uwc_attention_scratch_bytes(B, T, H))
      return uwc_fail("%s: escratch holds %llu bytes, %llu needed", fn, (unsigned long long)escratch_bytes,
                      (unsigned long long)uwc_attention_scratch_bytes(B, T, H));
    if ((uintptr_t)escratch & 15) return uwc_fail("%s: escratch must be 16-byte aligned", fn);
  }
  // with the scratch: sweep 1 (the row maxima) a launch, sweeps 2-4 another
  float* rows = escratch ? escratch + at_exp_bytes(B, T, H) / 4 : nullptr;
  // the row max's workgroups take HPW heads of one kv head (4, 2 or 1 of its G = H / Hkv)
  const int G = H / Hkv, hpw = G % 4 == 0 ? 4 : G % 2 == 0 ? 2 : 1;
  auto go = [&](auto hdc, auto esc) {
    constexpr int HDV = decltype(hdc)::value;
    if constexpr (decltype(esc)::value) {
      auto rowmax = [&](auto hp) {
        constexpr int HP = decltype(hp)::value;
        const dim3 rgrid((unsigned)((long)(Tp / 64) * (H / HP) * B));
        hipLaunchKernelGGL((attn_rowmax_kernel<HDV, 4, HP>), rgrid, dim3(256 * HP), 0, stream, qq, qs, kq, ks, T, Tp,
                           H, Hkv, rows);
      };
      if (hpw == 4) rowmax(std::integral_constant<int, 4>{});
      else if (hpw == 2) rowmax(std::integral_constant<int, 2>{});
      else rowmax(std::integral_constant<int, 1>{});
      hipLaunchKernelGGL((attention_kernel<HDV, true>), grid, dim3(256), 0, stream, qq, qs, kq, ks, vt, vs, T, Tp, H,
                         Hkv, inv_sqrt_hd, o, escratch, rows);
    } else {
      hipLaunchKernelGGL((attention_kernel<HDV, false>), grid, dim3(256), 0, stream, qq, qs, kq, ks, vt, vs, T, Tp,
                         H, Hkv, inv_sqrt_hd, o, nullptr, nullptr);
    }
  };
  auto go_hd = [&](auto esc) {
    if (hd == 32) go(std::integral_constant<int, 32>{}, esc);
    else if (hd == 64) go(std::integral_constant<int, 64>{}, esc);
    else go(std::integral_constant<int, 128>{}, esc);
  };
  if (escratch) go_hd(std::true_type{});
  else go_hd(std::false_type{});
  return uwc_launch_status(fn);
}

extern "C" int uwc_attention(const int8_t* qq, const float* qs, const int8_t* kq, const float* ks, const int8_t* vt,
                             const float* vs, int B, int T, int H, int Hkv, int hd, float inv_sqrt_hd, float* o,
                             hipStream_t stream) {
  return attention_go("uwc_attention", qq, qs, kq, ks, vt, vs, B, T, H, Hkv, hd, inv_sqrt_hd, o, nullptr, 0, stream);
}

extern "C" int uwc_attention_ws(const int8_t* qq, const float* qs, const int8_t* kq, const float* ks,
                                const int8_t* vt, const float* vs, int B, int T, int H, int Hkv, int hd,
                                float inv_sqrt_hd, float* o, float* escratch, uint64_t escratch_bytes,
                                hipStream_t stream) {
  if (!escratch) return uwc_fail("uwc_attention_ws: null escratch");
  return attention_go("uwc_attention_ws", qq, qs, kq, ks, vt, vs, B, T, H, Hkv, hd, inv_sqrt_hd, o, escratch,
                      escratch_bytes, stream);
}
