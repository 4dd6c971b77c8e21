// The block Walsh-Hadamard transform of 512-element groups held in registers (lane L holds
// elements 8 L .. 8 L + 7 of a group), shared by the activation quantizer (uwc_quant.hip) and the
// quantizing row kernels (uwc_rows.h): stages h = 1, 2, 4 pair elements inside a lane, stages
// h = 8 .. 256 pair lane L with lane L ^ (h / 8). Each output of a stage is one rounded add or
// subtract of the same two inputs, in the same stage order, as the LDS form (pairs (i, i + h) ->
// (a + b, a - b)), so the results are the same bits up to a per-lane sign the transforms return.
#pragma once
#include "uwc_common.h"

// The transform of G (<= NG) groups held as y[g][0..7], stage-major over the groups so that every
// stage's cross-lane exchanges are independent of each other; every lane of the wave must be
// active. Cross-lane stages, by lane bit (the pair of lanes L < U, a the value of L, b of U):
//   * bits 0, 1, 3 (h = 8, 16, 64): one v_fmac_f32 per element, w += c o with the partner's value
//     o through a DPP operand (quad_perm [1,0,3,2], [2,3,0,1], row_ror:8) and c = +1 in L, -1 in
//     U, under a per-lane sign as in the 16-per-lane form below: L gets s (a + b), U
//     s (b - a) = -s (a - b), and U's sign flips;
//   * bit 2 (h = 32): a DPP add in L (partner L + 4: row_ror:12, banks 0 and 2 of each row) and a
//     DPP subtract in U (partner U - 4: row_ror:4, banks 1 and 3) writing one new register, the
//     bank mask leaving the other lanes' value: a + b and a - b with no sign change;
//   * bits 4, 5 (h = 128, 256): v_permlane16/32_swap hands every lane a and b, then a + c b.
// The pair of every stage shares its sign (the sign depends on bits 0, 1, 3 only), c o is exact,
// and rounding to nearest is symmetric: every value is the reference's single rounded a + b or
// a - b, up to the lane's sign, which is returned (true: the lane holds the negated transform).
template <int CTRL>
__device__ __forceinline__ float qa_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

// The max over a fully active wave, in every lane: DPP partners inside each 16-lane row
// (quad_perm [1,0,3,2], [2,3,0,1], then row_ror:4 and :8 over the quads), v_permlane16_swap and
// v_permlane32_swap across rows; VALU operations only (a __shfl_xor step is an LDS round trip).
// A max is the same in any order.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, qa_dpp<0xB1>(v));
  v = fmaxf(v, qa_dpp<0x4E>(v));
  v = fmaxf(v, qa_dpp<0x124>(v));
  v = fmaxf(v, qa_dpp<0x128>(v));
  u32 u = __float_as_uint(v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  u = __float_as_uint(v);
  const auto b = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// w[j] += c * w[j] of the DPP partner lane for the 8 values of one group; s_nop 4 covers the wait
// states of a DPP read after a VALU (or EXEC) write of its source, whatever precedes the block
#define FW8_FMAC_STAGE(w, DPP)                                                                              \
  asm("s_nop 4\n\t"                                                                                         \
      "v_fmac_f32_dpp %0, %0, %8 " DPP "\n\tv_fmac_f32_dpp %1, %1, %8 " DPP "\n\t"                         \
      "v_fmac_f32_dpp %2, %2, %8 " DPP "\n\tv_fmac_f32_dpp %3, %3, %8 " DPP "\n\t"                         \
      "v_fmac_f32_dpp %4, %4, %8 " DPP "\n\tv_fmac_f32_dpp %5, %5, %8 " DPP "\n\t"                         \
      "v_fmac_f32_dpp %6, %6, %8 " DPP "\n\tv_fmac_f32_dpp %7, %7, %8 " DPP                                \
      : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]), "+v"(w[4]), "+v"(w[5]), "+v"(w[6]), "+v"(w[7])      \
      : "v"(c))

// n[j] = w[j] + w[j + 4 lanes] in banks 0, 2 and w[j - 4 lanes] - w[j] in banks 1, 3 of every row
__device__ __forceinline__ void fw8_lane4(const float w[8], float n[8]) {
  asm("s_nop 4\n\t"
      "v_add_f32_dpp %0, %8, %8 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %0, %8, %8 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %1, %9, %9 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %1, %9, %9 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %2, %10, %10 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %2, %10, %10 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %3, %11, %11 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %3, %11, %11 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %4, %12, %12 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %4, %12, %12 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %5, %13, %13 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %5, %13, %13 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %6, %14, %14 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %6, %14, %14 row_ror:4 row_mask:0xf bank_mask:0xa\n\t"
      "v_add_f32_dpp %7, %15, %15 row_ror:12 row_mask:0xf bank_mask:0x5\n\t"
      "v_sub_f32_dpp %7, %15, %15 row_ror:4 row_mask:0xf bank_mask:0xa"
      : "=&v"(n[0]), "=&v"(n[1]), "=&v"(n[2]), "=&v"(n[3]), "=&v"(n[4]), "=&v"(n[5]), "=&v"(n[6]), "=&v"(n[7])
      : "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3]), "v"(w[4]), "v"(w[5]), "v"(w[6]), "v"(w[7]));
}

template <int NG>
__device__ __forceinline__ bool fwht512_rows(float y[NG][8], int G, int lane, int lbs) {
#pragma unroll
  for (int lh = 0; lh < 3; lh++) {
    if (lh < lbs) {
      const int h = 1 << lh;
#pragma unroll
      for (int g = 0; g < NG; g++)
        if (g < G) {
#pragma unroll
          for (int j = 0; j < 8; j++)
            if (!(j & h)) {
              const float a = y[g][j], b = y[g][j + h];
              y[g][j] = __fadd_rn(a, b);
              y[g][j + h] = __fsub_rn(a, b);
            }
        }
    }
  }
  bool neg = false;
#pragma unroll
  for (int lh = 3; lh < 7; lh++) {
    if (lh < lbs) {
      if (lh == 5) {
#pragma unroll
        for (int g = 0; g < NG; g++)
          if (g < G) {
            float n[8];
            fw8_lane4(y[g], n);
#pragma unroll
            for (int j = 0; j < 8; j++) y[g][j] = n[j];
          }
      } else {
        const int bit = (lane >> (lh - 3)) & 1;
        const float c = bit ? -1.0f : 1.0f;
#pragma unroll
        for (int g = 0; g < NG; g++)
          if (g < G) {
            if (lh == 3) FW8_FMAC_STAGE(y[g], "quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf");
            else if (lh == 4) FW8_FMAC_STAGE(y[g], "quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf");
            else FW8_FMAC_STAGE(y[g], "row_ror:8 row_mask:0xf bank_mask:0xf");
          }
        neg ^= bit;
      }
    }
  }
#pragma unroll
  for (int lh = 7; lh < 9; lh++) {
    if (lh < lbs) {
      const float c = (lane >> (lh - 3)) & 1 ? -1.0f : 1.0f;
#pragma unroll
      for (int g = 0; g < NG; g++)
        if (g < G) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const u32 v = __float_as_uint(y[g][j]);
            const auto ab = lh == 7 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                                    : __builtin_amdgcn_permlane32_swap(v, v, false, false);
            y[g][j] = __builtin_fmaf(__uint_as_float(ab[1]), c, __uint_as_float(ab[0]));
          }
        }
    }
  }
  return neg;
}


// ------------------------------------------------------------------ the 16-per-lane layout
// A wave holds two 512-element groups, lane bit 2 choosing the group; inside a group, lane L
// holds the 16 consecutive elements 16 i .. 16 i + 15 with i = b0 + 2 b1 + 4 b3 + 8 b4 + 16 b5
// (b = the bits of L). Stages h = 1, 2, 4, 8 then pair elements inside a lane, and stages
// h = 16 .. 256 pair lane L with L ^ 1, ^ 2, ^ 8, ^ 16, ^ 32: lane bit 2, the one exchange the
// VALU cannot do in one DPP operand, is never crossed.
//
// A cross-lane stage is one VALU operation per element. Each lane holds its values times a sign
// s (+1 or -1, the same for all 16 of them and for both lanes of every pair still to be
// exchanged), so that the one operation w' = w + c o (w the lane's value, o the partner's, c = +1
// in the lower lane of the pair, -1 in the upper) serves both lanes: the lower lane gets
// s (a + b), the upper s (b - a) = -s (a - b), i.e. the pair (a + b, a - b) of the reference with
// the upper lane's sign flipped. c o is exact and rounding to nearest is symmetric, so each value
// is the reference's single rounded a + b or a - b, up to sign. For h = 16, 32, 64 the operation
// is v_fmac_f32 with the partner read through a DPP operand (quad_perm [1,0,3,2], [2,3,0,1],
// row_ror:8); for h = 128, 256 v_permlane16/32_swap hands every lane the pair's lower value a
// and upper value b, and every lane takes a + c b (no sign change). The sign is returned: the
// caller quantizes with a signed reciprocal (y / s = w * (sign / s) exactly) and takes |w| = |y|.
__device__ __forceinline__ int fw16_index(int lane) {
  return (lane & 3) | ((lane >> 1) & 0x1C);  // b0 + 2 b1 + 4 b3 + 8 b4 + 16 b5
}

// y[j] += c * y[j] of the DPP partner lane, for the 16 values of a lane. One asm block per stage:
// s_nop 4 covers the wait states a DPP read needs after a VALU write of its source (and after an
// EXEC write) whatever the compiler scheduled before the block; inside it every instruction reads
// and writes its own register only.
#define FW16_DPP_STAGE(DPP)                                                                                 \
  asm("s_nop 4\n\t"                                                                                         \
      "v_fmac_f32_dpp %0, %0, %16 " DPP "\n\tv_fmac_f32_dpp %1, %1, %16 " DPP "\n\t"                       \
      "v_fmac_f32_dpp %2, %2, %16 " DPP "\n\tv_fmac_f32_dpp %3, %3, %16 " DPP "\n\t"                       \
      "v_fmac_f32_dpp %4, %4, %16 " DPP "\n\tv_fmac_f32_dpp %5, %5, %16 " DPP "\n\t"                       \
      "v_fmac_f32_dpp %6, %6, %16 " DPP "\n\tv_fmac_f32_dpp %7, %7, %16 " DPP "\n\t"                       \
      "v_fmac_f32_dpp %8, %8, %16 " DPP "\n\tv_fmac_f32_dpp %9, %9, %16 " DPP "\n\t"                       \
      "v_fmac_f32_dpp %10, %10, %16 " DPP "\n\tv_fmac_f32_dpp %11, %11, %16 " DPP "\n\t"                   \
      "v_fmac_f32_dpp %12, %12, %16 " DPP "\n\tv_fmac_f32_dpp %13, %13, %16 " DPP "\n\t"                   \
      "v_fmac_f32_dpp %14, %14, %16 " DPP "\n\tv_fmac_f32_dpp %15, %15, %16 " DPP                          \
      : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]), "+v"(y[6]), "+v"(y[7]),     \
        "+v"(y[8]), "+v"(y[9]), "+v"(y[10]), "+v"(y[11]), "+v"(y[12]), "+v"(y[13]), "+v"(y[14]),          \
        "+v"(y[15])                                                                                         \
      : "v"(c))

// y[0..15]: the lane's elements of one double group; lbs = log2(bs), bs <= 512. Every lane of the
// wave must be active. Returns true when the lane holds the negated transform.
__device__ __forceinline__ bool fwht16(float y[16], int lane, int lbs) {
#pragma unroll
  for (int lh = 0; lh < 4; lh++) {
    if (lh < lbs) {
      const int h = 1 << lh;
#pragma unroll
      for (int j = 0; j < 16; j++)
        if (!(j & h)) {
          const float a = y[j], b = y[j + h];
          y[j] = __fadd_rn(a, b);
          y[j + h] = __fsub_rn(a, b);
        }
    }
  }
  bool neg = false;
  // stages h = 16, 32, 64 (lane bits 0, 1, 3)
#pragma unroll
  for (int lh = 4; lh < 7; lh++) {
    if (lh < lbs) {
      const int bit = (lane >> (lh == 4 ? 0 : lh == 5 ? 1 : 3)) & 1;
      const float c = bit ? -1.0f : 1.0f;
      if (lh == 4) FW16_DPP_STAGE("quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf");
      else if (lh == 5) FW16_DPP_STAGE("quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf");
      else FW16_DPP_STAGE("row_ror:8 row_mask:0xf bank_mask:0xf");
      neg ^= bit;
    }
  }
  // stages h = 128, 256 (lane bits 4, 5): both lanes of a pair hold the same sign here
#pragma unroll
  for (int lh = 7; lh < 9; lh++) {
    if (lh < lbs) {
      const float c = (lane >> (lh - 3)) & 1 ? -1.0f : 1.0f;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const u32 v = __float_as_uint(y[j]);
        const auto ab = lh == 7 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                                : __builtin_amdgcn_permlane32_swap(v, v, false, false);
        y[j] = __builtin_fmaf(__uint_as_float(ab[1]), c, __uint_as_float(ab[0]));
      }
    }
  }
  return neg;
}
