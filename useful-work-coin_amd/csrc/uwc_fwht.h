// The block Walsh-Hadamard transform of 512-element groups held in registers (lane L holds
// elements 8 L .. 8 L + 7 of a group), shared by the activation quantizer (uwc_quant.hip) and the
// quantizing row kernels (uwc_rows.h): stages h = 1, 2, 4 pair elements inside a lane, stages
// h = 8 .. 256 pair lane L with lane L ^ (h / 8). Each output of a stage is one rounded add or
// subtract of the same two inputs, in the same stage order, as the LDS form (pairs (i, i + h) ->
// (a + b, a - b)), so the results are the same bits.
#pragma once
#include "uwc_common.h"

// The transform of G (<= NG) groups held as y[g][0..7], stage-major over the groups so that every
// stage's cross-lane exchanges are independent of each other; every lane of the wave must be
// active. The exchanges run on the VALU:
// DPP quad_perm for lane ^ 1 and ^ 2, DPP row rotations for ^ 4 (row_ror:12 reads lane + 4,
// row_ror:4 lane - 4, inside 16-lane rows) and ^ 8 (row_ror:8), and v_permlane16_swap /
// v_permlane32_swap for ^ 16 and ^ 32, which hand every lane both values of its pair (the lower
// lane's in the first result, the upper's in the second).
template <int CTRL>
__device__ __forceinline__ float qa_dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}

template <int NG>
__device__ __forceinline__ void fwht512_rows(float y[NG][8], int G, int lane, int lbs) {
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
  // lane ^ 1, 2, 4, 8: the partner's value o; the lower lane keeps v + o, the upper o - v
#pragma unroll
  for (int lh = 3; lh < 7; lh++) {
    if (lh < lbs) {
      const int d = 1 << (lh - 3);
      const bool hi = lane & d;
#pragma unroll
      for (int g = 0; g < NG; g++)
        if (g < G) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            // every lane runs every exchange (a DPP read of a lane outside EXEC returns the bound
            // value, not the lane's), then selects: no branch may depend on hi before this point
            const float v = y[g][j];
            float o;
            if (d == 1) {
              o = qa_dpp<0xB1>(v);  // quad_perm [1,0,3,2]
            } else if (d == 2) {
              o = qa_dpp<0x4E>(v);  // quad_perm [2,3,0,1]
            } else if (d == 4) {
              const float up = qa_dpp<0x12C>(v), down = qa_dpp<0x124>(v);  // row_ror:12 / row_ror:4
              o = hi ? down : up;
            } else {
              o = qa_dpp<0x128>(v);  // row_ror:8
            }
            const float sum = __fadd_rn(v, o), dif = __fsub_rn(o, v);
            y[g][j] = hi ? dif : sum;
          }
        }
    }
  }
  // lane ^ 16, 32: the swap gives the pair's lower value a and upper value b in every lane
#pragma unroll
  for (int lh = 7; lh < 9; lh++) {
    if (lh < lbs) {
      const bool hi = lane & (1 << (lh - 3));
#pragma unroll
      for (int g = 0; g < NG; g++)
        if (g < G) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            const u32 v = __float_as_uint(y[g][j]);
            const auto ab = lh == 7 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                                    : __builtin_amdgcn_permlane32_swap(v, v, false, false);
            const float a = __uint_as_float(ab[0]), b = __uint_as_float(ab[1]);
            const float sum = __fadd_rn(a, b), dif = __fsub_rn(a, b);
            y[g][j] = hi ? dif : sum;
          }
        }
    }
  }
}


// ------------------------------------------------------------------ the 16-per-lane layout
// A wave holds two 512-element groups, lane bit 2 choosing the group; inside a group, lane L
// holds the 16 consecutive elements 16 i .. 16 i + 15 with i = b0 + 2 b1 + 4 b3 + 8 b4 + 16 b5
// (b = the bits of L). Stages h = 1, 2, 4, 8 then pair elements inside a lane, and stages
// h = 16 .. 256 pair lane L with L ^ 1, ^ 2, ^ 8, ^ 16, ^ 32: lane bit 2, the one exchange the
// VALU cannot do in one DPP operand, is never crossed. A cross-lane stage is one sign flip and
// one add per element: the lower lane of a pair computes o + v = v + o (a + b), the upper one
// o + (-v) = o - v (a - b), the same single rounded IEEE operation on the same two operands as
// the reference's pair (a + b, a - b), with the partner's value o read through a DPP operand of
// the add (or exchanged by v_permlane16/32_swap).
__device__ __forceinline__ int fw16_index(int lane) {
  return (lane & 3) | ((lane >> 1) & 0x1C);  // b0 + 2 b1 + 4 b3 + 8 b4 + 16 b5
}

// y[0..15]: the lane's elements of one double group; lbs = log2(bs), bs <= 512. Every lane of the
// wave must be active.
__device__ __forceinline__ void fwht16(float y[16], int lane, int lbs) {
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
  // stages h = 16, 32, 64 (lane bits 0, 1, 3): DPP quad_perm [1,0,3,2], [2,3,0,1], row_ror:8
#pragma unroll
  for (int lh = 4; lh < 7; lh++) {
    if (lh < lbs) {
      const int bit = lh == 4 ? 0 : lh == 5 ? 1 : 3;
      const u32 sgn = (lane >> bit) & 1 ? 0x80000000u : 0u;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const float v = y[j];
        const float sv = __uint_as_float(__float_as_uint(v) ^ sgn);
        const float o = lh == 4 ? qa_dpp<0xB1>(v) : lh == 5 ? qa_dpp<0x4E>(v) : qa_dpp<0x128>(v);
        y[j] = __fadd_rn(o, sv);
      }
    }
  }
  // stages h = 128, 256 (lane bits 4, 5): the swap hands every lane both values of its pair
#pragma unroll
  for (int lh = 7; lh < 9; lh++) {
    if (lh < lbs) {
      const u32 sgn = (lane >> (lh - 3)) & 1 ? 0x80000000u : 0u;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const u32 v = __float_as_uint(y[j]);
        const auto ab = lh == 7 ? __builtin_amdgcn_permlane16_swap(v, v, false, false)
                                : __builtin_amdgcn_permlane32_swap(v, v, false, false);
        // lower lane: a + b; upper lane: a + (-b)
        y[j] = __fadd_rn(__uint_as_float(ab[0]), __uint_as_float(ab[1] ^ sgn));
      }
    }
  }
}
