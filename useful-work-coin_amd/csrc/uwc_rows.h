// Row-wise exact fp32 helpers for the detrt decoder-layer kernels on gfx950: detrt's det_exp,
// SiLU, the exact fixed-point row sum behind RMSNorm, the block Walsh-Hadamard + symmetric
// quantizer, and wave / workgroup reductions (runtime/detrt/core.py:77-193; GPU twins
// runtime/detgpu/kernels.py:17-74).
//
// Every fp32 step is one correctly rounded IEEE operation in the reference's order
// (__fadd_rn/__fsub_rn/__fmul_rn/__fdiv_rn/uwc_sqrt_rn, never contracted; the library builds with
// -ffp-contract=off and keeps denormals). Integer and fixed-point sums are exact, so their order
// and the lane / workgroup split cannot change a bit.
#pragma once
#include "uwc_common.h"
#include "uwc_fwht.h"

// detrt's float32 constants (core.py:101-105), rounded once from the float64 literals.
#define DX_LOG2E 0x1.715476p+0f
#define DX_E0 0x1.0p+0f
#define DX_E1 0x1.62e43p-1f
#define DX_E2 0x1.ebfbdp-3f
#define DX_E3 0x1.c6b2acp-5f
#define DX_E4 0x1.3b0872p-7f
#define DX_E5 0x1.5fdb08p-10f
#define DX_E6 0x1.2d0dd8p-13f
#define DX_E7 0x1.6889f4p-16f

// det_exp (core.py:108-126): 2**t with t = z log2(e) split into floor and fraction, the
// fraction's power from a fixed degree-7 Horner polynomial (one rounding per op).
__device__ __forceinline__ float dx_exp(float z) {
  float t = __fmul_rn(z, DX_LOG2E);
  const bool under = t < -126.0f, over = t >= 128.0f;
  if (under || over || __builtin_isnan(t)) t = 0.0f;
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
  float r = __fmul_rn(p, __int_as_float(((int)n + 127) << 23));
  if (under) r = 0.0f;
  if (over) r = __int_as_float(0x7f800000);
  if (__builtin_isnan(z)) r = z;
  return r;
}

// det_silu (core.py:144-146): x / (1 + det_exp(-x)).
__device__ __forceinline__ float dx_silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, dx_exp(-x))); }

// detrt dequant fmul(fmul(f32(acc), s_row), s_col) (qwen3.py:125).
__device__ __forceinline__ float dx_deq(int acc, float s, float sw) { return __fmul_rn(__fmul_rn((float)acc, s), sw); }

// ceil(log2(n)) for n >= 1, at least 1 (core.py:84).
__host__ __device__ __forceinline__ int dx_log2ceil(int n) {
  int L = 0;
  while ((1 << L) < n) L++;
  return L < 1 ? 1 : L;
}

// exact_rowsum's fixed-point scale (core.py:84-90): 2**(e-1) <= amax < 2**e, shift = (62 - L) - e.
__device__ __forceinline__ int dx_shift(float amax, int L) {
  int e;
  frexpf(amax, &e);
  int sh = (62 - L) - e;
  return sh < -1000 ? -1000 : (sh > 1000 ? 1000 : sh);
}

// One term round_half_even(v * 2**sh) as int64 (exact: the scaling is a power of two).
__device__ __forceinline__ long long dx_fix(float v, int sh) {
  return (long long)rint(ldexp((double)v, sh));
}

// float32(float64(sum) * 2**-sh): the int64 sum rounded once to float64, scaled exactly,
// rounded once to float32 (core.py:95-97).
__device__ __forceinline__ float dx_unfix(long long s, int sh) { return (float)ldexp((double)s, -sh); }

// ------------------------------------------------------------------ wave reductions (wave64)
// Every lane gets the wave's max / sum; the wave must be fully active. Inside each 16-lane row the
// partners come through DPP operands (quad_perm [1,0,3,2], [2,3,0,1]: the quad; row_ror:4, 8: the
// four quads), across rows from v_permlane16_swap and v_permlane32_swap (each lane receives its
// pair's lower and upper value): VALU operations only, where __shfl_xor went through the LDS
// crossbar (ds_bpermute) with an LDS round trip per step. A max and an integer sum are the same
// in any order.
// wave_max: uwc_fwht.h

template <int CTRL>
__device__ __forceinline__ long long dpp64(long long x) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)x, CTRL, 0xF, 0xF, true);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(x >> 32), CTRL, 0xF, 0xF, true);
  return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}

__device__ __forceinline__ long long wave_sum64(long long v) {
  v += dpp64<0xB1>(v);
  v += dpp64<0x4E>(v);
  v += dpp64<0x124>(v);
  v += dpp64<0x128>(v);
#pragma unroll
  for (int s = 0; s < 2; s++) {
    const u32 lo = (u32)v, hi = (u32)((unsigned long long)v >> 32);
    const auto l = s ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false) : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = s ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false) : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = (long long)(((unsigned long long)h[0] << 32) | l[0]) + (long long)(((unsigned long long)h[1] << 32) | l[1]);
  }
  return v;
}

// The max and the int64 sum over each 16-lane row (the first four steps of wave_max and
// wave_sum64), in every lane of the row; rows reduce independently of each other.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, qa_dpp<0xB1>(v));
  v = fmaxf(v, qa_dpp<0x4E>(v));
  v = fmaxf(v, qa_dpp<0x124>(v));
  return fmaxf(v, qa_dpp<0x128>(v));
}

__device__ __forceinline__ long long row16_sum64(long long v) {
  v += dpp64<0xB1>(v);
  v += dpp64<0x4E>(v);
  v += dpp64<0x124>(v);
  return v + dpp64<0x128>(v);
}

// ------------------------------------------------------------------ workgroup (256 threads) reductions
struct DxRed {
  float f[4];
  long long l[4];
};

__device__ __forceinline__ float block_max256(float v, DxRed& red) {
  v = wave_max(v);
  __syncthreads();  // red may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) red.f[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red.f[0], red.f[1]), fmaxf(red.f[2], red.f[3]));
}

__device__ __forceinline__ long long block_sum256(long long v, DxRed& red) {
  v = wave_sum64(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red.l[threadIdx.x >> 6] = v;
  __syncthreads();
  return red.l[0] + red.l[1] + red.l[2] + red.l[3];
}

// det_rmsnorm in place on an LDS row (core.py:149-156): row[i] = (row[i] * r) * w[i],
// r = 1 / sqrt(exact_rowsum(row^2) / k + eps). 256 threads.
__device__ __forceinline__ void dx_rmsnorm_lds(float* row, int k, const float* __restrict__ w, float inv_d, float eps,
                                               DxRed& red) {
  const int tid = threadIdx.x;
  float mx = 0.f;
  for (int i = tid; i < k; i += 256) mx = fmaxf(mx, __fmul_rn(row[i], row[i]));
  mx = block_max256(mx, red);
  const int sh = dx_shift(mx, dx_log2ceil(k));
  long long acc = 0;
  for (int i = tid; i < k; i += 256) acc += dx_fix(__fmul_rn(row[i], row[i]), sh);
  acc = block_sum256(acc, red);
  const float ss = dx_unfix(acc, sh);
  const float r = __fdiv_rn(1.0f, uwc_sqrt_rn(__fadd_rn(__fmul_rn(ss, inv_d), eps)));
  for (int i = tid; i < k; i += 256) row[i] = __fmul_rn(__fmul_rn(row[i], r), w[i]);
  __syncthreads();
}

// dx_quant_lds for k % 512 == 0 and 1 <= bs = 2^lbs <= 512: each wave takes the 512-element groups
// g = wave, wave + 4, ... of the LDS row, transforms them in registers (fwht512_rows: the same
// adds and subtracts in the same order, so the same bits) and writes them back; after the row's
// max the wave quantizes its own groups, 8 elements per lane and one 8-byte store. Nine LDS
// passes with a barrier each become one read and one write.
__device__ __forceinline__ void dx_quant_lds_g(float* row, int k, int lbs, int qmax, i8* __restrict__ q,
                                               float* __restrict__ scale, DxRed& red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, G = k >> 9;
  float mx = 0.f;
  bool neg = false;  // the lane holds its groups' transform negated (the same sign for each)
  for (int g = wave; g < G; g += 4) {
    float4* p = reinterpret_cast<float4*>(row + g * 512 + lane * 8);
    const float4 a = p[0], b = p[1];
    float y[1][8] = {{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w}};
    neg = fwht512_rows<1>(y, 1, lane, lbs);
#pragma unroll
    for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(y[0][j]));
    p[0] = float4{y[0][0], y[0][1], y[0][2], y[0][3]};
    p[1] = float4{y[0][4], y[0][5], y[0][6], y[0][7]};
  }
  mx = block_max256(mx, red);
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(mx, 1e-8f), fq);
  // the lane reads back what it wrote: y / s = w * (+-1 / s)
  const double rs = neg ? -1.0 / (double)s : 1.0 / (double)s;
  for (int g = wave; g < G; g += 4) {
    const float4* p = reinterpret_cast<const float4*>(row + g * 512 + lane * 8);
    const float4 a = p[0], b = p[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    u64 packed = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float t = fminf(fmaxf(rintf(uwc_div_rd(v[j], rs)), -fq), fq);
      packed |= (u64)(u8)(i8)(int)t << (8 * j);
    }
    *reinterpret_cast<u64*>(q + g * 512 + lane * 8) = packed;
  }
  if (threadIdx.x == 0) *scale = lbs > 0 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)(1 << lbs)))) : s;
}

// quant_act on an LDS row (core.py:169-193): block FWHT of size bs (stages h = 1, 2, 4, ...,
// pairs (i, i+h) -> (a+b, a-b)), s = max(max|y|, 1e-8) / qmax, q = clamp(rint(y / s)), scale
// s * (1 / sqrt(bs)) when bs > 1. 256 threads; the row must be complete in LDS (barrier done).
__device__ __forceinline__ void dx_quant_lds(float* row, int k, int bs, int qmax, i8* __restrict__ q,
                                             float* __restrict__ scale, DxRed& red) {
  const int tid = threadIdx.x;
  if (bs > 1) {
    for (int lh = 0; (1 << lh) < bs; lh++) {
      const int h = 1 << lh;
      for (int p = tid; p < (k >> 1); p += 256) {
        const int i = ((p >> lh) << (lh + 1)) | (p & (h - 1)), j = i + h;
        const float a = row[i], b = row[j];
        row[i] = __fadd_rn(a, b);
        row[j] = __fsub_rn(a, b);
      }
      __syncthreads();
    }
  }
  float mx = 0.f;
  for (int i = tid; i < k; i += 256) mx = fmaxf(mx, fabsf(row[i]));
  mx = block_max256(mx, red);
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(mx, 1e-8f), fq);
  const double rs = 1.0 / (double)s;
  for (int i = tid; i < k; i += 256) {
    const float v = fminf(fmaxf(rintf(uwc_div_rd(row[i], rs)), -fq), fq);
    q[i] = (i8)(int)v;
  }
  if (tid == 0) *scale = bs > 1 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)bs))) : s;
}
