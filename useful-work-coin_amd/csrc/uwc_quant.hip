// detrt requant / dequant on gfx950, bit-identical to runtime/detrt/core.py:162-195 and
// runtime/detrt/qwen3.py:125 (GPU twins: runtime/detgpu/kernels.py:35, 75-114, 346-353).
//
// Every floating-point step is a single correctly rounded IEEE binary32 operation in the
// reference's order: __fadd_rn/__fsub_rn/__fmul_rn/__fdiv_rn/__fsqrt_rn are never contracted
// into fused multiply-adds, denormals are kept (no flush flags at build time), rintf rounds
// half to even, and max/abs/int->float conversions are exact or correctly rounded.
#include "uwc_common.h"

// One workgroup per row: the row is staged in LDS, transformed by the unnormalized block
// Walsh-Hadamard transform (stages h = 1, 2, 4, ... < bs; pairs (i, i+h) -> (a+b, a-b)),
// reduced to max|y|, then q = clamp(rint(y / s), -qmax, qmax), s = max(max|y|, 1e-8) / qmax,
// returned scale = s * (1 / sqrt(bs)) when bs > 1.
__global__ void __launch_bounds__(256) quant_act_kernel(const float* __restrict__ x, int k, int bs, int qmax,
                                                        i8* __restrict__ q, float* __restrict__ scale) {
  extern __shared__ float rowf[];
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const float* xr = x + (u64)row * k;
  for (int i = tid; i < k; i += 256) rowf[i] = xr[i];
  __syncthreads();
  if (bs > 1) {
    for (int lh = 0; (1 << lh) < bs; lh++) {
      const int h = 1 << lh;
      for (int p = tid; p < (k >> 1); p += 256) {
        const int i = ((p >> lh) << (lh + 1)) | (p & (h - 1)), j = i + h;
        const float a = rowf[i], b = rowf[j];
        rowf[i] = __fadd_rn(a, b);
        rowf[j] = __fsub_rn(a, b);
      }
      __syncthreads();
    }
  }
  float mx = 0.f;
  for (int i = tid; i < k; i += 256) mx = fmaxf(mx, fabsf(rowf[i]));
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) mx = fmaxf(mx, __shfl_xor(mx, s));
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(amax, 1e-8f), fq);
  i8* qr = q + (u64)row * k;
  for (int i = tid; i < k; i += 256) {
    const float v = fminf(fmaxf(rintf(__fdiv_rn(rowf[i], s)), -fq), fq);
    qr[i] = (i8)(int)v;
  }
  if (tid == 0) scale[row] = bs > 1 ? __fmul_rn(s, __fdiv_rn(1.0f, __fsqrt_rn((float)bs))) : s;
}

// y = (f32(acc) * sx[row]) * sw[col], each product rounded once (qwen3.py:125).
__global__ void dequant_kernel(const i32* __restrict__ acc, const float* __restrict__ sx, const float* __restrict__ sw,
                               int n, u64 total, float* __restrict__ y) {
  for (u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (u64)gridDim.x * blockDim.x) {
    const u64 r = i / (u64)n;
    const int c = (int)(i - r * n);
    y[i] = __fmul_rn(__fmul_rn((float)acc[i], sx[r]), sw[c]);
  }
}

extern "C" int uwc_quant_act_f32(const float* x, int rows, int k, int bs, int qmax, int8_t* q, float* scale,
                                 hipStream_t stream) {
  if (!x || !q || !scale || rows < 0 || k <= 0) return uwc_fail("uwc_quant_act_f32: null or empty arguments");
  if (bs > 1 && ((bs & (bs - 1)) || k % bs)) return uwc_fail("uwc_quant_act_f32: bs=%d must be a power of two dividing k=%d", bs, k);
  if (qmax < 1 || qmax > 127) return uwc_fail("uwc_quant_act_f32: qmax=%d outside 1..127", qmax);
  const size_t smem = (size_t)k * 4;
  if (smem > 160 * 1024) return uwc_fail("uwc_quant_act_f32: a row of k=%d floats exceeds LDS", k);
  if (rows == 0) return UWC_OK;
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)quant_act_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return uwc_fail("uwc_quant_act_f32: cannot raise LDS to %zu bytes: %s", smem, hipGetErrorString(e));
  }
  hipLaunchKernelGGL(quant_act_kernel, dim3(rows), dim3(256), smem, stream, x, k, bs, qmax, q, scale);
  return uwc_launch_status("quant_act");
}

extern "C" int uwc_dequant_f32(const int32_t* acc, const float* sx, const float* sw, int m, int n, float* y,
                               hipStream_t stream) {
  if (!acc || !sx || !sw || !y || m < 0 || n <= 0) return uwc_fail("uwc_dequant_f32: null or empty arguments");
  const u64 total = (u64)m * n;
  if (total == 0) return UWC_OK;
  const u64 blocks = (total + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream, acc, sx,
                     sw, n, total, y);
  return uwc_launch_status("dequant");
}
