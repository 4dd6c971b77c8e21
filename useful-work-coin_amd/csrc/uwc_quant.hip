// detrt requant / dequant on gfx950, bit-identical to runtime/detrt/core.py:162-195 and
// runtime/detrt/qwen3.py:125 (GPU twins: runtime/detgpu/kernels.py:35, 75-114, 346-353).
//
// Every floating-point step is a single correctly rounded IEEE binary32 operation in the
// reference's order: __fadd_rn/__fsub_rn/__fmul_rn/__fdiv_rn/uwc_sqrt_rn are never contracted
// into fused multiply-adds, denormals are kept (no flush flags at build time), rintf rounds
// half to even, and max/abs/int->float conversions are exact or correctly rounded.
#include "uwc_common.h"
#include "uwc_fwht.h"

// One workgroup per row: the row is staged in LDS, transformed by the unnormalized block
// Walsh-Hadamard transform (stages h = 1, 2, 4, ... < bs; pairs (i, i+h) -> (a+b, a-b)),
// reduced to max|y|, then q = clamp(rint(y / s), -qmax, qmax), s = max(max|y|, 1e-8) / qmax,
// returned scale = s * (1 / sqrt(bs)) when bs > 1.
// Input elements: fp32, or bf16 bit patterns widened exactly (bits << 16).
__device__ __forceinline__ float qa_in(const float* p, long i) { return p[i]; }
__device__ __forceinline__ float qa_in(const uint16_t* p, long i) { return __uint_as_float((u32)p[i] << 16); }

template <typename T>
__global__ void __launch_bounds__(256) quant_act_kernel(const T* __restrict__ x, int k, int bs, int qmax,
                                                        i8* __restrict__ q, float* __restrict__ scale) {
  extern __shared__ float rowf[];
  __shared__ float red[4];
  const int row = blockIdx.x, tid = threadIdx.x;
  const T* xr = x + (u64)row * k;
  for (int i = tid; i < k; i += 256) rowf[i] = qa_in(xr, i);
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
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(amax, 1e-8f), fq);
  const double rs = 1.0 / (double)s;
  i8* qr = q + (u64)row * k;
  for (int i = tid; i < k; i += 256) {
    const float v = fminf(fmaxf(rintf(uwc_div_rd(rowf[i], rs)), -fq), fq);
    qr[i] = (i8)(int)v;
  }
  if (tid == 0) scale[row] = bs > 1 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)bs))) : s;
}

// The same quant_act with one wave per row and no LDS: for k % 512 == 0 and bs <= 512. A row is
// processed in groups of 512 elements, lane L holding elements 8 L .. 8 L + 7 of a group as
// registers. Stages h = 1, 2, 4 pair elements inside a lane; stages h = 8 .. 256 pair lane L
// with lane L ^ (h / 8): the lane holding index i (bit h clear) keeps a + b, its partner
// keeps a - b, with a = y[i] and b = y[i + h]. Each output of a stage is one rounded add or
// subtract of the same two inputs as in the reference's stage order, so the result is
// bit-identical to the LDS form. With STASH the row's transformed values stay in registers
// (k <= 512 * QA_GMAX) and every load of the row is issued before the first transform, so a
// wave has its whole row in flight at once (one row per wave leaves few waves per SIMD at
// M = 2048: the loads, not the occupancy, must cover the memory latency); otherwise the
// quantizing pass reloads and transforms again.
#define QA_GMAX 16

// one group: the lane's sign is returned as by fwht512_rows
__device__ __forceinline__ bool fwht512(float v[8], int lane, int lbs) {
  return fwht512_rows<1>(reinterpret_cast<float(*)[8]>(v), 1, lane, lbs);
}

__device__ __forceinline__ void load8(const float* p, float v[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// 8 bf16 values (one 16-byte load), widened exactly to fp32
__device__ __forceinline__ void load8(const uint16_t* p, float v[8]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  const u32 w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[2 * j] = __uint_as_float(w[j] << 16);
    v[2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
  }
}

template <bool STASH, typename T>
__global__ void __launch_bounds__(256) quant_act_wave_kernel(const T* __restrict__ x, int rows, int k, int lbs,
                                                             int qmax, i8* __restrict__ q, float* __restrict__ scale) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole waves only; no barriers below
  const int G = k >> 9;
  const T* xr = x + (u64)row * k + lane * 8;
  float y[STASH ? QA_GMAX : 1][8];
  float mx = 0.f;
  bool neg = false;  // the lane holds the negated transform (the same for every group)
  if constexpr (STASH) {
#pragma unroll
    for (int g = 0; g < QA_GMAX; g++)
      if (g < G) load8(xr + g * 512, y[g]);
    neg = fwht512_rows<QA_GMAX>(y, G, lane, lbs);
#pragma unroll
    for (int g = 0; g < QA_GMAX; g++)
      if (g < G) {
#pragma unroll
        for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(y[g][j]));
      }
  } else {
    for (int g = 0; g < G; g++) {
      load8(xr + g * 512, y[0]);
      neg = fwht512(y[0], lane, lbs);
#pragma unroll
      for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(y[0][j]));
    }
  }
  mx = wave_max(mx);
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(mx, 1e-8f), fq);
  const double rs = neg ? -1.0 / (double)s : 1.0 / (double)s;  // y / s = w * (+-1 / s)
  i8* qr = q + (u64)row * k + lane * 8;
  auto emit = [&](const float v[8], int g) {
    u64 packed = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float t = fminf(fmaxf(rintf(uwc_div_rd(v[j], rs)), -fq), fq);
      packed |= (u64)(u8)(i8)(int)t << (8 * j);
    }
    *reinterpret_cast<u64*>(qr + g * 512) = packed;
  };
  if constexpr (STASH) {
#pragma unroll
    for (int g = 0; g < QA_GMAX; g++)
      if (g < G) emit(y[g], g);
  } else {
    for (int g = 0; g < G; g++) {
      load8(xr + g * 512, y[0]);
      fwht512(y[0], lane, lbs);
      emit(y[0], g);
    }
  }
  if (lane == 0) scale[row] = lbs > 0 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)(1 << lbs)))) : s;
}

// The same quant_act with one workgroup per row and one wave per 512-element group (k % 512 == 0,
// k / 512 <= QA_GMAX, bs <= 512): the groups transform independently (a Hadamard block never
// spans two groups), the waves combine their max|y| through LDS, and each quantizes its own
// group. A row of 2048 then runs on 4 waves instead of 1: at M = 2048 the one-wave form leaves
// half the SIMDs without a wave and the rest with one, whose dependent transform and division
// chains then run at their full latency.
template <typename T>
__global__ void __launch_bounds__(64 * QA_GMAX) quant_act_group_kernel(const T* __restrict__ x, int k, int lbs,
                                                                       int qmax, i8* __restrict__ q,
                                                                       float* __restrict__ scale) {
  __shared__ float wmax[QA_GMAX];
  const int lane = threadIdx.x & 63, g = threadIdx.x >> 6, G = blockDim.x >> 6;
  const u64 row = blockIdx.x;
  float y[1][8];
  load8(x + row * k + g * 512 + lane * 8, y[0]);
  const bool neg = fwht512_rows<1>(y, 1, lane, lbs);
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) mx = fmaxf(mx, fabsf(y[0][j]));
  mx = wave_max(mx);
  if (lane == 0) wmax[g] = mx;
  __syncthreads();
  mx = wmax[0];
  for (int i = 1; i < G; i++) mx = fmaxf(mx, wmax[i]);
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(mx, 1e-8f), fq);
  const double rs = neg ? -1.0 / (double)s : 1.0 / (double)s;  // y / s = w * (+-1 / s)
  u64 packed = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const float t = fminf(fmaxf(rintf(uwc_div_rd(y[0][j], rs)), -fq), fq);
    packed |= (u64)(u8)(i8)(int)t << (8 * j);
  }
  *reinterpret_cast<u64*>(q + row * k + g * 512 + lane * 8) = packed;
  if (threadIdx.x == 0) scale[row] = lbs > 0 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)(1 << lbs)))) : s;
}

// 16 consecutive fp32 values, or bf16 bit patterns widened exactly (two 16-byte loads)
__device__ __forceinline__ void load16(const float* p, float v[16]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 a = reinterpret_cast<const float4*>(p)[i];
    v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
  }
}
__device__ __forceinline__ void load16(const uint16_t* p, float v[16]) {
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint4 a = reinterpret_cast<const uint4*>(p)[i];
    const u32 w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[8 * i + 2 * j] = __uint_as_float(w[j] << 16);
      v[8 * i + 2 * j + 1] = __uint_as_float(w[j] & 0xFFFF0000u);
    }
  }
}

// quant_act in the 16-per-lane layout of uwc_fwht.h with one wave per double group and one
// workgroup per row (k % 512 == 0,
// k <= 1024 QD_MAX, bs <= 512): a double group is 1024 elements of the row, two 512-element groups
// split on lane bit 2, 16 consecutive elements per lane (one 64-byte run: four 16-byte loads of
// fp32, two of bf16). The transform costs two VALU operations per element per cross-lane stage
// instead of four; the waves combine their max|y| through LDS and each quantizes its own 1024
// elements with one 16-byte store per lane. A group past the row's end (k / 512 odd) is held as
// zeros and never stored. Measured against the 512-group form (graph-replayed, fp32, bs 512):
// 2048 x 2048 8.96 -> 8.14 us, 2048 x 6144 19.4 -> 16.9, 8192 x 4096 50.9 -> 35.7, 8192 x 14336
// 257 -> 134; below about two waves per SIMD (64 or 100 rows) the 512-group form is faster.
#define QD_MAX 16
template <typename T>
__global__ void __launch_bounds__(64 * QD_MAX) quant_act_dgroup_kernel(const T* __restrict__ x, int k, int lbs,
                                                                       int qmax, i8* __restrict__ q,
                                                                       float* __restrict__ scale) {
  __shared__ float wmax[QD_MAX];
  const int lane = threadIdx.x & 63, d = threadIdx.x >> 6, D = blockDim.x >> 6;
  const int G = k >> 9, grp = (lane >> 2) & 1;
  const bool valid = 2 * d + grp < G;
  const u64 off = (u64)blockIdx.x * k + d * 1024 + grp * 512 + 16 * fw16_index(lane);
  float y[16];
  if (valid) {
    load16(x + off, y);
  } else {
#pragma unroll
    for (int j = 0; j < 16; j++) y[j] = 0.f;
  }
  const bool neg = fwht16(y, lane, lbs);
  float mx = 0.f;
#pragma unroll
  for (int j = 0; j < 16; j++) mx = fmaxf(mx, fabsf(y[j]));
  mx = wave_max(mx);
  if (lane == 0) wmax[d] = mx;
  __syncthreads();
  mx = wmax[0];
  for (int i = 1; i < D; i++) mx = fmaxf(mx, wmax[i]);
  const float fq = (float)qmax;
  const float s = __fdiv_rn(fmaxf(mx, 1e-8f), fq);
  // the lane holds y or -y: y / s = w * (+-1 / s), the sign exact in the float64 product
  const double rs = neg ? -1.0 / (double)s : 1.0 / (double)s;
  u32 w[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    u32 acc = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float t = fminf(fmaxf(rintf(uwc_div_rd(y[4 * i + j], rs)), -fq), fq);
      acc |= (u32)(u8)(i8)(int)t << (8 * j);
    }
    w[i] = acc;
  }
  if (valid) *reinterpret_cast<v4i*>(q + off) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  if (threadIdx.x == 0) scale[blockIdx.x] = lbs > 0 ? __fmul_rn(s, __fdiv_rn(1.0f, uwc_sqrt_rn((float)(1 << lbs)))) : s;
}

// y = (f32(acc) * sx[row]) * sw[col], each product rounded once (qwen3.py:125).
// Rows on grid y, four columns per thread in 16-byte loads and stores (n % 4 == 0, 16-byte aligned
// rows): no division per element. The grid-stride form below divides a 64-bit index by n for every
// element, which made it VALU-bound (8192 x 151936 logits: 1.71 ms for 10 GB of traffic).
__global__ void dequant4_kernel(const v4i* __restrict__ acc, const float* __restrict__ sx,
                                const float4* __restrict__ sw, int n4, int rows, float4* __restrict__ y) {
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= n4) return;
  const float4 w = sw[c];
  for (int r = blockIdx.y; r < rows; r += gridDim.y) {
    const float s = sx[r];
    const v4i a = __builtin_nontemporal_load(acc + (long)r * n4 + c);
    float4 o;
    o.x = __fmul_rn(__fmul_rn((float)a[0], s), w.x);
    o.y = __fmul_rn(__fmul_rn((float)a[1], s), w.y);
    o.z = __fmul_rn(__fmul_rn((float)a[2], s), w.z);
    o.w = __fmul_rn(__fmul_rn((float)a[3], s), w.w);
    uwc_store_nt(y + (long)r * n4 + c, o);
  }
}

__global__ void dequant_kernel(const i32* __restrict__ acc, const float* __restrict__ sx, const float* __restrict__ sw,
                               int n, u64 total, float* __restrict__ y) {
  for (u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (u64)gridDim.x * blockDim.x) {
    const u64 r = i / (u64)n;
    const int c = (int)(i - r * n);
    y[i] = __fmul_rn(__fmul_rn((float)acc[i], sx[r]), sw[c]);
  }
}

template <typename T>
static int quant_rows(const char* fn, const T* x, int rows, int k, int bs, int qmax, int8_t* q, float* scale,
                      hipStream_t stream) {
  if (!x || !q || !scale || rows < 0 || k <= 0) return uwc_fail("%s: null or empty arguments", fn);
  if (bs > 1 && ((bs & (bs - 1)) || k % bs)) return uwc_fail("%s: bs=%d must be a power of two dividing k=%d", fn, bs, k);
  if (qmax < 1 || qmax > 127) return uwc_fail("%s: qmax=%d outside 1..127", fn, qmax);
  if (rows == 0) return UWC_OK;
  const int bse = bs > 1 ? bs : 1;
  if (k % 512 == 0 && k <= 1024 * QD_MAX && bse <= 512 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 15) == 0 &&
      (long)rows * ((k + 1023) / 1024) >= 2L * 4 * uwc_cu_count()) {
    const int lbs = 31 - __builtin_clz((unsigned)bse);
    hipLaunchKernelGGL(quant_act_dgroup_kernel<T>, dim3((unsigned)rows), dim3(64 * ((k + 1023) / 1024)), 0, stream, x, k,
                       lbs, qmax, q, scale);
    return uwc_launch_status(fn);
  }
  if (k % 512 == 0 && bse <= 512 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 7) == 0) {
    const int lbs = 31 - __builtin_clz((unsigned)bse);
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (k <= 512 * QA_GMAX)
      hipLaunchKernelGGL(quant_act_group_kernel<T>, dim3((unsigned)rows), dim3(64 * (k >> 9)), 0, stream, x, k, lbs,
                         qmax, q, scale);
    else
      hipLaunchKernelGGL((quant_act_wave_kernel<false, T>), grid, dim3(256), 0, stream, x, rows, k, lbs, qmax, q, scale);
    return uwc_launch_status(fn);
  }
  const size_t smem = (size_t)k * 4;
  if (smem > 160 * 1024) return uwc_fail("%s: a row of k=%d floats exceeds LDS", fn, k);
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)quant_act_kernel<T>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return uwc_fail("%s: cannot raise LDS to %zu bytes: %s", fn, smem, hipGetErrorString(e));
  }
  hipLaunchKernelGGL(quant_act_kernel<T>, dim3(rows), dim3(256), smem, stream, x, k, bs, qmax, q, scale);
  return uwc_launch_status(fn);
}

extern "C" int uwc_quant_act_f32(const float* x, int rows, int k, int bs, int qmax, int8_t* q, float* scale,
                                 hipStream_t stream) {
  return quant_rows("uwc_quant_act_f32", x, rows, k, bs, qmax, q, scale, stream);
}

extern "C" int uwc_quant_rows_had(const uint16_t* x, int rows, int k, int bs, int8_t* q, float* scale,
                                  hipStream_t stream) {
  if (k % 8) return uwc_fail("uwc_quant_rows_had: k=%d must be a multiple of 8", k);
  return quant_rows("uwc_quant_rows_had", x, rows, k, bs, 64, q, scale, stream);
}

extern "C" int uwc_dequant_f32(const int32_t* acc, const float* sx, const float* sw, int m, int n, float* y,
                               hipStream_t stream) {
  if (!acc || !sx || !sw || !y || m < 0 || n <= 0) return uwc_fail("uwc_dequant_f32: null or empty arguments");
  const u64 total = (u64)m * n;
  if (total == 0) return UWC_OK;
  if (n % 4 == 0 && (((uintptr_t)acc | (uintptr_t)sw | (uintptr_t)y) & 15) == 0) {
    const int n4 = n / 4;
    const dim3 grid((unsigned)((n4 + 255) / 256), (unsigned)(m < 65535 ? m : 65535));
    hipLaunchKernelGGL(dequant4_kernel, grid, dim3(256), 0, stream, reinterpret_cast<const v4i*>(acc), sx,
                       reinterpret_cast<const float4*>(sw), n4, m, reinterpret_cast<float4*>(y));
    return uwc_launch_status("dequant");
  }
  const u64 blocks = (total + 255) / 256;
  hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream, acc, sx,
                     sw, n, total, y);
  return uwc_launch_status("dequant");
}
