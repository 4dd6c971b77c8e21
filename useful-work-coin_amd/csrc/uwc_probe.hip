// Sustained int8 MFMA rate of this part: a register-only loop of v_mfma_i32_32x32x32_i8 on
// every SIMD (8 independent 32 x 32 accumulators per wave, 2 waves per SIMD, one workgroup per
// CU), with operands that are either constant or seeded random bytes. The matrix cores draw more
// power when their operands switch, and the part then runs at a lower clock: the random-operand
// rate is the practical ceiling of an int8 GEMM on real data, the figure the bench reports next
// to the published dense peak.
#include "uwc_common.h"

template <bool RANDOM>
__global__ void __launch_bounds__(512) mfma_rate_kernel(int iters, u32 seed0, u32* __restrict__ sink) {
  v16i acc[8];
#pragma unroll
  for (int j = 0; j < 8; j++) acc[j] = v16i{};
  u32 seed = seed0 ^ (threadIdx.x * 2654435761u + blockIdx.x * 40503u);
  v4i fa[4], fb[2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      seed = seed * 1664525u + 1013904223u;
      fa[i][e] = RANDOM ? (int)seed : 0x01010101;
    }
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int e = 0; e < 4; e++) {
      seed = seed * 1664525u + 1013904223u;
      fb[i][e] = RANDOM ? (int)seed : 0x01010101;
    }
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int mb = 0; mb < 4; mb++)
#pragma unroll
      for (int nb = 0; nb < 2; nb++)
        acc[mb * 2 + nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[mb], fb[nb], acc[mb * 2 + nb], 0, 0, 0);
  }
  u32 s = 0;
#pragma unroll
  for (int j = 0; j < 8; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) s += (u32)acc[j][e];
  sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

extern "C" int uwc_mfma_rate_probe(int iters, int random_operands, uint32_t* sink, int64_t sink_words, hipStream_t stream) {
  const char* fn = "uwc_mfma_rate_probe";
  const int cus = uwc_cu_count();
  if (!sink || iters <= 0) return uwc_fail("%s: null sink or iters <= 0", fn);
  if (sink_words < (int64_t)cus * 512) return uwc_fail("%s: sink needs %d words", fn, cus * 512);
  if (random_operands)
    hipLaunchKernelGGL(mfma_rate_kernel<true>, dim3(cus), dim3(512), 0, stream, iters, 0x9E3779B9u, sink);
  else
    hipLaunchKernelGGL(mfma_rate_kernel<false>, dim3(cus), dim3(512), 0, stream, iters, 0x9E3779B9u, sink);
  return uwc_launch_status(fn);
}
