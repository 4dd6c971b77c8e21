// Shared device helpers for the gfx950 kernels of the int8 GEMM hot path.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "uwc.h"

typedef uint32_t u32;
typedef int32_t i32;
typedef int8_t i8;
typedef uint8_t u8;
typedef uint64_t u64;
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

// 16-byte stores and loads with the non-temporal hint (the nt bit: streamed through the caches
// rather than kept), for data written once and read once much later, e.g. a scratch larger than
// the caches, so that it does not evict what the kernel rereads from L2.
typedef u32 u2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void uwc_store_nt(void* p, float4 v) {
  __builtin_nontemporal_store(f4v{v.x, v.y, v.z, v.w}, reinterpret_cast<f4v*>(p));
}
__device__ __forceinline__ void uwc_store_nt(void* p, v4i v) { __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(p)); }
__device__ __forceinline__ void uwc_store_nt(void* p, uint2 v) {
  __builtin_nontemporal_store(u2v{v.x, v.y}, reinterpret_cast<u2v*>(p));
}
__device__ __forceinline__ float4 uwc_load_nt(const float* p) {
  const f4v t = __builtin_nontemporal_load(reinterpret_cast<const f4v*>(p));
  return float4{t.x, t.y, t.z, t.w};
}

#define UWC_OK 0

// Correctly rounded float32 square root. HIP's __fsqrt_rn is the native (approximate) sqrt
// unless OCML's rounded operations are enabled, so the root is taken in float64 (correctly
// rounded) and rounded once to float32: double rounding is innocuous for sqrt since
// 53 >= 2 * 24 + 2. (__fdiv_rn / __fmul_rn / __fadd_rn are the plain correctly rounded ops;
// the library builds with -ffp-contract=off so they are never fused.)
__device__ __forceinline__ float uwc_sqrt_rn(float x) { return (float)__builtin_sqrt((double)x); }

// x / d correctly rounded to float32, for float32 x and a normal float32 d > 0 given as
// rd = 1.0 / (double)d (correctly rounded in float64): the float64 product x * rd is within
// 2^-52 (relative) of x / d, while a quotient of two float32 values is never a float32 rounding
// midpoint and lies more than 2^-49 (relative) from every midpoint (with x = X 2^a, d = D 2^b and
// a midpoint M 2^c, M odd of 25 bits: x - M 2^c d is a nonzero multiple of 2^(b+c), so the
// quotient's distance from the midpoint is at least 2^c / D > 2^(c-24), against M 2^c < 2^(c+25)),
// so rounding the product to float32 rounds the exact quotient. Three instructions instead of the
// IEEE division sequence, for divisions of many values by one per-row constant.
__device__ __forceinline__ float uwc_div_rd(float x, double rd) { return (float)((double)x * rd); }

// Records a message for uwc_last_error() and returns UWC_EINVAL.
int uwc_fail(const char* fmt, ...);
// hipGetLastError() after a launch, converted to a status (and a message on failure).
int uwc_launch_status(const char* kernel);
// Compute units of the current device (cached per device).
int uwc_cu_count();

// ------------------------------------------------------------------ BLAKE3
// The keyed one-block compression used for tile digests, noise words and tree nodes.
// Restated from the BLAKE3 specification (the reference's CUDA version is
// miner/ampere/uwc_ampere/kernels.cu:48-101).
#define B3_CHUNK_START 1u
#define B3_CHUNK_END 2u
#define B3_PARENT 4u
#define B3_ROOT 8u
#define B3_KEYED 16u

__device__ __forceinline__ u32 b3_iv(int i) {
  // BLAKE3 IV (the SHA-256 initial hash words); a switch keeps it in immediates.
  switch (i) {
    case 0: return 0x6A09E667u; case 1: return 0xBB67AE85u; case 2: return 0x3C6EF372u;
    case 3: return 0xA54FF53Au; case 4: return 0x510E527Fu; case 5: return 0x9B05688Cu;
    case 6: return 0x1F83D9ABu; default: return 0x5BE0CD19u;
  }
}

// Message word used by round `r` at position `i`: the permutation applied r times.
__device__ constexpr int kB3Sched[7][16] = {
    {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15},
    {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8},
    {3, 4, 10, 12, 13, 2, 7, 14, 6, 5, 9, 0, 11, 15, 8, 1},
    {10, 7, 12, 9, 14, 3, 13, 15, 4, 0, 11, 2, 5, 8, 1, 6},
    {12, 13, 9, 11, 15, 10, 14, 8, 7, 2, 5, 3, 0, 1, 6, 4},
    {9, 14, 11, 5, 8, 12, 15, 1, 13, 3, 0, 10, 2, 6, 4, 7},
    {11, 15, 5, 0, 1, 9, 8, 6, 14, 10, 2, 12, 3, 4, 7, 13},
};

__device__ __forceinline__ u32 rotr32(u32 x, int n) { return __builtin_amdgcn_alignbit(x, x, n); }

#define UWC_B3G(a, b, c, d, x, y)            \
  a = a + b + (x); d = rotr32(d ^ a, 16);    \
  c = c + d;       b = rotr32(b ^ c, 12);    \
  a = a + b + (y); d = rotr32(d ^ a, 8);     \
  c = c + d;       b = rotr32(b ^ c, 7);

// out[0..7] = first half of compress(cv, m, counter, blen, flags).
__device__ __forceinline__ void b3_compress(const u32 cv[8], const u32 m[16], u64 counter, u32 blen, u32 flags,
                                            u32 out[8]) {
  u32 v0 = cv[0], v1 = cv[1], v2 = cv[2], v3 = cv[3], v4 = cv[4], v5 = cv[5], v6 = cv[6], v7 = cv[7];
  u32 v8 = b3_iv(0), v9 = b3_iv(1), v10 = b3_iv(2), v11 = b3_iv(3);
  u32 v12 = (u32)counter, v13 = (u32)(counter >> 32), v14 = blen, v15 = flags;
#pragma unroll
  for (int r = 0; r < 7; r++) {
    UWC_B3G(v0, v4, v8, v12, m[kB3Sched[r][0]], m[kB3Sched[r][1]]);
    UWC_B3G(v1, v5, v9, v13, m[kB3Sched[r][2]], m[kB3Sched[r][3]]);
    UWC_B3G(v2, v6, v10, v14, m[kB3Sched[r][4]], m[kB3Sched[r][5]]);
    UWC_B3G(v3, v7, v11, v15, m[kB3Sched[r][6]], m[kB3Sched[r][7]]);
    UWC_B3G(v0, v5, v10, v15, m[kB3Sched[r][8]], m[kB3Sched[r][9]]);
    UWC_B3G(v1, v6, v11, v12, m[kB3Sched[r][10]], m[kB3Sched[r][11]]);
    UWC_B3G(v2, v7, v8, v13, m[kB3Sched[r][12]], m[kB3Sched[r][13]]);
    UWC_B3G(v3, v4, v9, v14, m[kB3Sched[r][14]], m[kB3Sched[r][15]]);
  }
  out[0] = v0 ^ v8; out[1] = v1 ^ v9; out[2] = v2 ^ v10; out[3] = v3 ^ v11;
  out[4] = v4 ^ v12; out[5] = v5 ^ v13; out[6] = v6 ^ v14; out[7] = v7 ^ v15;
}

// Keyed digest of one 64-byte message (a single-block, single-chunk root).
__device__ __forceinline__ void b3_keyed64(const u32 key[8], const u32 m[16], u32 out[8]) {
  b3_compress(key, m, 0, 64, B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, out);
}

// Plain (unkeyed) digest of one 64-byte message.
__device__ __forceinline__ void b3_plain64(const u32 m[16], u32 out[8]) {
  u32 iv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) iv[i] = b3_iv(i);
  b3_compress(iv, m, 0, 64, B3_CHUNK_START | B3_CHUNK_END | B3_ROOT, out);
}

// Little-endian U256 compare h <= t (the jackpot rule).
__device__ __forceinline__ bool u256_le(const u32 h[8], const u32* t) {
  bool le = true, decided = false;
#pragma unroll
  for (int i = 7; i >= 0; i--) {
    const u32 tv = t[i];
    if (!decided && h[i] != tv) { le = h[i] < tv; decided = true; }
  }
  return le;
}
