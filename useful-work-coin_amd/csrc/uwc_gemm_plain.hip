// gfx950 plain int8 x int8 -> int32 GEMM (no transcript, no denoise) for the detrt linears whose
// 256 x 256 tiles would leave CUs idle: the Qwen3-1.7B prefill linears at M = 2048 give 64-192
// such tiles for 256 CUs. Same contract and epilogues as the plain path of uwc_noisy_gemm
// (runtime/detrt/qwen3.py:106-126: int32 out, or fp32 / bf16 of f32(acc) * sx[i] * sw[j]).
//
//   * Workgroup tile BM x BN (128 x 128 or 128 x 256), k step 128, 4 wave64s in 2 x 2, each wave
//     a (BM / 2) x (BN / 2) block of v_mfma_i32_32x32x32_i8 (64 or 128 int32 accumulators).
//   * Operands go HBM -> LDS with global_load_lds_dwordx4 into a ring of S k steps; every wave
//     issues its share of each step (1 KiB segments, the window base in SGPRs, a fixed 32-bit
//     lane offset), S - 1 steps ahead of the one being multiplied. One barrier per k step.
//   * LDS rows are 128 bytes; 16-byte chunk c of tile row r sits at chunk c ^ ((r ^ (r >> 3)) & 7),
//     so the 32-row fragment reads are conflict-free; the swizzle is applied on the global side.
//   * Two fragment sets: the reads of pass p + 1 go out before the MFMAs of pass p.
//   * Transposed C (the B fragment is the MFMA's first operand): lane l holds row l & 31 of a
//     32 x 32 block and 4 consecutive columns per register group; the epilogue turns pairs of
//     blocks around through LDS so that each store instruction writes whole row segments.
//   * int32 sums are exact, so any tiling and k order gives the same accumulators as the other
//     GEMM kernels of this library.
#include <type_traits>

#include "uwc_common.h"

#define P_BK 128
#define P_THREADS 256
#define P_OUT_NONE 0
#define P_OUT_I32 1
#define P_OUT_BF16 2
#define P_OUT_F32 3
// lambdas are always inlined: an out-of-line call would take the accumulator arrays' addresses
#define P_AI __attribute__((always_inline))

namespace {

struct PlainParams {
  const i8* A;
  const i8* B;
  int m, n, k;
  const float* a_scale;
  const float* b_scale;
  void* out;
  int ldc;  // output row stride in elements
};

template <int I, int N, class F>
__device__ __forceinline__ void p_static_for_(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    p_static_for_<I + 1, N>(f);
  }
}
template <int N, class F>
__device__ __forceinline__ void p_static_for(F&& f) {
  p_static_for_<0, N>(f);
}

typedef void __attribute__((address_space(3)))* p_lptr_t;
typedef const v4i __attribute__((address_space(3)))* p_lds_v4i_t;

__device__ __forceinline__ u32 p_lds_addr(const u8* q) { return (u32)(uintptr_t)(p_lptr_t)q; }
__device__ __forceinline__ v4i p_lds(u32 a) { return *(p_lds_v4i_t)(uintptr_t)a; }
__device__ __forceinline__ int p_swz(int r) { return (r ^ (r >> 3)) & 7; }

// One wave-wide DMA: lane i's 16 bytes at sbase + voff land at LDS byte lds + 16 i (lds goes in
// M0). In asm so that the compiler's wait-count model does not see an LDS write in flight (it
// would then wait for every LDS read before each fragment use); the kernel waits on vmcnt and
// barriers itself before any stage is read, and refills a stage only after the barrier that ends
// every read of it.
__device__ __forceinline__ void p_dma(u32 voff, const void* sbase, u32 lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds) : "memory", "m0");
}

// Wait until at most `younger` k steps of this wave's DMA (SEG instructions each) are in flight.
template <int SEG, int MAXY>
__device__ __forceinline__ void p_wait_vm(int younger) {
  static_assert(MAXY * SEG < 64, "vmcnt is 6 bits");
  if (MAXY >= 3 && younger >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * SEG) : "memory");
  else if (MAXY >= 2 && younger >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * SEG) : "memory");
  else if (MAXY >= 1 && younger >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SEG) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__device__ __forceinline__ u32 p_bf16_rne(float f) {
  const u32 u = __float_as_uint(f);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

template <int BM, int BN, int S, bool SPREAD, int OUT>
__global__ void __launch_bounds__(P_THREADS) plain_gemm_kernel(PlainParams p) {
  constexpr int WM = BM / 2, WN = BN / 2;  // wave block
  constexpr int MB = WM / 32, NB = WN / 32;  // 32 x 32 MFMA blocks per wave
  constexpr int TA = BM * P_BK, TB = BN * P_BK;  // bytes of one stage's A and B tile
  constexpr int SA = BM / 32, SB = BN / 32;  // 1 KiB DMA segments per wave per k step
  constexpr int SEG = SA + SB;
  static_assert(MB % 2 == 0 && NB % 2 == 0, "block parity is the row bit 5 of the swizzle");
  static_assert(S >= 2 && S <= 4, "ring depth");
  extern __shared__ __attribute__((aligned(1024))) u8 sm[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // workgroup -> tile: XCD-contiguous runs of ids (dispatch is round-robin over 8 XCDs), rastered
  // in groups of 4 tile rows so that one XCD's tiles share A and B panels in its L2
  int bm0, bn0;
  {
    const int npm = p.m / BM, npn = p.n / BN, total = npm * npn;
    int pid = blockIdx.x;
    if ((total & 7) == 0) pid = (pid & 7) * (total >> 3) + (pid >> 3);
    constexpr int GROUP_M = 4;
    const int grp = GROUP_M * npn, gid = pid / grp, first = gid * GROUP_M;
    const int gsz = min(npm - first, GROUP_M), in = pid - gid * grp;
    bm0 = (first + in % gsz) * BM;
    bn0 = (in / gsz) * BN;
  }
  const long k = p.k;
  const int KT = p.k / P_BK;
  const u32 base = __builtin_amdgcn_readfirstlane(p_lds_addr(sm));
  auto lds_a = [&](int st) P_AI { return base + (u32)(st * TA); };
  auto lds_b = [&](int st) P_AI { return base + (u32)(S * TA + st * TB); };

  // DMA: this wave fills segments wave SA + t of A and wave SB + t of B; lane i of a segment
  // writes LDS bytes [16 i, 16 i + 16): tile row 8 s + i / 8, physical chunk i % 8, so it
  // fetches logical chunk (i % 8) ^ swz(row)
  u32 offa[SA], offb[SB];
#pragma unroll
  for (int t = 0; t < SA; t++) {
    const int row = 8 * (wave * SA + t) + (lane >> 3);
    offa[t] = (u32)((long)row * k + (((lane & 7) ^ p_swz(row)) << 4));
  }
#pragma unroll
  for (int t = 0; t < SB; t++) {
    const int row = 8 * (wave * SB + t) + (lane >> 3);
    offb[t] = (u32)((long)row * k + (((lane & 7) ^ p_swz(row)) << 4));
  }
  const i8* a_win = p.A + (long)bm0 * k;
  const i8* b_win = p.B + (long)bn0 * k;
  // DMA instructions [D0, D1) of a k step (A segments first, then B)
  auto issue_part = [&](auto d0c, auto d1c, int st, long k0) P_AI {
    constexpr int D0 = decltype(d0c)::value, D1 = decltype(d1c)::value;
    p_static_for<SEG>([&](auto dc) P_AI {
      constexpr int d = decltype(dc)::value;
      if constexpr (d >= D0 && d < D1) {
        if constexpr (d < SA) p_dma(offa[d], a_win + k0, lds_a(st) + (u32)((wave * SA + d) * 1024));
        else p_dma(offb[d - SA], b_win + k0, lds_b(st) + (u32)((wave * SB + d - SA) * 1024));
      }
    });
  };
  auto issue = [&](int st, long k0) P_AI {
    issue_part(std::integral_constant<int, 0>{}, std::integral_constant<int, SEG>{}, st, k0);
  };

  // fragment addresses: row (lane & 31) of a 32-row block, logical chunk 2 kp + (lane >> 5);
  // odd blocks (row bit 5 set) flip swizzle bit 2, i.e. use pass kp ^ 2's offset
  u32 fa[4], fb[4];
#pragma unroll
  for (int kp = 0; kp < 4; kp++) {
    const int r = lane & 31, c = 2 * kp + (lane >> 5);
    const u32 o = (u32)(r * P_BK + ((c ^ p_swz(r)) << 4));
    fa[kp] = lds_a(0) + (u32)(wm * WM * P_BK) + o;
    fb[kp] = lds_b(0) + (u32)(wn * WN * P_BK) + o;
  }
  struct Frag {
    v4i a[MB], b[NB];
  };
  auto read = [&](Frag& f, int st, int kp) P_AI {
#pragma unroll
    for (int j = 0; j < NB; j++) f.b[j] = p_lds(fb[(j & 1) ? kp ^ 2 : kp] + (u32)(st * TB + j * 32 * P_BK));
#pragma unroll
    for (int i = 0; i < MB; i++) f.a[i] = p_lds(fa[(i & 1) ? kp ^ 2 : kp] + (u32)(st * TA + i * 32 * P_BK));
  };

  v16i acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; i++)
#pragma unroll
    for (int j = 0; j < NB; j++) acc[i][j] = v16i{};

  // prologue: every stage of the ring loading, then step 0 resident and its first pass read
#pragma unroll
  for (int s = 0; s < S; s++)
    if (s < KT) issue(s, (long)s * P_BK);
  p_wait_vm<SEG, S - 1>(min(KT - 1, S - 1));
  __builtin_amdgcn_s_barrier();
  Frag f[2];
  read(f[0], 0, 0);

  // k step kt in stage ST = kt % S (a compile-time constant: every LDS address is a base
  // register plus an immediate). Before the last pass the wave waits for step kt + 1 (vmcnt,
  // then the barrier: every wave has also finished reading stage ST) and refills ST with step
  // kt + S; the last pass reads the next step's first fragments (on the final step a read of a
  // resident stage that nothing uses, which keeps the MFMA code free of branches).
  auto step = [&](auto stc, int kt) P_AI {
    constexpr int ST = decltype(stc)::value;
    p_static_for<4>([&](auto kpc) P_AI {
      constexpr int kp = decltype(kpc)::value;
      constexpr int nst = kp == 3 ? (ST + 1) % S : ST, nkp = (kp + 1) & 3;
      // SPREAD: the refill of the previous step's stage, continued: quarter kp + 1 of its DMA
      // before pass kp (kp < 3) of this step (the first quarter went out after that step's
      // barrier), so that no wave's MFMAs queue behind a whole step's DMA burst
      if constexpr (SPREAD && kp < 3) {
        if (kt >= 1 && kt - 1 + S < KT) {
          constexpr int PST = (ST + S - 1) % S;
          issue_part(std::integral_constant<int, SEG * (kp + 1) / 4>{}, std::integral_constant<int, SEG * (kp + 2) / 4>{},
                     PST, (long)(kt - 1 + S) * P_BK);
        }
      }
      if constexpr (kp == 3) {
        if (kt + 1 < KT) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          p_wait_vm<SEG, S - 2>(min(KT - 2 - kt, S - 2));
          __builtin_amdgcn_s_barrier();
          if (kt + S < KT) {
            if constexpr (SPREAD)
              issue_part(std::integral_constant<int, 0>{}, std::integral_constant<int, SEG / 4>{}, ST,
                         (long)(kt + S) * P_BK);
            else
              issue(ST, (long)(kt + S) * P_BK);
          }
        }
      }
      Frag& cur = f[kp & 1];
      read(f[(kp + 1) & 1], nst, nkp);
#pragma unroll
      for (int i = 0; i < MB; i++)
#pragma unroll
        for (int j = 0; j < NB; j++)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.b[j], cur.a[i], acc[i][j], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, MB + NB, 0);
#pragma unroll
      for (int q = 0; q < MB * NB; q++) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    });
  };
  for (int kt0 = 0; kt0 < KT; kt0 += S) {
    p_static_for<S>([&](auto sc) P_AI {
      const int kt = kt0 + decltype(sc)::value;
      if (kt < KT) step(sc, kt);
    });
  }

  // epilogue: the wave's blocks, two at a time, through its own 8 KiB of the idle ring, stored by
  // rows. In the MFMA layout lane hh 32 + rr holds row rr of a block and, in register group j,
  // columns 8 j + 4 hh .. + 3; that piece goes to slot piece (4 b + j) 64 + hh 32 + (rr ^ 2 (2 j +
  // hh)) for block b of the pair. Store instruction jj then has lane l take row 8 jj + l / 8,
  // columns 4 (l % 8) .. + 3 of a block: 8 whole row segments per instruction instead of 32 rows
  // of 16 bytes (the output burst at the end of a launch drains faster). The XOR keeps the 16
  // lanes of each write (16 rows) and of each read (2 rows x 8 pieces) on distinct 16-byte bank
  // groups. The stores carry the non-temporal hint, so that the output stream does not evict the
  // operand panels other workgroups of the XCD still read from L2 (the M = 2048 Qwen3-1.7B
  // linears 4-8% faster).
  if constexpr (OUT != P_OUT_NONE) {
    constexpr int ES = OUT == P_OUT_BF16 ? 2 : 4;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // every wave is done reading the ring
    u8* slot = sm + wave * 8192;
    const int hh = lane >> 5, rr = lane & 31;
    const int rj = (lane & 7) >> 1, rh = lane & 1;  // the piece a row read takes
#pragma unroll
    for (int i = 0; i < MB; i++) {
#pragma unroll
      for (int j0 = 0; j0 < NB; j0 += 2) {
#pragma unroll
        for (int b = 0; b < 2; b++)
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const v16i& v = acc[i][j0 + b];
            *reinterpret_cast<v4i*>(slot + ((4 * b + g) * 64 + hh * 32 + (rr ^ (2 * (2 * g + hh)))) * 16) =
                v4i{v[4 * g], v[4 * g + 1], v[4 * g + 2], v[4 * g + 3]};
          }
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const int row0 = bm0 + wm * WM + i * 32, col = bn0 + wn * WN + (j0 + b) * 32 + 4 * (lane & 7);
          u8* base = reinterpret_cast<u8*>(p.out) + ((long)row0 * p.ldc + col) * ES;
          float4 sw{};
          if constexpr (OUT != P_OUT_I32) sw = *reinterpret_cast<const float4*>(p.b_scale + col);
          // the four LDS reads (and row scales) first, then the stores: read, wait, store in turn
          // put an LDS round trip (and a scale load) in front of every store
          v4i xs[4];
          float ascs[4];
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int r = 8 * jj + (lane >> 3);
            xs[jj] = *reinterpret_cast<const v4i*>(slot + ((4 * b + rj) * 64 + rh * 32 + (r ^ (2 * (2 * rj + rh)))) * 16);
            if constexpr (OUT != P_OUT_I32) ascs[jj] = p.a_scale[row0 + r];
          }
#pragma unroll
          for (int jj = 0; jj < 4; jj++) {
            const int r = 8 * jj + (lane >> 3);
            const v4i x = xs[jj];
            u8* dst = base + (long)r * p.ldc * ES;
            if constexpr (OUT == P_OUT_I32) {
              uwc_store_nt(dst, x);
            } else {
              const float asc = ascs[jj];
              const float y0 = __fmul_rn(__fmul_rn((float)x[0], asc), sw.x);
              const float y1 = __fmul_rn(__fmul_rn((float)x[1], asc), sw.y);
              const float y2 = __fmul_rn(__fmul_rn((float)x[2], asc), sw.z);
              const float y3 = __fmul_rn(__fmul_rn((float)x[3], asc), sw.w);
              if constexpr (OUT == P_OUT_F32) {
                uwc_store_nt(dst, float4{y0, y1, y2, y3});
              } else {
                uwc_store_nt(dst, uint2{p_bf16_rne(y0) | (p_bf16_rne(y1) << 16), p_bf16_rne(y2) | (p_bf16_rne(y3) << 16)});
              }
            }
          }
        }
      }
    }
  }
}

template <int BM, int BN, int S, bool SPREAD, int OUT>
void plain_go(hipStream_t s, const PlainParams& p) {
  auto kern = plain_gemm_kernel<BM, BN, S, SPREAD, OUT>;
  constexpr int lds = S * (BM + BN) * P_BK;
  static_assert(lds <= 160 * 1024, "LDS exceeds 160 KiB");
  static bool attr = false;  // one attribute call per instantiation (the library is process-wide)
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    attr = true;
  }
  hipLaunchKernelGGL(kern, dim3((p.m / BM) * (p.n / BN)), dim3(P_THREADS), lds, s, p);
}

template <int BM, int BN, int S, bool SPREAD>
void plain_out(int out_mode, hipStream_t s, const PlainParams& p) {
  switch (out_mode) {
    case P_OUT_NONE: plain_go<BM, BN, S, SPREAD, P_OUT_NONE>(s, p); break;
    case P_OUT_I32: plain_go<BM, BN, S, SPREAD, P_OUT_I32>(s, p); break;
    case P_OUT_BF16: plain_go<BM, BN, S, SPREAD, P_OUT_BF16>(s, p); break;
    default: plain_go<BM, BN, S, SPREAD, P_OUT_F32>(s, p); break;
  }
}

}  // namespace

// The configurations of the plain DMA kernel: BM x BN, ring depth; c | 4 spreads each step's DMA.
struct PlainCfg {
  int bm, bn, stages;
};
static const PlainCfg kPlainCfgs[] = {{128, 128, 4}, {128, 256, 3}, {128, 128, 2}, {128, 256, 2}};
#define PLAIN_NCFG 8

int uwc_plain_cfg_count() { return PLAIN_NCFG; }

// Whether configuration cfg takes the shape: whole tiles, whole k steps, 16-byte output rows.
bool uwc_plain_fits(int cfg, int m, int n, int k, int ldc, const void* out, int out_mode, const float* b_scale) {
  if (cfg < 0 || cfg >= PLAIN_NCFG) return false;
  const PlainCfg& c = kPlainCfgs[cfg & 3];
  const bool vec_out = out_mode == P_OUT_NONE || ((uintptr_t)out % 16 == 0 && ldc % 4 == 0);
  // the dequant epilogues read 4 column scales at once
  const bool vec_scale = out_mode != P_OUT_F32 && out_mode != P_OUT_BF16 || (uintptr_t)b_scale % 16 == 0;
  return vec_scale && m % c.bm == 0 && n % c.bn == 0 && k % P_BK == 0 && k >= P_BK && k <= (1 << 23) && vec_out;
}

// Called by uwc_noisy_gemm for a plain GEMM after its argument checks and uwc_plain_fits.
int uwc_gemm_plain(int cfg, const int8_t* A, const int8_t* B, int m, int n, int k, const float* a_scale,
                   const float* b_scale, void* out, int out_mode, int ldc, hipStream_t stream) {
  if (!uwc_plain_fits(cfg, m, n, k, ldc, out, out_mode, b_scale))
    return uwc_fail("uwc_gemm_plain: configuration %d does not take m=%d n=%d k=%d", cfg, m, n, k);
  const PlainParams p{A, B, m, n, k, a_scale, b_scale, out, ldc};
  switch (cfg) {
    case 0: plain_out<128, 128, 4, false>(out_mode, stream, p); break;
    case 1: plain_out<128, 256, 3, false>(out_mode, stream, p); break;
    case 2: plain_out<128, 128, 2, false>(out_mode, stream, p); break;
    case 3: plain_out<128, 256, 2, false>(out_mode, stream, p); break;
    case 4: plain_out<128, 128, 4, true>(out_mode, stream, p); break;
    case 5: plain_out<128, 256, 3, true>(out_mode, stream, p); break;
    case 6: plain_out<128, 128, 2, true>(out_mode, stream, p); break;
    default: plain_out<128, 256, 2, true>(out_mode, stream, p); break;
  }
  return uwc_launch_status("plain_gemm");
}
