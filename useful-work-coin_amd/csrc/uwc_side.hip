// Per-nonce operand side of the mined forward in one launch (kernels.cu:303-404, ops.py:134-168,
// reference.py:96-104):
//   A side:  ApEA = int8(A + EAL[:, P0] - EAL[:, P1]);  X = A S_B^T  -> corrA limbs at corr_a_off,
//            EAL copied into every limb of corrA at ecopy_off;  maxabs[0] = max |X|
//   B side:  Y = BpEBt S_A^T                              -> corrB limbs at corr_b_off;
//            maxabs[1] = max |Y|
// with S^T given as the r x k selection matrix St[j][l] = [P0[l] == j] - [P1[l] == j], and the
// A-side noise EAL[:, P0] - EAL[:, P1] = (SpA EAL^T)^T with SpA = S_A as k rows of 64 bytes.
//
// Workgroup = 32 rows of the A side or of the B side over the full k: 8 compute wave64s and
// SP_PROD producer wave64s. k goes in chunks of 256 columns through an LDS ring (global_load_lds,
// 1 KiB contiguous segments): the chunk's 32 source rows, its r rows of St and (A side) its 256
// rows of SpA. Only the producer waves issue these loads: a chunk is 24-40 DMA instructions per
// CU, which keep the issuing waves blocked on the texture address unit for ~1000 cycles, and in
// the compute waves that would hold up the chunk's MFMAs behind them. Compute wave w computes
// the 16-row tile w & 1 on the 64-column step w >> 1 of every chunk, so each byte crosses the
// texture address unit once per workgroup (per-wave fragment loads from global memory made
// that unit the bottleneck). Everything runs on v_mfma_i32_16x16x64_i8: the projection
// accumulates A-tile x St; the noise of a step is four MFMAs SpA-rows x EAL-tile whose row
// order is permuted so that each lane's 16 results are the noise of exactly its own 16 source
// bytes (then a byte-wise SWAR add), replacing a byte gather per element.
// LDS rows: 256-byte rows with 16-byte chunk c of row R at c ^ (R & 15); 64-byte SpA rows with
// chunk c of row R at c ^ ((R >> 4) & 3): the fragment reads of 16 lanes are conflict-free.
// The four steps' int32 partials add in LDS, then the workgroup writes the balanced base-128
// limbs (digit d = ((v + 64) & 127) - 64, v = (v - d) / 128), the EAL copy and one atomicMax.
// No workgroup waits on another (a cross-workgroup handoff would need device-scope fences,
// which write back and invalidate a whole XCD's L2).
#include "uwc_common.h"

#define SP_ROWS 32
#define SP_WAVES 8                       // compute waves
#define SP_PROD 4                        // producer (DMA) waves
#define SP_THREADS (64 * (SP_WAVES + SP_PROD))
#define SP_MAXR 64
#define SP_CH 256  // columns per chunk

struct SideParams {
  const i8* A;
  const i8* EA;
  const i8* SpA;
  i8* ApEA;
  const i8* StB;
  i8* corrA;
  const i8* Bp;
  const i8* StA;
  i8* corrB;
  i32* maxabs;
  int m, n, k, r, lmax, corr_a_off, ecopy_off, corr_b_off;
};

typedef void __attribute__((address_space(3)))* side_lptr_t;

// Lane i's 16 bytes at g land at LDS byte lds + 16 i (lds wave-uniform, in M0); asm so the
// compiler's wait-count model does not see an LDS write in flight (it would then wait for every
// outstanding LDS read at each use). The kernel waits on vmcnt and barriers itself.
__device__ __forceinline__ void side_dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// A producer wave's wait until at most `younger` chunks (SPW DMA instructions each) of its own
// are still in flight (loads retire in issue order).
template <int SPW>
__device__ __forceinline__ void side_wait(int younger) {
  static_assert(3 * SPW < 64, "vmcnt is 6 bits");
  if (younger >= 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * SPW) : "memory");
  else if (younger == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * SPW) : "memory");
  else if (younger == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SPW) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int NB, bool ASIDE>
struct SideGeom {
  static constexpr int r = NB * 16;
  static constexpr int SRC = SP_ROWS * SP_CH;   // source rows of a chunk
  static constexpr int STB = r * SP_CH;         // St rows of a chunk
  static constexpr int SPT = ASIDE ? SP_CH * 64 : 0;  // SpA rows of a chunk
  static constexpr int STAGE = SRC + STB + SPT;
  static constexpr int NSEG = STAGE / 1024;     // 1 KiB DMA segments per chunk
  static constexpr int SPW = (NSEG + SP_PROD - 1) / SP_PROD;  // per producer wave (the last repeats)
  static constexpr int NS = ASIDE ? 3 : 5;      // ring stages (NS - 1 chunks in flight)
  static constexpr int LDS = NS * STAGE;
};

template <int NB>
constexpr int side_lds() {
  return SideGeom<NB, true>::LDS > SideGeom<NB, false>::LDS ? SideGeom<NB, true>::LDS : SideGeom<NB, false>::LDS;
}

// The byte-wise sum a + c mod 256 of four packed bytes (carries stop at byte boundaries).
__device__ __forceinline__ u32 add_bytes(u32 a, u32 c) {
  return ((a & 0x7F7F7F7Fu) + (c & 0x7F7F7F7Fu)) ^ ((a ^ c) & 0x80808080u);
}

// The chunk loop of one side: projections into acc (C layout of the 16x16x64 MFMA); on the A
// side also the noised source bytes into dst. Producer waves (wave >= SP_WAVES) only load; one
// barrier per chunk: before it the producers wait for chunk c, after it they refill the stage
// every compute wave finished with (chunk c - 1's) while the compute waves work on chunk c.
template <int NB, bool ASIDE>
__device__ __forceinline__ void side_chunks(v4i acc[NB], u8* ring, const i8* src, const i8* St, const i8* SpA,
                                            const i8* EA, i8* dst, int row0, int k, int wave, int lane) {
  using G = SideGeom<NB, ASIDE>;
  const int NC = k / SP_CH;
  const u32 ring_base = __builtin_amdgcn_readfirstlane((u32)(uintptr_t)(side_lptr_t)ring);
  // DMA of chunk c into stage c % NS: segment g (producer pw issues g = t * SP_PROD + pw, the
  // last segment repeating to keep the count per wave uniform) holds 4 rows of 256 bytes (source rows, then
  // St rows) or 16 SpA rows of 64 bytes. 256-byte rows: lane i -> row 4 g' + (i >> 4), physical
  // chunk i & 15 = logical chunk (i & 15) ^ (row & 15). SpA rows: lane i -> row 16 g'' + (i >> 2),
  // physical chunk i & 3 = logical chunk (i & 3) ^ (g'' & 3).
  auto issue = [&](int c) {
    const u32 stage = ring_base + (u32)((c % G::NS) * G::STAGE);
    const int col0 = c * SP_CH;
#pragma unroll
    for (int t = 0; t < G::SPW; t++) {
      const int g = min(t * SP_PROD + (wave - SP_WAVES), G::NSEG - 1);
      const u32 lds = __builtin_amdgcn_readfirstlane(stage + (u32)g * 1024u);
      const void* gp;
      if (g < (G::SRC + G::STB) / 1024) {
        const bool is_src = g < G::SRC / 1024;
        const int R = (is_src ? g : g - G::SRC / 1024) * 4 + (lane >> 4);
        const int col = col0 + (((lane & 15) ^ (R & 15)) << 4);
        gp = is_src ? (const void*)(src + (u64)(row0 + R) * k + col) : (const void*)(St + (u64)R * k + col);
      } else {
        const int g2 = g - (G::SRC + G::STB) / 1024;
        gp = SpA + (u64)(col0 + 16 * g2 + (lane >> 2)) * 64 + (((lane & 3) ^ (g2 & 3)) << 4);
      }
      side_dma16(gp, lds);
    }
  };

  const bool prod = wave >= SP_WAVES;
  if (prod) {
#pragma unroll
    for (int c = 0; c < G::NS - 1; c++)
      if (c < NC) issue(c);
    for (int c = 0; c < NC; c++) {
      // chunk c has landed once every producer has waited for its own DMAs and the barrier
      // passed; every compute wave is then also done with chunk c - 1, whose stage is refilled
      side_wait<G::SPW>(min(NC - 1 - c, G::NS - 2));
      __builtin_amdgcn_s_barrier();
      if (c + G::NS - 1 < NC) issue(c + G::NS - 1);
    }
    return;
  }
  const int rt = wave & 1, si = wave >> 1, rr = lane & 15, q = lane >> 4;
  const int lrow = rt * 16 + rr;
  const int phys = ((si * 4 + q) ^ rr) << 4;  // fragment byte offset in a 256-byte row
  v4i ef = v4i{0, 0, 0, 0};                    // the noise MFMA's B operand: EAL[row][16q, 16q + 16)
  if constexpr (ASIDE)
    if (16 * q < G::r) ef = *reinterpret_cast<const v4i*>(EA + (u64)(row0 + lrow) * G::r + 16 * q);
  i8* drow = ASIDE ? dst + (u64)(row0 + lrow) * k + si * 64 + q * 16 : nullptr;

  for (int c = 0; c < NC; c++) {
    __builtin_amdgcn_s_barrier();
    const u8* st = ring + (c % G::NS) * G::STAGE;
    const v4i a = *reinterpret_cast<const v4i*>(st + lrow * SP_CH + phys);
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const v4i s = *reinterpret_cast<const v4i*>(st + G::SRC + (b * 16 + rr) * SP_CH + phys);
      acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, s, acc[b], 0, 0, 0);
    }
    if constexpr (ASIDE) {
      // MFMA t: A-operand row rr = SpA row 16 (rr >> 2) + 4 t + (rr & 3) of the step, so C element
      // e of lane (rr, q) is the noise of column 16 q + 4 t + e of source row rr: this lane's byte
      // 4 t + e
      const u8* sp = st + G::SRC + G::STB + (si * 64 + 16 * (rr >> 2) + (rr & 3)) * 64 + ((q ^ (rr >> 2)) << 4);
      v4i o;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const v4i sf = *reinterpret_cast<const v4i*>(sp + 4 * t * 64);
        const v4i nz = __builtin_amdgcn_mfma_i32_16x16x64_i8(sf, ef, v4i{0, 0, 0, 0}, 0, 0, 0);
        const u32 cw = ((u32)nz[0] & 0xFFu) | (((u32)nz[1] & 0xFFu) << 8) | (((u32)nz[2] & 0xFFu) << 16) |
                       ((u32)nz[3] << 24);
        o[t] = (int)add_bytes((u32)a[t], cw);
      }
      *reinterpret_cast<v4i*>(drow + c * SP_CH) = o;
    }
  }
}

template <int NB>
__global__ void __launch_bounds__(SP_THREADS) side_kernel(SideParams p) {
  extern __shared__ __attribute__((aligned(1024))) u8 ring[];
  __shared__ __attribute__((aligned(16))) i8 Es[SP_ROWS * SP_MAXR];
  __shared__ i32 Xs[SP_ROWS * SP_MAXR];
  __shared__ int wmax[SP_WAVES + SP_PROD];
  constexpr int r = NB * 16;
  // the wave index is uniform: readfirstlane keeps everything derived from it scalar
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nA = p.m / SP_ROWS;
  const bool aside = (int)blockIdx.x < nA;
  const int row0 = (aside ? blockIdx.x : blockIdx.x - nA) * SP_ROWS;
  const int rows = aside ? p.m : p.n;

  if (aside && tid < SP_ROWS * r / 16)
    reinterpret_cast<v4i*>(Es)[tid] = reinterpret_cast<const v4i*>(p.EA + (u64)row0 * r)[tid];
  for (int i = tid; i < SP_ROWS * r; i += SP_THREADS) Xs[i] = 0;
  __syncthreads();

  v4i acc[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) acc[b] = v4i{0, 0, 0, 0};
  if (aside) side_chunks<NB, true>(acc, ring, p.A, p.StB, p.SpA, p.EA, p.ApEA, row0, p.k, wave, lane);
  else side_chunks<NB, false>(acc, ring, p.Bp, p.StA, nullptr, nullptr, nullptr, row0, p.k, wave, lane);

  // C layout of the 16x16x64 MFMA: lane holds rows 4 (lane >> 4) + e, column lane & 15
  const int rt = wave & 1, rr = lane & 15, q = lane >> 4;
  if (wave < SP_WAVES)
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int e = 0; e < 4; e++) atomicAdd(&Xs[(rt * 16 + 4 * q + e) * r + b * 16 + rr], acc[b][e]);
  __syncthreads();

  // limbs (+ the EAL copy on the A side) and the workgroup max
  i8* corr = aside ? p.corrA : p.corrB;
  const int off = aside ? p.corr_a_off : p.corr_b_off;
  const u64 limb_stride = (u64)rows * 2 * r;
  int local_max = 0;
  for (int i = tid; i < SP_ROWS * r; i += SP_THREADS) {
    const int ro = i / r, j = i - ro * r;
    int v = Xs[i];
    local_max = max(local_max, abs(v));
    const u64 base = (u64)(row0 + ro) * 2 * r;
    for (int li = 0; li < p.lmax; li++) {
      const int d = ((v + 64) & 127) - 64;
      corr[li * limb_stride + base + off + j] = (i8)d;
      v = (v - d) >> 7;
    }
    if (aside && p.ecopy_off >= 0) {
      const i8 e = Es[i];
      for (int li = 0; li < p.lmax; li++) corr[li * limb_stride + base + p.ecopy_off + j] = e;
    }
  }
  if (p.maxabs) {
#pragma unroll
    for (int s = 32; s > 0; s >>= 1) local_max = max(local_max, __shfl_xor(local_max, s));
    if (lane == 0) wmax[wave] = local_max;
    __syncthreads();
    if (tid == 0) {
      int mx = 0;
#pragma unroll
      for (int w = 0; w < SP_WAVES + SP_PROD; w++) mx = max(mx, wmax[w]);
      atomicMax(p.maxabs + (aside ? 0 : 1), mx);
    }
  }
}

template <int NB>
static void side_go(dim3 grid, hipStream_t stream, const SideParams& p) {
  auto kern = side_kernel<NB>;
  static bool attr = false;  // one attribute call per instantiation (the library is process-wide)
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, side_lds<NB>());
    attr = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(SP_THREADS), side_lds<NB>(), stream, p);
}

extern "C" int uwc_side_project(const int8_t* A, int m, const int8_t* EA, const int8_t* SpA, int8_t* ApEA,
                                const int8_t* StB, int8_t* corrA, int corr_a_off, int ecopy_off, const int8_t* Bp,
                                int n, const int8_t* StA, int8_t* corrB, int corr_b_off, int k, int r,
                                int32_t* maxabs, int lmax, hipStream_t stream) {
  if (!A || !EA || !SpA || !ApEA || !StB || !corrA || !Bp || !StA || !corrB)
    return uwc_fail("uwc_side_project: null pointer argument");
  if (m <= 0 || n <= 0 || k <= 0 || m % SP_ROWS || n % SP_ROWS || k % SP_CH)
    return uwc_fail("uwc_side_project: m=%d and n=%d must be positive multiples of %d and k=%d of %d", m, n, SP_ROWS, k,
                    SP_CH);
  if (r != 16 && r != 32 && r != 64) return uwc_fail("uwc_side_project: r=%d must be 16, 32 or 64", r);
  if (lmax < 1 || lmax > 4) return uwc_fail("uwc_side_project: lmax=%d must be 1..4", lmax);
  if (corr_a_off < 0 || corr_a_off + r > 2 * r || corr_b_off < 0 || corr_b_off + r > 2 * r || ecopy_off + r > 2 * r)
    return uwc_fail("uwc_side_project: corr offsets must address one half of a 2r row");
  if ((((uintptr_t)A | (uintptr_t)ApEA | (uintptr_t)Bp | (uintptr_t)StA | (uintptr_t)StB | (uintptr_t)SpA |
        (uintptr_t)EA) & 15u) != 0)
    return uwc_fail("uwc_side_project: A, ApEA, Bp, StA, StB, SpA and EA must be 16-byte aligned");
  SideParams p{A, EA, SpA, ApEA, StB, corrA, Bp, StA, corrB, maxabs, m, n, k, r, lmax, corr_a_off, ecopy_off,
               corr_b_off};
  const dim3 grid(m / SP_ROWS + n / SP_ROWS);
  switch (r) {
    case 16: side_go<1>(grid, stream, p); break;
    case 32: side_go<2>(grid, stream, p); break;
    default: side_go<4>(grid, stream, p); break;
  }
  return uwc_launch_status("side_project");
}
