// The operand side of a group of nonces in one launch (kernels.cu:303-404, ops.py:331-336,
// reference.py:96-104), for the shapes of a mining sweep (m, n % 128, k % 128, r 16 / 32 / 64):
// for every nonce i of the group
//   A side:  ApEA_i = int8(A_i + EA_i[:, P0] - EA_i[:, P1]);  X_i = A_i S_B^T -> corrA_i limbs at
//            corr_a_off, EA_i copied into every limb of corrA_i at ecopy_off;  maxabs_i[0] = max |X_i|
//   B side:  Y_i = Bp S_Ai^T -> corrB_i limbs at corr_b_off;  maxabs_i[1] = max |Y_i|
// with the selection matrices given as St (r x k: St[j][l] = [P0[l] == j] - [P1[l] == j]) and,
// for the noise, SpA_i = S_Ai as k rows of 64 bytes (zero past r).
//
// A workgroup takes 128 rows of one nonce's A side or B side over the full k, in chunks of 128
// columns staged through an LDS ring by 4 producer waves (global_load_lds, 1 KiB segments):
// the chunk's 128 source rows, its r rows of St and (A side) its 128 rows of SpA. Compute wave w
// owns rows 16 w .. 16 w + 15 for the whole k, so its projection accumulators (v_mfma_i32_16x16x64_i8,
// A = 16 source rows x 64 columns, B = 64 columns x 16 rows of St) need no reduction across
// waves, and each St / SpA byte staged in LDS serves the 8 row tiles of the workgroup. The noise
// of a 64-column step is four MFMAs of SpA rows x the wave's E rows whose A-operand rows are
// permuted so that each lane's 16 results are the noise of its own 16 source bytes, added with
// a byte-wise SWAR add. A group of nonces is one launch of count x m / 128 A-side and
// ceil(count / 2) x n / 128 B-side workgroups: enough to keep every CU loading while others
// compute (the per-nonce form keeps one latency-bound workgroup per CU). A B-side workgroup
// projects its 128 rows of B' for two nonces (their St tiles take the stage space the A side
// gives to SpA), so each row of B' is read once per nonce pair (32 nonces per launch: 11.6 ->
// 10.9 us per nonce for both sides).
//
// LDS rows of 128 bytes keep 16-byte chunk c of row R at c ^ ((R ^ (R >> 3)) & 7); 64-byte SpA
// rows keep chunk c of row R at c ^ ((R >> 4) & 3): the 16 lanes of a fragment read hit
// distinct banks.
#include "uwc_common.h"

#define SM_ROWS 128
#define SM_CH 128                        // columns per chunk
#define SM_WAVES 8                       // compute waves (16 rows each)
#define SM_PROD 4                        // producer (DMA) waves
#define SM_THREADS (64 * (SM_WAVES + SM_PROD))
#define SM_MAXB 32

struct SideManyItem {
  const i8* A;
  const i8* EA;
  const i8* SpA;
  i8* ApEA;
  i8* corrA;
  const i8* StA;
  i8* corrB;
  i32* maxabs;
};

struct SideManyParams {
  const i8* StB;
  const i8* Bp;
  int m, n, k, r, lmax, corr_a_off, ecopy_off, corr_b_off, count;
  SideManyItem it[SM_MAXB];
};

typedef void __attribute__((address_space(3)))* sm_lptr_t;

__device__ __forceinline__ void sm_dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}

// wait until at most `younger` chunks (SPW DMA instructions each) of this producer are in flight
template <int SPW>
__device__ __forceinline__ void sm_wait(int younger) {
  static_assert(5 * SPW < 64, "vmcnt is 6 bits");
  if (younger >= 5) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * SPW) : "memory");
  else if (younger == 4) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * SPW) : "memory");
  else if (younger == 3) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * SPW) : "memory");
  else if (younger == 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * SPW) : "memory");
  else if (younger == 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(SPW) : "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

__device__ __forceinline__ int sm_swz(int R) { return (R ^ (R >> 3)) & 7; }

__device__ __forceinline__ u32 sm_add_bytes(u32 a, u32 c) {
  return ((a & 0x7F7F7F7Fu) + (c & 0x7F7F7F7Fu)) ^ ((a ^ c) & 0x80808080u);
}

template <int NB, bool ASIDE>
struct SmGeom {
  static constexpr int r = NB * 16;
  static constexpr int NST = ASIDE ? 1 : 2;                 // selection matrices (B side: a nonce pair's)
  static constexpr int SRC = SM_ROWS * SM_CH;               // source rows of a chunk
  static constexpr int STB = r * SM_CH;                     // St rows of a chunk, per selection matrix
  static constexpr int SPT = ASIDE ? SM_CH * 64 : 0;        // SpA rows of a chunk
  static constexpr int STAGE = SRC + NST * STB + SPT;
  static constexpr int NSEG = STAGE / 1024;                 // 1 KiB DMA segments per chunk
  static constexpr int SPW = (NSEG + SM_PROD - 1) / SM_PROD;  // per producer wave (the last repeats)
  // ring stages: two (64 KiB at r = 64). A deeper ring measured no faster alone, and the batched
  // commitment of the next group, queued beside this launch on another stream, then fits on the
  // same CUs (five of its 18 KiB workgroups next to one of these; one next to a 4-stage ring)
  static constexpr int NS = 2;
  static constexpr int LDS = NS * STAGE;
};

template <int NB>
constexpr int sm_lds() {
  return SmGeom<NB, true>::LDS > SmGeom<NB, false>::LDS ? SmGeom<NB, true>::LDS : SmGeom<NB, false>::LDS;
}

// One workgroup: 128 rows (row0 ..) of src over the full k, with the selection matrix St and, on
// the A side, the noise (E, SpA) into dst. The B side projects its rows of B' for two nonces at
// once (St, corr, maxabs and St2, corr2, maxabs2; corr2 NULL: no second nonce, St2 = St), so a
// group reads each row of B' half as often.
template <int NB, bool ASIDE>
__device__ __forceinline__ void sm_side(u8* ring, const i8* src, const i8* St, const i8* SpA, const i8* E, i8* dst,
                                        i8* corr, int corr_off, int ecopy_off, i32* maxabs, const i8* St2, i8* corr2,
                                        i32* maxabs2, int rows, int row0, int k, int lmax, int wave, int lane,
                                        int* wmax) {
  using G = SmGeom<NB, ASIDE>;
  constexpr int r = G::r;
  const int NC = k / SM_CH;
  const u32 ring_base = __builtin_amdgcn_readfirstlane((u32)(uintptr_t)(sm_lptr_t)ring);
  if (wave >= SM_WAVES) {
    // producer: chunk c into stage c % NS; segment g holds 8 rows of 128 bytes (source, then St,
    // then on the B side St2) or 16 rows of 64 bytes (A side: SpA): lane i -> row 8 g + (i >> 3)
    // (St rows counted from each matrix's first segment), physical chunk i & 7 (logical
    // chunk (i & 7) ^ swz(row)); SpA: row 16 g' + (i >> 2), physical chunk i & 3 (logical chunk
    // (i & 3) ^ (g' & 3))
    const int pw = wave - SM_WAVES;
    auto issue = [&](int c) {
      const u32 stage = ring_base + (u32)((c % G::NS) * G::STAGE);
      const int col0 = c * SM_CH;
#pragma unroll
      for (int t = 0; t < G::SPW; t++) {
        const int g = min(t * SM_PROD + pw, G::NSEG - 1);
        const u32 lds = __builtin_amdgcn_readfirstlane(stage + (u32)g * 1024u);
        const void* gp;
        if (g < (G::SRC + G::NST * G::STB) / 1024) {
          const bool is_src = g < G::SRC / 1024;
          const int gs = g - G::SRC / 1024;  // St segment; on the B side segments STB / 1024 on are St2's
          const int R = (is_src ? g : gs % (G::STB / 1024)) * 8 + (lane >> 3);
          const int col = col0 + (((lane & 7) ^ sm_swz(R)) << 4);
          const i8* stp = (G::NST == 2 && gs >= G::STB / 1024) ? St2 : St;
          gp = is_src ? (const void*)(src + (u64)(row0 + R) * k + col) : (const void*)(stp + (u64)R * k + col);
        } else {
          const int g2 = g - (G::SRC + G::NST * G::STB) / 1024;
          gp = SpA + (u64)(col0 + 16 * g2 + (lane >> 2)) * 64 + (((lane & 3) ^ (g2 & 3)) << 4);
        }
        sm_dma16(gp, lds);
      }
    };
#pragma unroll
    for (int c = 0; c < G::NS - 1; c++)
      if (c < NC) issue(c);
    for (int c = 0; c < NC; c++) {
      sm_wait<G::SPW>(min(NC - 1 - c, G::NS - 2));
      __builtin_amdgcn_s_barrier();
      if (c + G::NS - 1 < NC) issue(c + G::NS - 1);
    }
  } else {
    const int rr = lane & 15, q = lane >> 4;
    const int lrow = wave * 16 + rr;  // this lane's source row in the tile (fragment and noise)
    v4i acc[NB], acc2[NB];  // acc2: the B side's second nonce
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] = acc2[b] = v4i{0, 0, 0, 0};
    static_assert(SM_CH == 128, "a chunk is two 64-column noise steps per row");
    v4i ef = v4i{0, 0, 0, 0};  // the noise MFMA's B operand: E[row][16 q, 16 q + 16)
    v4i o0 = v4i{0, 0, 0, 0};  // the noised bytes of the chunk's first 64 columns
    if constexpr (ASIDE)
      if (16 * q < r) ef = *reinterpret_cast<const v4i*>(E + (u64)(row0 + lrow) * r + 16 * q);
    for (int c = 0; c < NC; c++) {
      __builtin_amdgcn_s_barrier();
      const u8* st = ring + (c % G::NS) * G::STAGE;
#pragma unroll
      for (int s = 0; s < SM_CH / 64; s++) {
        const int lc = 4 * s + q;  // logical 16-byte chunk of the row
        const v4i a = *reinterpret_cast<const v4i*>(st + lrow * SM_CH + ((lc ^ sm_swz(lrow)) << 4));
#pragma unroll
        for (int b = 0; b < NB; b++) {
          const int R = b * 16 + rr;
          const v4i sf = *reinterpret_cast<const v4i*>(st + G::SRC + R * SM_CH + ((lc ^ sm_swz(R)) << 4));
          acc[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, sf, acc[b], 0, 0, 0);
          if constexpr (!ASIDE) {
            const v4i sf2 =
                *reinterpret_cast<const v4i*>(st + G::SRC + G::STB + R * SM_CH + ((lc ^ sm_swz(R)) << 4));
            acc2[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, sf2, acc2[b], 0, 0, 0);
          }
        }
        if constexpr (ASIDE) {
          // noise MFMA t: A-operand row rr = SpA row 64 s + 16 (rr >> 2) + 4 t + (rr & 3) of the
          // chunk, so C element e of lane (rr, q) is the noise of column 16 q + 4 t + e of the
          // step for source row rr: this lane's byte 4 t + e
          const int R0 = 64 * s + 16 * (rr >> 2) + (rr & 3);
          const u8* sp = st + G::SRC + G::NST * G::STB + R0 * 64 + ((q ^ ((R0 >> 4) & 3)) << 4);
          v4i o;
#pragma unroll
          for (int t = 0; t < 4; t++) {
            const v4i sf = *reinterpret_cast<const v4i*>(sp + 4 * t * 64);
            const v4i nz = __builtin_amdgcn_mfma_i32_16x16x64_i8(sf, ef, v4i{0, 0, 0, 0}, 0, 0, 0);
            const u32 cw = ((u32)nz[0] & 0xFFu) | (((u32)nz[1] & 0xFFu) << 8) | (((u32)nz[2] & 0xFFu) << 16) |
                           ((u32)nz[3] << 24);
            o[t] = (int)sm_add_bytes((u32)a[t], cw);
          }
          if (s == 0) {
            o0 = o;
          } else {
            // The chunk's noised bytes of the wave's 16 rows, stored as 8 whole rows (128 bytes) per
            // instruction: lane (rr, q) holds bytes 16 q .. of row rr (o0) and 64 + 16 q .. (o), and
            // swaps the latter with lane rr ^ 8 (DPP row_ror:8 inside its 16-lane row); stores
            // of 16 rows x 64 bytes drained measurably slower (94.7 -> 88.2 us per 8 nonces).
            v4i x;
#pragma unroll
            for (int t = 0; t < 4; t++) x[t] = __builtin_amdgcn_update_dpp(0, o[t], 0x128, 0xF, 0xF, true);
            const bool lo = rr < 8;
            i8* rowp = dst + (u64)(row0 + wave * 16 + (rr & 7)) * k + c * SM_CH;
            *reinterpret_cast<v4i*>(rowp + 16 * (lo ? q : 4 + q)) = lo ? o0 : x;
            *reinterpret_cast<v4i*>(rowp + (u64)8 * k + 16 * (lo ? 4 + q : q)) = lo ? x : o0;
          }
        }
      }
    }
    // C layout of the 16 x 16 x 64 MFMA: lane (j, q) holds rows 4 q + e of the wave's tile,
    // column 16 b + j of the projection
    const u64 limb_stride = (u64)rows * 2 * r;
    auto emit = [&](const v4i* ac, i8* cp) {
      int mx = 0;
#pragma unroll
      for (int b = 0; b < NB; b++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          int v = ac[b][e];
          mx = max(mx, abs(v));
          i8* out = cp + (u64)(row0 + wave * 16 + 4 * q + e) * 2 * r + corr_off + 16 * b + rr;
          for (int li = 0; li < lmax; li++) {
            const int d = ((v + 64) & 127) - 64;
            out[li * limb_stride] = (i8)d;
            v = (v - d) >> 7;
          }
        }
#pragma unroll
      for (int s = 32; s > 0; s >>= 1) mx = max(mx, __shfl_xor(mx, s));
      return mx;
    };
    const int mx = emit(acc, corr);
    if (lane == 0) wmax[wave] = mx;
    if constexpr (!ASIDE) {
      if (corr2) {
        const int mx2 = emit(acc2, corr2);
        if (lane == 0) wmax[SM_WAVES + wave] = mx2;
      }
    }
    if (ASIDE && ecopy_off >= 0) {
      // the wave's 16 E rows (r bytes each) into every limb: lane -> row lane / (r / 16) ... in
      // 16-byte pieces
      constexpr int PIECES = r / 16;  // 16-byte pieces per row
      for (int p = lane; p < 16 * PIECES; p += 64) {
        const int row = row0 + wave * 16 + p / PIECES, col = (p % PIECES) * 16;
        const v4i e = *reinterpret_cast<const v4i*>(E + (u64)row * r + col);
        for (int li = 0; li < lmax; li++)
          *reinterpret_cast<v4i*>(corr + li * limb_stride + (u64)row * 2 * r + ecopy_off + col) = e;
      }
    }
  }
  __syncthreads();
  if (threadIdx.x == 0 && maxabs) {
    int m = 0;
#pragma unroll
    for (int w = 0; w < SM_WAVES; w++) m = max(m, wmax[w]);
    atomicMax(maxabs, m);
  }
  if (!ASIDE && threadIdx.x == 0 && corr2 && maxabs2) {
    int m = 0;
#pragma unroll
    for (int w = 0; w < SM_WAVES; w++) m = max(m, wmax[SM_WAVES + w]);
    atomicMax(maxabs2, m);
  }
}

template <int NB>
__global__ void __launch_bounds__(SM_THREADS) side_many_kernel(SideManyParams p) {
  extern __shared__ __attribute__((aligned(1024))) u8 ring[];
  __shared__ int wmax[2 * SM_WAVES];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tA = p.m / SM_ROWS, tB = p.n / SM_ROWS, nA = p.count * tA;
  const int b = blockIdx.x;
  if (b < nA) {
    const SideManyItem& I = p.it[b / tA];
    sm_side<NB, true>(ring, I.A, p.StB, I.SpA, I.EA, I.ApEA, I.corrA, p.corr_a_off, p.ecopy_off, I.maxabs, nullptr,
                      nullptr, nullptr, p.m, (b % tA) * SM_ROWS, p.k, p.lmax, wave, lane, wmax);
  } else {
    // B side: nonces 2 j and 2 j + 1 (if any) of pair j = (b - nA) / tB
    const int i0 = 2 * ((b - nA) / tB);
    const SideManyItem& I = p.it[i0];
    const bool two = i0 + 1 < p.count;
    const SideManyItem& J = p.it[two ? i0 + 1 : i0];
    sm_side<NB, false>(ring, p.Bp, I.StA, nullptr, nullptr, nullptr, I.corrB, p.corr_b_off, -1,
                       I.maxabs ? I.maxabs + 1 : nullptr, J.StA, two ? J.corrB : nullptr,
                       two && J.maxabs ? J.maxabs + 1 : nullptr, p.n, ((b - nA) % tB) * SM_ROWS, p.k, p.lmax, wave,
                       lane, wmax);
  }
}

template <int NB>
static void sm_go(dim3 grid, hipStream_t stream, const SideManyParams& p) {
  auto kern = side_many_kernel<NB>;
  static bool attr = false;  // one attribute call per instantiation (the library is process-wide)
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, sm_lds<NB>());
    attr = true;
  }
  hipLaunchKernelGGL(kern, grid, dim3(SM_THREADS), sm_lds<NB>(), stream, p);
}

static bool sm_aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

extern "C" int uwc_side_project_many(int count, const int8_t* const* A, const int8_t* const* EA,
                                     const int8_t* const* SpA, int8_t* const* ApEA, const int8_t* StB,
                                     int8_t* const* corrA, int corr_a_off, int ecopy_off, const int8_t* Bp,
                                     const int8_t* const* StA, int8_t* const* corrB, int corr_b_off, int m, int n,
                                     int k, int r, int32_t* const* maxabs, int lmax, hipStream_t stream) {
  static const char* fn = "uwc_side_project_many";
  if (count < 1 || count > SM_MAXB) return uwc_fail("%s: count=%d outside 1..%d", fn, count, SM_MAXB);
  if (!A || !EA || !SpA || !ApEA || !StB || !corrA || !Bp || !StA || !corrB || !maxabs)
    return uwc_fail("%s: null pointer or array argument", fn);
  if (m <= 0 || n <= 0 || k <= 0 || m % SM_ROWS || n % SM_ROWS || k % SM_CH)
    return uwc_fail("%s: m=%d and n=%d must be positive multiples of %d and k=%d of %d", fn, m, n, SM_ROWS, k, SM_CH);
  if (r != 16 && r != 32 && r != 64) return uwc_fail("%s: r=%d must be 16, 32 or 64", fn, r);
  if (lmax < 1 || lmax > 4) return uwc_fail("%s: lmax=%d must be 1..4", fn, lmax);
  if ((corr_a_off != 0 && corr_a_off != r) || (corr_b_off != 0 && corr_b_off != r) ||
      (ecopy_off >= 0 && ecopy_off != 0 && ecopy_off != r))
    return uwc_fail("%s: corr offsets must be 0 or r (ecopy_off may be -1)", fn);
  if (!sm_aligned16(StB) || !sm_aligned16(Bp)) return uwc_fail("%s: StB and Bp must be 16-byte aligned", fn);
  SideManyParams p{};
  p.StB = StB;
  p.Bp = Bp;
  p.m = m, p.n = n, p.k = k, p.r = r, p.lmax = lmax;
  p.corr_a_off = corr_a_off, p.ecopy_off = ecopy_off, p.corr_b_off = corr_b_off;
  p.count = count;
  for (int i = 0; i < count; i++) {
    if (!A[i] || !EA[i] || !SpA[i] || !ApEA[i] || !corrA[i] || !StA[i] || !corrB[i] || !maxabs[i])
      return uwc_fail("%s: item %d has a null pointer", fn, i);
    if (!sm_aligned16(A[i]) || !sm_aligned16(EA[i]) || !sm_aligned16(SpA[i]) || !sm_aligned16(ApEA[i]) ||
        !sm_aligned16(StA[i]) || (ecopy_off >= 0 && !sm_aligned16(corrA[i])))
      return uwc_fail("%s: item %d: A, EA, SpA, ApEA, StA (and corrA for the E copy) must be 16-byte aligned", fn, i);
    p.it[i] = SideManyItem{A[i], EA[i], SpA[i], ApEA[i], corrA[i], StA[i], corrB[i], maxabs[i]};
  }
  const dim3 grid(count * (m / SM_ROWS) + (count + 1) / 2 * (n / SM_ROWS));
  switch (r) {
    case 16: sm_go<1>(grid, stream, p); break;
    case 32: sm_go<2>(grid, stream, p); break;
    default: sm_go<4>(grid, stream, p); break;
  }
  return uwc_launch_status("side_project_many");
}
