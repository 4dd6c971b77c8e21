// Keyed BLAKE3 tree commitment of an operand and Pearl's salted seed derivation on gfx950
// (miner/ampere/uwc_ampere/kernels.cu:138-244, reference.py:41-64, ops.py:99-118).
//
// BLAKE3 over 16 MiB is 16384 independent chunk chains of 16 compressions each, then a
// 14-level tree. One operand alone is latency-bound, not throughput-bound: for small batches one
// compression is therefore
// spread over the 4 lanes of a quad: lane q holds column q of the 4 x 4 state
// (a = v[q], b = v[4+q], c = v[8+q], d = v[12+q]), runs the column G on it, and the diagonal
// step rotates b, c, d across the quad with DPP quad permutes (v0 v5 v10 v15 ... become one
// lane's a b c d). Message words reach each lane from LDS at precomputed per-lane offsets
// (lane q of round r reads words S[r][2q], S[r][2q+1], S[r][8+2q], S[r][9+2q]).
// This quarters the dependent instruction chain per compression and gives 4x the waves. Batches
// of four or more 16 MiB operands have the waves anyway and run one chunk per lane instead
// (b3_lanes_kernel: measured over 16 MiB operands, 20 per launch 157 -> 130 us, 32 per launch
// 228 -> 194 us; 1 per launch 31 -> 39 us, 2 per launch 38 -> 41 us).
#include "uwc_common.h"

#include <mutex>

#define QROT1 0x39  // quad_perm [1,2,3,0]: lane q takes lane (q+1) & 3
#define QROT2 0x4E  // quad_perm [2,3,0,1]
#define QROT3 0x93  // quad_perm [3,0,1,2]

template <int CTRL>
__device__ __forceinline__ u32 qperm(u32 x) {
  return (u32)__builtin_amdgcn_mov_dpp((int)x, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ void b3_g1(u32& a, u32& b, u32& c, u32& d, u32 x, u32 y) {
  a = a + b + x; d = rotr32(d ^ a, 16);
  c = c + d;     b = rotr32(b ^ c, 12);
  a = a + b + y; d = rotr32(d ^ a, 8);
  c = c + d;     b = rotr32(b ^ c, 7);
}

// Byte offsets, within a 16-word message, of the 28 words lane q consumes (round-major:
// column pair then diagonal pair).
struct QuadMsgOffsets {
  u32 o[28];
};

__device__ __forceinline__ QuadMsgOffsets quad_offsets(int q) {
  QuadMsgOffsets t;
#pragma unroll
  for (int r = 0; r < 7; r++) {
    t.o[4 * r + 0] = 4u * kB3Sched[r][2 * q];
    t.o[4 * r + 1] = 4u * kB3Sched[r][2 * q + 1];
    t.o[4 * r + 2] = 4u * kB3Sched[r][8 + 2 * q];
    t.o[4 * r + 3] = 4u * kB3Sched[r][9 + 2 * q];
  }
  return t;
}

// The 28 message words lane q of a quad consumes, read from a 16-word message in LDS.
__device__ __forceinline__ void quad_msg(const u8* msg, const QuadMsgOffsets& off, u32 m[28]) {
#pragma unroll
  for (int j = 0; j < 28; j++) m[j] = *reinterpret_cast<const u32*>(msg + off.o[j]);
}

// One compression by a quad on message words m (quad_msg). (ca, cb): this lane's chaining
// value words cv[q], cv[4+q]. Returns this lane's output words out[q] = a ^ c, out[4+q] = b ^ d.
__device__ __forceinline__ void quad_compress_m(const u32 m[28], int q, u32 ca, u32 cb, u64 counter, u32 blen,
                                                u32 flags, u32& lo, u32& hi) {
  u32 a = ca, b = cb, c = b3_iv(0), d = (u32)counter;
  // c = IV[q], d = (counter lo, counter hi, blen, flags)[q]
  if (q == 1) { c = b3_iv(1); d = (u32)(counter >> 32); }
  if (q == 2) { c = b3_iv(2); d = blen; }
  if (q == 3) { c = b3_iv(3); d = flags; }
#pragma unroll
  for (int r = 0; r < 7; r++) {
    b3_g1(a, b, c, d, m[4 * r], m[4 * r + 1]);
    b = qperm<QROT1>(b); c = qperm<QROT2>(c); d = qperm<QROT3>(d);
    b3_g1(a, b, c, d, m[4 * r + 2], m[4 * r + 3]);
    b = qperm<QROT3>(b); c = qperm<QROT2>(c); d = qperm<QROT1>(d);
  }
  lo = a ^ c;
  hi = b ^ d;
}

// The byte offsets of message word j (0..3) of round r for the 4 lanes of a quad, one per byte:
// lane q extracts byte q (one v_bfe), so no lane keeps a table of 28 offsets in registers.
__device__ constexpr u32 quad_off_pack(int r, int j) {
  u32 v = 0;
  for (int q = 0; q < 4; q++) {
    const int w = j < 2 ? kB3Sched[r][2 * q + j] : kB3Sched[r][8 + 2 * q + (j - 2)];
    v |= (u32)(4 * w) << (8 * q);
  }
  return v;
}

// quad_compress_m with the message words read from LDS round by round (4 live words instead of
// 28, offsets from quad_off_pack). q8 = 8 q; word w is read at msg + ((4 w) ^ xmask), for
// messages stored with their 16-byte quarters permuted by xmask (0 for a plain message).
__device__ __forceinline__ void quad_compress_rounds(const u8* msg, u32 q8, u32 xmask, int q, u32 ca, u32 cb,
                                                     u64 counter, u32 blen, u32 flags, u32& lo, u32& hi) {
  u32 a = ca, b = cb, c = b3_iv(0), d = (u32)counter;
  if (q == 1) { c = b3_iv(1); d = (u32)(counter >> 32); }
  if (q == 2) { c = b3_iv(2); d = blen; }
  if (q == 3) { c = b3_iv(3); d = flags; }
#pragma unroll
  for (int r = 0; r < 7; r++) {
    u32 o[4];
#pragma unroll
    for (int j = 0; j < 4; j++) o[j] = __builtin_amdgcn_ubfe(quad_off_pack(r, j), q8, 8) ^ xmask;
    const u32 m0 = *reinterpret_cast<const u32*>(msg + o[0]);
    const u32 m1 = *reinterpret_cast<const u32*>(msg + o[1]);
    const u32 m2 = *reinterpret_cast<const u32*>(msg + o[2]);
    const u32 m3 = *reinterpret_cast<const u32*>(msg + o[3]);
    b3_g1(a, b, c, d, m0, m1);
    b = qperm<QROT1>(b); c = qperm<QROT2>(c); d = qperm<QROT3>(d);
    b3_g1(a, b, c, d, m2, m3);
    b = qperm<QROT3>(b); c = qperm<QROT2>(c); d = qperm<QROT1>(d);
  }
  lo = a ^ c;
  hi = b ^ d;
}

// quad_compress_m on a message in LDS.
__device__ __forceinline__ void quad_compress(const u8* msg, const QuadMsgOffsets& off, int q, u32 ca, u32 cb,
                                              u64 counter, u32 blen, u32 flags, u32& lo, u32& hi) {
  u32 m[28];
  quad_msg(msg, off, m);
  quad_compress_m(m, q, ca, cb, counter, blen, flags, lo, hi);
}

// Level-wise pairwise reduction, by quads, of `count` chaining values in LDS (8 words each):
// pairs (2i, 2i+1) merge, an odd last value carries up. Over a group that starts at a multiple
// of a power of two covering it, this is exactly BLAKE3's left-complete tree.
__device__ __forceinline__ void quad_level_reduce(u32* cvs, int count, u32 k_lo, u32 k_hi, u32 kflag, bool root_at_end) {
  const int tid = threadIdx.x, q = tid & 3, quad = tid >> 2, nquads = blockDim.x >> 2;
  while (count > 1) {
    const int pairs = count >> 1;
    const bool last = (count == 2) && root_at_end;
    // up to 2 pairs per quad (groups of at most 4 * blockDim / 4 values)
    u32 lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;
    if (quad < pairs)
      quad_compress_rounds(reinterpret_cast<const u8*>(cvs + quad * 16), 8 * q, 0, q, k_lo, k_hi, 0, 64,
                           B3_PARENT | kflag | (last ? B3_ROOT : 0u), lo0, hi0);
    if (quad + nquads < pairs)
      quad_compress_rounds(reinterpret_cast<const u8*>(cvs + (quad + nquads) * 16), 8 * q, 0, q, k_lo, k_hi, 0, 64,
                           B3_PARENT | kflag, lo1, hi1);
    u32 carry = 0;
    const bool has_carry = (count & 1) && tid < 8;
    if (has_carry) carry = cvs[(count - 1) * 8 + tid];
    __syncthreads();
    if (quad < pairs) { cvs[quad * 8 + q] = lo0; cvs[quad * 8 + 4 + q] = hi0; }
    if (quad + nquads < pairs) { cvs[(quad + nquads) * 8 + q] = lo1; cvs[(quad + nquads) * 8 + 4 + q] = hi1; }
    if (has_carry) cvs[pairs * 8 + tid] = carry;
    __syncthreads();
    count = pairs + (count & 1);
  }
}

#define B3_CHUNKS_PER_WG 64
#define B3_RING 4  // blocks of every chunk in flight, per wave (the wait switch below covers up to 4)
#define B3_QSTRIDE 80  // LDS bytes per quad's message block in nonce_noise (64 + 16 pad: fewer bank conflicts)

// Inputs of a batch of equal-size commitments (blockIdx.y = item): one launch commits several
// operands at once.
#define B3_MAXB 32
struct B3In {
  const u8* data[B3_MAXB];
};
struct B3Out {
  u32* root[B3_MAXB];
  u32* seed[B3_MAXB];
};

typedef void __attribute__((address_space(3)))* b3_lptr;

__device__ __forceinline__ void b3_dma16(const void* g, u32 lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void b3_waitv() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// 64 chunks per workgroup (4 waves x 16 quads, one quad per chunk). A chunk is a chain of 16
// dependent compressions of ~180 dependent instructions each, and a batch of 8 operands is 8
// waves per SIMD of ~4100 VALU instructions each: at 4 cycles per wave64 VALU instruction the
// batch is VALU-bound (~63 us for 8 x 16 MiB), so the kernel keeps 6 waves per SIMD resident
// (78 VGPRs; at 8 the compiler spills) and its LDS reads free of bank conflicts. A wave streams
// its 16 chunks' blocks through its own LDS ring by DMA, B3_RING blocks ahead (lane l fetches
// bytes [16 (l & 3), + 16) of block b of chunk l / 4, so one DMA instruction brings one block of
// all 16 chunks); the ring is the wave's own, so no barrier is needed, only the wave's vmcnt. A
// lane reads the message words of each round from the ring at its precomputed offsets.
// Item blockIdx.y hashes bt.data[item] into wg_cvs + item * stride (stride in words).
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6)))
b3_chunks_kernel(B3In bt, u64 nchunks, const u32* __restrict__ key, u32* __restrict__ wg_cvs, u64 stride) {
  __shared__ __attribute__((aligned(16))) u8 ring[4][B3_RING][1024];  // [wave][slot][16 chunks x 64 bytes]
  __shared__ u32 cvs[B3_CHUNKS_PER_WG * 8];
  const u8* __restrict__ data = bt.data[blockIdx.y];
  wg_cvs += blockIdx.y * stride;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = tid & 3, c = tid >> 2;
  const u64 base = (u64)blockIdx.x * B3_CHUNKS_PER_WG;
  const int count = (int)min((u64)B3_CHUNKS_PER_WG, nchunks - base);
  const u32 k_lo = key[q], k_hi = key[4 + q];
  const bool active = c < count;
  // this lane's 16 bytes of every block (chunks past the end read the first chunk: not stored).
  // Chunk slot i of a ring entry holds the chunk's block with its 16-byte quarters permuted,
  // quarter p at position p ^ (i >> 2): lane 4 i + q fetches quarter q ^ (i >> 2). Chunks i and
  // i + 4 (64 bytes apart: the same banks) then keep any given word in different banks, and the
  // 16 quads' reads of one message word no longer collide 4 to a bank.
  const u32 xmask = lane & 48;  // (i >> 2) << 4
  const u8* src = data + (base + (active ? c : 0)) * 1024ull + ((q * 16) ^ xmask);
  const u32 rbase = __builtin_amdgcn_readfirstlane((u32)(uintptr_t)(b3_lptr)&ring[wave][0][0]);
#pragma unroll
  for (int b = 0; b < B3_RING; b++) b3_dma16(src + b * 64, rbase + b * 1024);
  u32 lo = k_lo, hi = k_hi;
#pragma unroll
  for (int b = 0; b < 16; b++) {
    // blocks b .. min(b + B3_RING - 1, 15) are in flight: wait for block b (the count folds to
    // a constant in the unrolled loop)
    switch (min(B3_RING - 1, 15 - b)) {
      case 0: b3_waitv<0>(); break;
      case 1: b3_waitv<1>(); break;
      case 2: b3_waitv<2>(); break;
      default: b3_waitv<3>(); break;
    }
    const u8* blk = &ring[wave][b % B3_RING][(lane >> 2) * 64];
    const u32 flags = B3_KEYED | (b == 0 ? B3_CHUNK_START : 0u) | (b == 15 ? B3_CHUNK_END : 0u) |
                      ((b == 15 && nchunks == 1) ? B3_ROOT : 0u);
    quad_compress_rounds(blk, 8 * q, xmask, q, lo, hi, base + c, 64, flags, lo, hi);
    if (b + B3_RING < 16) {
      // the slot's reads are done (their values were used above) before the DMA overwrites it
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      b3_dma16(src + (b + B3_RING) * 64, rbase + (b % B3_RING) * 1024);
    }
  }
  if (active) { cvs[c * 8 + q] = lo; cvs[c * 8 + 4 + q] = hi; }
  __syncthreads();
  quad_level_reduce(cvs, count, k_lo, k_hi, B3_KEYED, gridDim.x == 1);
  if (tid < 8) wg_cvs[blockIdx.x * 8 + tid] = cvs[tid];
}

// The same chunk values with one chunk per lane, for batches large enough to give every SIMD
// several waves: a lane runs the plain 16-word compression (b3_compress), so a compression costs
// 64 lanes' ~700 VALU instructions per 64 chunks instead of the quad form's ~1290 lane
// instructions per chunk (its DPP rotations and per-round LDS message reads are gone), at 4x
// the dependent chain per wave. A lane reads its chunk's 64-byte blocks straight from memory
// (four 16-byte loads; the next block's loads are issued before the current block's
// compression), and 256 chunks per workgroup reduce to one subtree value in LDS. 61 VGPRs, so 8
// waves per SIMD: 32 operands (8,192 waves) run in one round instead of 7 waves per SIMD and a
// partial second round (measured 196.7 -> 193.4 us for 32, 135.6 -> 132.4 us for 20).
#define B3L_CHUNKS_PER_WG 256
#ifndef B3_LANES_MIN_CHUNKS
#define B3_LANES_MIN_CHUNKS (1u << 16)  // 4 operands of 16 MiB (1 wave per SIMD): from there on the lane form is faster
#endif

__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8)))
b3_lanes_kernel(B3In bt, u64 nchunks, const u32* __restrict__ key, u32* __restrict__ wg_cvs, u64 stride) {
  __shared__ u32 cvs[B3L_CHUNKS_PER_WG * 8];
  const u8* __restrict__ data = bt.data[blockIdx.y];
  wg_cvs += blockIdx.y * stride;
  const int tid = threadIdx.x, q = tid & 3;
  const u64 base = (u64)blockIdx.x * B3L_CHUNKS_PER_WG;
  const int count = (int)min((u64)B3L_CHUNKS_PER_WG, nchunks - base);
  const bool active = tid < count;
  // chunks past the end read the first chunk of the workgroup (not stored)
  const uint4* __restrict__ src = reinterpret_cast<const uint4*>(data + (base + (active ? tid : 0)) * 1024ull);
  u32 cv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) cv[i] = key[i];
  uint4 nx[4];
#pragma unroll
  for (int j = 0; j < 4; j++) nx[j] = src[j];
  const u64 chunk = base + tid;
#pragma unroll 1
  for (int b = 0; b < 16; b++) {
    u32 m[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      m[4 * j] = nx[j].x; m[4 * j + 1] = nx[j].y; m[4 * j + 2] = nx[j].z; m[4 * j + 3] = nx[j].w;
    }
    if (b < 15) {
#pragma unroll
      for (int j = 0; j < 4; j++) nx[j] = src[4 * (b + 1) + j];
    }
    const u32 flags = B3_KEYED | (b == 0 ? B3_CHUNK_START : 0u) | (b == 15 ? B3_CHUNK_END : 0u) |
                      ((b == 15 && nchunks == 1) ? B3_ROOT : 0u);
    b3_compress(cv, m, chunk, 64, flags, cv);
  }
  if (active) {
#pragma unroll
    for (int i = 0; i < 8; i++) cvs[tid * 8 + i] = cv[i];
  }
  __syncthreads();
  quad_level_reduce(cvs, count, key[q], key[4 + q], B3_KEYED, gridDim.x == 1);
  if (tid < 8) wg_cvs[blockIdx.x * 8 + tid] = cvs[tid];
}

#define B3_GROUP 1024
// Reduces aligned groups of up to 1024 chaining values (256 threads = 64 quads). With a single
// group (final), the last merge carries ROOT and the salted seed may follow:
//   seed = BLAKE3(prefix || keyed_BLAKE3(salt, root || dim_le32 || 0^28))
// (Pearl's v3 derivation: b_seed with prefix = job_key, a_seed with prefix = b_seed).
// Item blockIdx.y of a batch reads in_cvs + item * stride and writes out_cvs + item * stride (or,
// in the final launch, outs.root[item] and outs.seed[item], either may be NULL).
__global__ void __launch_bounds__(256) b3_reduce_kernel(const u32* __restrict__ in_cvs, int count,
                                                        const u32* __restrict__ key, u32* __restrict__ out_cvs,
                                                        u64 stride, int final_level, const u32* __restrict__ prefix,
                                                        const u32* __restrict__ salt, u32 dim, B3Out outs) {
  __shared__ __attribute__((aligned(16))) u32 cvs[B3_GROUP * 8];
  in_cvs += blockIdx.y * stride;
  if (out_cvs) out_cvs += blockIdx.y * stride;
  u32* __restrict__ root_out = outs.root[blockIdx.y];
  u32* __restrict__ seed_out = outs.seed[blockIdx.y];
  const int tid = threadIdx.x, q = tid & 3;
  const int base = blockIdx.x * B3_GROUP, cnt = min(B3_GROUP, count - base);
  for (int i = tid; i < cnt * 8; i += blockDim.x) cvs[i] = in_cvs[(u64)base * 8 + i];
  __syncthreads();
  const QuadMsgOffsets off = quad_offsets(q);
  const u32 k_lo = key[q], k_hi = key[4 + q];
  // level 0 has up to 512 pairs for 64 quads: reduce in passes of 128 pairs (2 per quad)
  int c2 = cnt;
  while (c2 > 256) {
    // pairwise merge of the first 256 values, then of the next 256, ... keeping order
    const int pairs = c2 >> 1;
    for (int p0 = 0; p0 < pairs; p0 += 128) {
      const int quad = tid >> 2;
      u32 lo0 = 0, hi0 = 0, lo1 = 0, hi1 = 0;
      const int pa = p0 + quad, pb = p0 + quad + 64;
      if (pa < pairs)
        quad_compress(reinterpret_cast<const u8*>(cvs + pa * 16), off, q, k_lo, k_hi, 0, 64, B3_PARENT | B3_KEYED, lo0,
                      hi0);
      if (pb < pairs)
        quad_compress(reinterpret_cast<const u8*>(cvs + pb * 16), off, q, k_lo, k_hi, 0, 64, B3_PARENT | B3_KEYED, lo1,
                      hi1);
      __syncthreads();
      // pair p's output goes to slot p: slots below p0 are final already, slots >= p0 are
      // read only by pairs >= p0, which this pass has consumed
      if (pa < pairs) { cvs[pa * 8 + q] = lo0; cvs[pa * 8 + 4 + q] = hi0; }
      if (pb < pairs) { cvs[pb * 8 + q] = lo1; cvs[pb * 8 + 4 + q] = hi1; }
      __syncthreads();
    }
    if (c2 & 1) {
      u32 carry = tid < 8 ? cvs[(c2 - 1) * 8 + tid] : 0u;
      __syncthreads();
      if (tid < 8) cvs[pairs * 8 + tid] = carry;
      __syncthreads();
    }
    c2 = pairs + (c2 & 1);
  }
  quad_level_reduce(cvs, c2, k_lo, k_hi, B3_KEYED, final_level != 0);
  if (!final_level) {
    if (tid < 8) out_cvs[blockIdx.x * 8 + tid] = cvs[tid];
    return;
  }
  // root, then the seed: two one-block hashes by quad 0 (messages staged in LDS)
  u32* msg = cvs + 16;
  if (tid < 8) {
    if (root_out) root_out[tid] = cvs[tid];
    msg[tid] = cvs[tid];
    msg[8 + tid] = tid == 0 ? dim : 0u;
  }
  if (!seed_out) return;
  __syncthreads();
  u32 lo = 0, hi = 0;
  if (tid < 4)
    quad_compress(reinterpret_cast<const u8*>(msg), off, q, salt[q], salt[4 + q], 0, 64,
                  B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, lo, hi);
  __syncthreads();
  if (tid < 4) { msg[8 + q] = lo; msg[12 + q] = hi; }
  if (tid < 8) msg[tid] = prefix[tid];
  __syncthreads();
  if (tid < 4) {
    quad_compress(reinterpret_cast<const u8*>(msg), off, q, b3_iv(q), b3_iv(4 + q), 0, 64,
                  B3_CHUNK_START | B3_CHUNK_END | B3_ROOT, lo, hi);
    seed_out[q] = lo;
    seed_out[4 + q] = hi;
  }
}

extern "C" int uwc_b3_scratch_words(uint64_t nbytes) {
  const u64 nch = nbytes / 1024, nwg = (nch + B3_CHUNKS_PER_WG - 1) / B3_CHUNKS_PER_WG;
  u64 words = nwg * 8, cnt = nwg;
  while (cnt > B3_GROUP) {  // intermediate levels are kept after the first one
    cnt = (cnt + B3_GROUP - 1) / B3_GROUP;
    words += cnt * 8;
  }
  return words > 0x7fffffff ? -1 : (int)words;
}

// Commitments (and seeds) of `count` equal-size inputs; item i uses scratch words
// [i * stride, (i + 1) * stride).
static int b3_launch(const B3In& in, int count, u64 nbytes, const u32* key, const u32* prefix, const u32* salt, u32 dim,
                     const B3Out& outs, u32* scratch, u64 stride, hipStream_t stream) {
  // subtree values per item: one per workgroup, in at most the words uwc_b3_scratch_words counts
  // (a workgroup of the lane form covers more chunks than one of the quad form)
  const u64 nch = nbytes / 1024;
  int cnt;
  if ((u64)count * nch >= B3_LANES_MIN_CHUNKS) {
    cnt = (int)((nch + B3L_CHUNKS_PER_WG - 1) / B3L_CHUNKS_PER_WG);
    hipLaunchKernelGGL(b3_lanes_kernel, dim3(cnt, count), dim3(256), 0, stream, in, nch, key, scratch, stride);
  } else {
    cnt = (int)((nch + B3_CHUNKS_PER_WG - 1) / B3_CHUNKS_PER_WG);
    hipLaunchKernelGGL(b3_chunks_kernel, dim3(cnt, count), dim3(256), 0, stream, in, nch, key, scratch, stride);
  }
  int st = uwc_launch_status("b3_chunks");
  if (st) return st;
  u32* cur = scratch;
  while (cnt > B3_GROUP) {
    const int groups = (cnt + B3_GROUP - 1) / B3_GROUP;
    u32* nxt = cur + (u64)cnt * 8;
    hipLaunchKernelGGL(b3_reduce_kernel, dim3(groups, count), dim3(256), 0, stream, cur, cnt, key, nxt, stride, 0,
                       nullptr, nullptr, 0u, B3Out{});
    if ((st = uwc_launch_status("b3_reduce"))) return st;
    cur = nxt;
    cnt = groups;
  }
  hipLaunchKernelGGL(b3_reduce_kernel, dim3(1, count), dim3(256), 0, stream, cur, cnt, key, nullptr, stride, 1, prefix,
                     salt, dim, outs);
  return uwc_launch_status("b3_reduce_final");
}

static int b3_check(u64 nbytes, const u32* key, const u32* prefix, const u32* salt, bool seeds, const char* fn) {
  if (!key) return uwc_fail("%s: null key", fn);
  if (nbytes == 0 || nbytes % 1024)
    return uwc_fail("%s: nbytes=%llu must be a positive multiple of 1024", fn, (unsigned long long)nbytes);
  if (seeds && (!prefix || !salt)) return uwc_fail("%s: a seed needs prefix and salt", fn);
  if (uwc_b3_scratch_words(nbytes) < 0) return uwc_fail("%s: input too large", fn);
  return 0;
}

extern "C" int uwc_b3_root_and_seed(const uint8_t* data, uint64_t nbytes, const uint32_t* key, const uint32_t* prefix,
                                    const uint32_t* salt, uint32_t dim, uint32_t* root_out, uint32_t* seed_out,
                                    uint32_t* scratch, uint64_t scratch_words, hipStream_t stream) {
  if (!data || !scratch) return uwc_fail("uwc_b3_root_and_seed: null data or scratch");
  if (int st = b3_check(nbytes, key, prefix, salt, seed_out != nullptr, "uwc_b3_root_and_seed")) return st;
  if (((uintptr_t)data & 15u) != 0) return uwc_fail("uwc_b3_root_and_seed: data must be 16-byte aligned");
  const int need = uwc_b3_scratch_words(nbytes);
  if (scratch_words < (u64)need)
    return uwc_fail("uwc_b3_root_and_seed: scratch has %llu words, needs %d", (unsigned long long)scratch_words, need);
  B3In in{};
  B3Out outs{};
  in.data[0] = data;
  outs.root[0] = root_out;
  outs.seed[0] = seed_out;
  return b3_launch(in, 1, nbytes, key, prefix, salt, dim, outs, scratch, (u64)need, stream);
}

extern "C" int uwc_b3_root_and_seed_many(const uint8_t* const* data, int count, uint64_t nbytes, const uint32_t* key,
                                         const uint32_t* prefix, const uint32_t* salt, uint32_t dim,
                                         uint32_t* const* root_out, uint32_t* const* seed_out, uint32_t* scratch,
                                         uint64_t scratch_words, hipStream_t stream) {
  if (!data || !scratch) return uwc_fail("uwc_b3_root_and_seed_many: null data array or scratch");
  if (count < 1 || count > B3_MAXB) return uwc_fail("uwc_b3_root_and_seed_many: count=%d must be 1..%d", count, B3_MAXB);
  if (int st = b3_check(nbytes, key, prefix, salt, seed_out != nullptr, "uwc_b3_root_and_seed_many")) return st;
  const int need = uwc_b3_scratch_words(nbytes);
  if (scratch_words < (u64)need * count)
    return uwc_fail("uwc_b3_root_and_seed_many: scratch has %llu words, needs %llu", (unsigned long long)scratch_words,
                    (unsigned long long)need * count);
  B3In in{};
  B3Out outs{};
  for (int i = 0; i < count; i++) {
    if (!data[i] || ((uintptr_t)data[i] & 15u))
      return uwc_fail("uwc_b3_root_and_seed_many: data[%d] is null or not 16-byte aligned", i);
    if ((root_out && !root_out[i]) || (seed_out && !seed_out[i]))
      return uwc_fail("uwc_b3_root_and_seed_many: root_out[%d] / seed_out[%d] is null", i, i);
    in.data[i] = data[i];
    outs.root[i] = root_out ? root_out[i] : nullptr;
    outs.seed[i] = seed_out ? seed_out[i] : nullptr;
  }
  return b3_launch(in, count, nbytes, key, prefix, salt, dim, outs, scratch, (u64)need, stream);
}

// ------------------------------------------------------------------ allocation-free commitment
// uwc_b3_root_and_seed for callers that cannot allocate (code under graph capture, serving loops):
// the workspace the chunk and reduce kernels pass subtree values through is a file-scope device
// array instead of a caller's buffer, sized for inputs up to UWC_B3_STATIC_MAX_BYTES. Each GPU
// the library runs on holds its own copy until the process ends. Host code never uses the
// array's name as an address: the first call on a device looks its device address up with
// hipGetSymbolAddress and keeps it per device. Every call on one GPU shares that GPU's array, so
// calls that overlap on one GPU (on different streams) race; calls on one stream are ordered.
// Nothing in the workspace needs to start at zero: the chunk kernel writes every value a
// reduction then reads, and the previous call's contents are overwritten.
#define UWC_B3_STATIC_MAX_BYTES (1ull << 30)
#define UWC_MAX_DEVICES 64

constexpr u64 b3_words_for(u64 nbytes) {
  u64 cnt = (nbytes / 1024 + B3_CHUNKS_PER_WG - 1) / B3_CHUNKS_PER_WG, words = cnt * 8;
  while (cnt > B3_GROUP) {
    cnt = (cnt + B3_GROUP - 1) / B3_GROUP;
    words += cnt * 8;
  }
  return words;
}
#define B3_STATIC_WORDS b3_words_for(UWC_B3_STATIC_MAX_BYTES)
static_assert(B3_STATIC_WORDS == 131200, "1 GiB: 16384 subtree values, then 16 group values");

static __device__ __align__(256) u32 b3_static_scratch[B3_STATIC_WORDS];

static std::mutex g_b3_static_mu;
static u32* g_b3_static_ptr[UWC_MAX_DEVICES];  // device address of b3_static_scratch, per device

// The current device's address of b3_static_scratch (looked up once per device), or NULL after
// recording the error.
static u32* b3_static_workspace(const char* fn) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= UWC_MAX_DEVICES) {
    uwc_fail("%s: no usable current device (%d)", fn, dev);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_b3_static_mu);
  if (!g_b3_static_ptr[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(b3_static_scratch));
    if (e != hipSuccess || !ptr) {
      uwc_fail("%s: hipGetSymbolAddress of the static workspace failed on device %d: %s", fn, dev,
               hipGetErrorString(e));
      return nullptr;
    }
    g_b3_static_ptr[dev] = static_cast<u32*>(ptr);
  }
  return g_b3_static_ptr[dev];
}

extern "C" int uwc_b3_root_and_seed_static(const uint8_t* data, uint64_t nbytes, const uint32_t* key,
                                           const uint32_t* prefix, const uint32_t* salt, uint32_t dim,
                                           uint32_t* root_out, uint32_t* seed_out, hipStream_t stream) {
  static const char* fn = "uwc_b3_root_and_seed_static";
  if (!data) return uwc_fail("%s: null data", fn);
  if (int st = b3_check(nbytes, key, prefix, salt, seed_out != nullptr, fn)) return st;
  if (nbytes > UWC_B3_STATIC_MAX_BYTES)
    return uwc_fail("%s: %llu bytes exceed the static workspace's maximum of %llu bytes (use uwc_b3_root_and_seed "
                    "with a scratch buffer)", fn, (unsigned long long)nbytes, (unsigned long long)UWC_B3_STATIC_MAX_BYTES);
  if (((uintptr_t)data & 15u) != 0) return uwc_fail("%s: data must be 16-byte aligned", fn);
  u32* ws = b3_static_workspace(fn);
  if (!ws) return UWC_EINVAL;
  B3In in{};
  B3Out outs{};
  in.data[0] = data;
  outs.root[0] = root_out;
  outs.seed[0] = seed_out;
  return b3_launch(in, 1, nbytes, key, prefix, salt, dim, outs, ws, b3_words_for(nbytes), stream);
}

// ------------------------------------------------------------------ per-nonce noise in one launch
// E (rows x r, the uniform_matrix), P (k pairs) and optionally St (the r x k selection matrix
// of P) and SpT (its transpose as k rows of 64 bytes, zero past r) from one keyed random_hash
// per quad (reference.py:67-93, kernels.cu:246-301, ops.py:152-158), and zeroes two counter
// ranges, in a single latency-bound launch instead of four. Workgroups [0, nE) make E blocks
// (one lane per 32-byte block: the plain compression issues about half the instructions of the
// quad form, and a group's thousands of blocks give every SIMD waves anyway); the rest make 8
// pairs per quad. A P wave owns 128 consecutive
// columns: it builds their St rows (r x 128 bytes) and SpT rows (128 x 64 bytes) in LDS by a
// zero fill and a 2-byte scatter per pair, then writes them with 16-byte stores (column-wise
// byte stores of St cost several times more).
#define NN_COLS 128  // columns per P wave
#define NN_EBLK 256  // E blocks per workgroup (one per lane)

__device__ __forceinline__ void pair_of(u32 u, u32 r, u32& first, u32& second) {
  first = u & (r - 1);
  second = first ^ (1u + __umulhi(r - 1, u));
}

// Per-item outputs of a batch of nonces (blockIdx.y = item); St, SpT, z0, z1 entries are all NULL
// or all set.
struct NNBatch {
  i8* E[B3_MAXB];
  u32* P[B3_MAXB];
  i8* St[B3_MAXB];
  i8* SpT[B3_MAXB];
  const u32* key[B3_MAXB];
  i32* z0[B3_MAXB];
  i32* z1[B3_MAXB];
};

__global__ void __launch_bounds__(256) nonce_noise_kernel(NNBatch nb, u32 eblocks, u32 nE, u32 k, u32 r,
                                                          const u32* __restrict__ label, int n0, int n1) {
  __shared__ __attribute__((aligned(16))) u8 msgs[64 * B3_QSTRIDE];
  extern __shared__ __attribute__((aligned(16))) u8 nn_blk[];  // per P wave: St [r][128], SpT [128][64]
  const int item = blockIdx.y;
  i8* __restrict__ E = nb.E[item];
  u32* __restrict__ P = nb.P[item];
  i8* __restrict__ St = nb.St[item];
  i8* __restrict__ SpT = nb.SpT[item];
  const u32* __restrict__ key = nb.key[item];
  i32* __restrict__ z0 = nb.z0[item];
  i32* __restrict__ z1 = nb.z1[item];
  const int tid = threadIdx.x, q = tid & 3, lq = tid >> 2, lane = tid & 63, wave = tid >> 6;
  if (blockIdx.x == 0) {
    if (z0 && tid < n0) z0[tid] = 0;
    if (z1 && tid < n1) z1[tid] = 0;
  }
  if (blockIdx.x < nE) {
    // E block `index` (32 bytes) per lane: the keyed digest of message word 0 = 1 + index, words
    // 8..15 = label, the rest 0, as one lane's plain compression; digest bytes -> (y & 63) - 32:
    // the 6-bit value (y & 63) ^ 32 sign-extended per byte
    const u32 index = blockIdx.x * NN_EBLK + tid;
    if (index < eblocks) {
      u32 m[16], kv[8], o[8];
      m[0] = 1u + index;
#pragma unroll
      for (int i = 1; i < 8; i++) m[i] = 0u;
#pragma unroll
      for (int i = 0; i < 8; i++) { m[8 + i] = label[i]; kv[i] = key[i]; }
      b3_compress(kv, m, 0, 64, B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, o);
      u32* dst = reinterpret_cast<u32*>(E + (u64)index * 32);
#pragma unroll
      for (int w = 0; w < 8; w++) {
        const u32 z = (o[w] & 0x3F3F3F3Fu) ^ 0x20202020u, sg = z & 0x20202020u;
        dst[w] = z | (sg << 1) | (sg << 2);
      }
    }
    return;
  }
  const u32 index = (blockIdx.x - nE) * 64 + lq;  // pair octet
  // message words 4q..4q+3 of msg: 0 except word 1 = 1 + index; words 8..15 = label
  u32* mw = reinterpret_cast<u32*>(msgs + lq * B3_QSTRIDE);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int w = 4 * q + i;
    mw[w] = w >= 8 ? label[w - 8] : (w == 1 ? 1u + index : 0u);
  }
  __builtin_amdgcn_wave_barrier();
  const QuadMsgOffsets off = quad_offsets(q);
  u32 lo, hi;
  quad_compress(msgs + lq * B3_QSTRIDE, off, q, key[q], key[4 + q], 0, 64,
                B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, lo, hi);
  // pairs l = 8 index + q + 4 h
  u32 f[2], sc[2];
  bool v[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const u32 l = index * 8 + q + 4 * h;
    v[h] = l < k;
    pair_of(h ? hi : lo, r, f[h], sc[h]);
    if (v[h]) P[l] = f[h] | (sc[h] << 16);
  }
  if (!St && !SpT) return;
  if (r > 128) {  // large r: St column by column (SpT needs r <= 64)
#pragma unroll
    for (int h = 0; h < 2; h++)
      if (v[h] && St)
        for (u32 j = 0; j < r; j++)
          St[(u64)j * k + index * 8 + q + 4 * h] = (i8)((int)(f[h] == j) - (int)(sc[h] == j));
    return;
  }
  const int stb = St ? (int)r * NN_COLS : 0, blk = stb + (SpT ? NN_COLS * 64 : 0);
  u8* wst = nn_blk + wave * blk;  // this wave's St block, then its SpT block
  u8* wsp = wst + stb;
  for (int i = lane * 16; i < blk; i += 64 * 16) *reinterpret_cast<v4i*>(wst + i) = v4i{0, 0, 0, 0};
  __builtin_amdgcn_wave_barrier();  // a wave's LDS accesses complete in order
#pragma unroll
  for (int h = 0; h < 2; h++) {
    if (!v[h]) continue;
    const int c = (lq & 15) * 8 + q + 4 * h;  // column within the wave's 128
    if (St) { wst[f[h] * NN_COLS + c] = 1; wst[sc[h] * NN_COLS + c] = 0xFF; }
    if (SpT) { wsp[c * 64 + f[h]] = 1; wsp[c * 64 + sc[h]] = 0xFF; }
  }
  __builtin_amdgcn_wave_barrier();
  const u32 l0 = ((blockIdx.x - nE) * 64 + wave * 16) * 8;
  if (St) {
    const bool vec = (k % 16) == 0;
    for (int idx = lane; idx < (int)r * 8; idx += 64) {
      const int j = idx >> 3, cc = idx & 7;
      const u32 col = l0 + 16 * cc;
      if (col >= k) continue;
      const v4i d = *reinterpret_cast<const v4i*>(wst + j * NN_COLS + 16 * cc);
      if (vec) {
        *reinterpret_cast<v4i*>(St + (u64)j * k + col) = d;
      } else {
        for (int b = 0; b < 16 && col + b < k; b++) St[(u64)j * k + col + b] = (i8)(((u32)d[b >> 2] >> (8 * (b & 3))) & 0xFF);
      }
    }
  }
  if (SpT)
    for (int idx = lane; idx < NN_COLS * 4; idx += 64) {
      const int c = idx >> 2, cc = idx & 3;
      if (l0 + c < k)
        *reinterpret_cast<v4i*>(SpT + (u64)(l0 + c) * 64 + 16 * cc) = *reinterpret_cast<const v4i*>(wsp + c * 64 + 16 * cc);
    }
}

static int nn_launch(const NNBatch& nb, int count, int rows, int r, int k, bool st, bool spt, const uint32_t* label,
                     int n0, int n1, hipStream_t stream, const char* fn) {
  if (!label || rows < 0 || k < 0) return uwc_fail("%s: null label or negative sizes", fn);
  if (spt && r > 64) return uwc_fail("%s: SpT needs r <= 64", fn);
  if (r < 2 || r > 65536 || (r & (r - 1))) return uwc_fail("%s: r=%d must be a power of two", fn, r);
  if (((u64)rows * r) % 32) return uwc_fail("%s: rows * r must be a multiple of 32", fn);
  if (n0 < 0 || n1 < 0 || n0 > 256 || n1 > 256) return uwc_fail("%s: zero ranges must be 0..256 words", fn);
  for (int i = 0; i < count; i++) {
    if (!nb.E[i] || !nb.P[i] || !nb.key[i]) return uwc_fail("%s: item %d has a null E, P or key", fn, i);
    if ((uintptr_t)nb.E[i] & 3u) return uwc_fail("%s: E must be 4-byte aligned", fn);
    if (spt && (!nb.SpT[i] || ((uintptr_t)nb.SpT[i] & 15u)))
      return uwc_fail("%s: SpT[%d] is null or not 16-byte aligned", fn, i);
    if (st && !nb.St[i]) return uwc_fail("%s: St[%d] is null", fn, i);
    if ((n0 && !nb.z0[i]) || (n1 && !nb.z1[i])) return uwc_fail("%s: zero range of item %d without a pointer", fn, i);
  }
  const u64 eblocks = (u64)rows * r / 32, nE = (eblocks + NN_EBLK - 1) / NN_EBLK, nP = (((u64)k + 7) / 8 + 63) / 64;
  const u64 blocks = nE + nP > 0 ? nE + nP : 1;
  if (blocks > 0x7fffffff) return uwc_fail("%s: too large", fn);
  const size_t smem = r <= 128 ? (size_t)4 * ((st ? (size_t)r * NN_COLS : 0) + (spt ? NN_COLS * 64 : 0)) : 0;
  static bool attr = false;  // one attribute call (96 KiB at r = 128 with SpT absent, 64 KiB + 32 KiB max)
  if (!attr) {
    (void)hipFuncSetAttribute((const void*)nonce_noise_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                              4 * (128 * NN_COLS + NN_COLS * 64));
    attr = true;
  }
  hipLaunchKernelGGL(nonce_noise_kernel, dim3((unsigned)blocks, count), dim3(256), smem, stream, nb, (u32)eblocks,
                     (u32)nE, (u32)k, (u32)r, label, n0, n1);
  return uwc_launch_status("nonce_noise");
}

extern "C" int uwc_nonce_noise(int8_t* E, int rows, int r, uint32_t* P, int k, int8_t* St, int8_t* SpT,
                               const uint32_t* label, const uint32_t* key, int32_t* zero0, int n0, int32_t* zero1, int n1,
                               hipStream_t stream) {
  NNBatch nb{};
  nb.E[0] = E;
  nb.P[0] = P;
  nb.St[0] = St;
  nb.SpT[0] = SpT;
  nb.key[0] = key;
  nb.z0[0] = zero0;
  nb.z1[0] = zero1;
  return nn_launch(nb, 1, rows, r, k, St != nullptr, SpT != nullptr, label, n0, n1, stream, "uwc_nonce_noise");
}

extern "C" int uwc_nonce_noise_many(int count, int8_t* const* E, int rows, int r, uint32_t* const* P, int k,
                                    int8_t* const* St, int8_t* const* SpT, const uint32_t* label,
                                    const uint32_t* const* key, int32_t* const* zero0, int n0, int32_t* const* zero1,
                                    int n1, hipStream_t stream) {
  if (!E || !P || !key) return uwc_fail("uwc_nonce_noise_many: null E, P or key array");
  if (count < 1 || count > B3_MAXB) return uwc_fail("uwc_nonce_noise_many: count=%d must be 1..%d", count, B3_MAXB);
  NNBatch nb{};
  for (int i = 0; i < count; i++) {
    nb.E[i] = E[i];
    nb.P[i] = P[i];
    nb.St[i] = St ? St[i] : nullptr;
    nb.SpT[i] = SpT ? SpT[i] : nullptr;
    nb.key[i] = key[i];
    nb.z0[i] = zero0 ? zero0[i] : nullptr;
    nb.z1[i] = zero1 ? zero1[i] : nullptr;
  }
  return nn_launch(nb, count, rows, r, k, St != nullptr, SpT != nullptr, label, n0, n1, stream, "uwc_nonce_noise_many");
}
