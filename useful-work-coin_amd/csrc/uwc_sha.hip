// Stage commitments on gfx950: SHA-256 row roots, tagged leaves and Merkle roots, identical to
// runtime/detrt/stage.py:33-77 (RFC 6962 trees: leaf = H(0x00 || x), node = H(0x01 || l || r),
// split at the largest power of two) and the stage-output root of
// spec/stage-program.md:82-88 (leaf H(0x00 || "sout" || u32le t || row_root)); the reference's
// GPU twin is runtime/detgpu/sha.py:19-153.
//
//   row root     rows are little-endian 4-byte words cut into 1 KiB blocks; one thread hashes
//                one block (17 compressions for a full block); the per-row tree is built
//                bottom-up, pairing neighbours and promoting an odd last node, which equals
//                the recursive split;
//   tagged leaf  H(0x00 || tag || u32le index || row_root), index = (base + row) % mod;
//   tree root    one workgroup per tree of n leaves, bottom-up through a scratch buffer.
//
// Every message here is a prefix byte followed by a stream of 32-bit words (row words, digest
// words, the tag and index words). With the stream in big-endian order Z_0 .. Z_{n-1} and
// Z_{-1} = the prefix byte, message word j is (Z_{j-1} << 24) | (Z_j >> 8): the one-byte
// prefix shifts the stream by a byte, so no byte-wise packing is needed. SHA-256 itself is
// restated from FIPS 180-4 (constants: fractional parts of the cube and square roots of the
// first primes).
#include "uwc_common.h"

__device__ __constant__ u32 kSha256K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
    0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
    0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
    0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
    0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
    0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

__device__ __forceinline__ void sha_init(u32 s[8]) {
  s[0] = 0x6a09e667u; s[1] = 0xbb67ae85u; s[2] = 0x3c6ef372u; s[3] = 0xa54ff53au;
  s[4] = 0x510e527fu; s[5] = 0x9b05688cu; s[6] = 0x1f83d9abu; s[7] = 0x5be0cd19u;
}

__device__ __forceinline__ u32 ror(u32 x, int n) { return __builtin_amdgcn_alignbit(x, x, n); }

// The three-input bitwise functions as single v_bitop3_b32 instructions (truth tables over the
// operand masks 0xF0, 0xCC, 0xAA): x ^ y ^ z, Ch(x, y, z) = x ? y : z, Maj(x, y, z).
__device__ __forceinline__ u32 sha_xor3(u32 x, u32 y, u32 z) { return __builtin_amdgcn_bitop3_b32(x, y, z, 0x96); }
__device__ __forceinline__ u32 sha_ch(u32 x, u32 y, u32 z) { return __builtin_amdgcn_bitop3_b32(x, y, z, 0xCA); }
__device__ __forceinline__ u32 sha_maj(u32 x, u32 y, u32 z) { return __builtin_amdgcn_bitop3_b32(x, y, z, 0xE8); }

// One compression of the 16-word block w (big-endian words) into s.
__device__ __forceinline__ void sha_compress(u32 s[8], u32 w[16]) {
  u32 a = s[0], b = s[1], c = s[2], d = s[3], e = s[4], f = s[5], g = s[6], h = s[7];
#pragma unroll
  for (int i = 0; i < 64; i++) {
    u32 wi;
    if (i < 16) {
      wi = w[i];
    } else {
      const u32 w15 = w[(i + 1) & 15], w2 = w[(i + 14) & 15];
      const u32 s0 = sha_xor3(ror(w15, 7), ror(w15, 18), w15 >> 3);
      const u32 s1 = sha_xor3(ror(w2, 17), ror(w2, 19), w2 >> 10);
      wi = w[i & 15] = w[i & 15] + s0 + w[(i + 9) & 15] + s1;
    }
    const u32 S1 = sha_xor3(ror(e, 6), ror(e, 11), ror(e, 25));
    const u32 ch = sha_ch(e, f, g);
    const u32 t1 = h + S1 + ch + kSha256K[i] + wi;
    const u32 S0 = sha_xor3(ror(a, 2), ror(a, 13), ror(a, 22));
    const u32 mj = sha_maj(a, b, c);
    h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + S0 + mj;
  }
  s[0] += a; s[1] += b; s[2] += c; s[3] += d; s[4] += e; s[5] += f; s[6] += g; s[7] += h;
}

// SHA-256 of (prefix byte || z[0..n) as big-endian words) for a short stream held in
// registers (n <= 16, compile time).
template <int N>
__device__ __forceinline__ void sha_short(u32 prefix, const u32 z[N], u32 out[8]) {
  constexpr int NB = (4 * N + 1 + 1 + 8 + 63) / 64;  // 64-byte blocks after padding
  u32 w[NB * 16];
#pragma unroll
  for (int j = 0; j < NB * 16; j++) w[j] = 0;
#pragma unroll
  for (int j = 0; j <= N; j++) {
    const u32 prev = j == 0 ? prefix : z[j - 1];
    const u32 cur = j < N ? (z[j] >> 8) : 0x00800000u;
    w[j] = (prev << 24) | cur;
  }
  w[NB * 16 - 1] = (u32)((4 * N + 1) * 8);
  sha_init(out);
#pragma unroll
  for (int b = 0; b < NB; b++) sha_compress(out, w + 16 * b);
}

__device__ __forceinline__ void sha_node(const u32* l, const u32* r, u32 out[8]) {
  u32 z[16];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    z[i] = l[i];
    z[8 + i] = r[i];
  }
  sha_short<16>(1u, z, out);
}

// The raw data words 16 b .. 16 b + 15 of a block of n words at p (zero past n).
template <bool VEC>
__device__ __forceinline__ void sha_load16(const u32* __restrict__ p, int n, int b, u32 d[16]) {
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int j0 = 16 * b + 4 * q;
    if (VEC && j0 + 4 <= n) {
      const uint4 v = *reinterpret_cast<const uint4*>(p + j0);
      d[4 * q] = v.x; d[4 * q + 1] = v.y; d[4 * q + 2] = v.z; d[4 * q + 3] = v.w;
    } else {
#pragma unroll
      for (int t = 0; t < 4; t++) d[4 * q + t] = j0 + t < n ? p[j0 + t] : 0u;
    }
  }
}

// H(0x00 || block) of n little-endian data words at p (n <= 256); VEC: p is 16-byte aligned.
// The next 64-byte piece's words are loaded before the current one is compressed, so the load
// latency hides behind a compression (one wave per SIMD runs these chains: the leaves of a
// 8192 x 2048 stage output are 65,536 chains). Message word j of the prefixed stream is
// (Z[j-1] << 24) | (Z[j] >> 8) with Z[j] = bswap(d[j]): bytes d[j-1].3, d[j].0, d[j].1, d[j].2,
// one v_perm_b32 of the raw words (selector 0x07000102) for every piece whose 16 words are all
// data; the last piece (the tail, the 0x80 terminator and the length) takes the general form.
template <bool VEC>
__device__ void sha_block_leaf(const u32* __restrict__ p, int n, u32 out[8]) {
  const int nb = (4 * n + 1 + 1 + 8 + 63) / 64;
  sha_init(out);
  u32 prevraw = 0;  // the raw word before the piece: the top byte of the first is the 0x00 prefix
  u32 d[16];
  sha_load16<VEC>(p, n, 0, d);
  for (int b = 0; b < nb; b++) {
    u32 nxt[16];
    if (b + 1 < nb) sha_load16<VEC>(p, n, b + 1, nxt);
    u32 w[16];
    if (16 * b + 16 <= n) {
#pragma unroll
      for (int t = 0; t < 16; t++) w[t] = __builtin_amdgcn_perm(t ? d[t - 1] : prevraw, d[t], 0x07000102u);
      prevraw = d[15];
    } else {
      u32 prev = __builtin_bswap32(prevraw);
#pragma unroll
      for (int t = 0; t < 16; t++) {
        const int j = 16 * b + t;
        u32 cur;
        if (j < n) cur = __builtin_bswap32(d[t]) >> 8;
        else if (j == n) cur = 0x00800000u;
        else cur = 0;
        w[t] = (j <= n ? (prev << 24) : 0u) | cur;
        prev = j < n ? __builtin_bswap32(d[t]) : 0u;
      }
      prevraw = __builtin_bswap32(prev);
      if (b == nb - 1) w[15] = (u32)((4 * n + 1) * 8);
    }
    sha_compress(out, w);
#pragma unroll
    for (int t = 0; t < 16; t++) d[t] = nxt[t];
  }
}

#define SHA_BLOCK_WORDS 256  // 1 KiB

// One thread per (row, block): the block leaves of every row.
template <bool VEC>
__global__ void sha_block_leaves_kernel(const u32* __restrict__ rows, long nrows, int row_words, int nblk,
                                        u32* __restrict__ leaves) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * nblk) return;
  const long r = i / nblk;
  const int b = (int)(i - r * nblk);
  const int off = b * SHA_BLOCK_WORDS, n = min(SHA_BLOCK_WORDS, row_words - off);
  u32 h[8];
  sha_block_leaf<VEC>(rows + r * row_words + off, n, h);
  uint4* o = reinterpret_cast<uint4*>(leaves + i * 8);
  o[0] = make_uint4(h[0], h[1], h[2], h[3]);
  o[1] = make_uint4(h[4], h[5], h[6], h[7]);
}

// One thread per row: the row root from its block leaves (bottom-up in place in the leaf
// buffer), then the tagged leaf H(0x00 || tag || u32le index || root).
__global__ void sha_row_leaf_kernel(u32* __restrict__ leaves, long nrows, int nblk, u32 tag, u32 base, u32 mod,
                                    u32* __restrict__ roots, u32* __restrict__ out) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= nrows) return;
  u32* lv = leaves + r * nblk * 8;
  int n = nblk;
  while (n > 1) {
    const int half = n >> 1;
    for (int i = 0; i < half; i++) {
      u32 h[8];
      sha_node(lv + 16 * i, lv + 16 * i + 8, h);
#pragma unroll
      for (int k = 0; k < 8; k++) lv[8 * i + k] = h[k];
    }
    if (n & 1) {
#pragma unroll
      for (int k = 0; k < 8; k++) lv[8 * half + k] = lv[8 * (n - 1) + k];
    }
    n = half + (n & 1);
  }
  u32 root[8];
#pragma unroll
  for (int k = 0; k < 8; k++) root[k] = lv[k];
  if (roots) {
#pragma unroll
    for (int k = 0; k < 8; k++) roots[r * 8 + k] = root[k];
  }
  if (out) {
    u32 idx = base + (u32)r;
    if (mod) idx %= mod;
    u32 z[10];
    z[0] = tag;
    z[1] = __builtin_bswap32(idx);  // u32 little-endian bytes as a big-endian word
#pragma unroll
    for (int k = 0; k < 8; k++) z[2 + k] = root[k];
    u32 h[8];
    sha_short<10>(0u, z, h);
#pragma unroll
    for (int k = 0; k < 8; k++) out[r * 8 + k] = h[k];
  }
}

// The same with one quad per row (16 rows per 64-thread workgroup) for rows of at most
// SHA_QUAD_MAXBLK blocks: the row's block leaves are copied to LDS and each level of the row tree
// is computed by the quad's lanes, node i by lane i % 4. A lane reads both children of its node
// inside sha_node before any lane of the wave writes a parent (the lanes issue the same
// instructions in order, and a wave's LDS operations complete in order); a level's parent i
// overwrites child slot i, which only parents <= i / 2 of earlier iterations read. The chain per
// row is then log2 of the block count in node pairs instead of the block count, and a wave holds
// 16 rows instead of 64 (4x the waves for the 8192 rows of a stage output).
#define SHA_QUAD_MAXBLK 64
#define SHA_QUAD_ROWS 16
__global__ void __launch_bounds__(64) sha_row_leaf_quad_kernel(const u32* __restrict__ leaves, long nrows, int nblk,
                                                               u32 tag, u32 base, u32 mod, u32* __restrict__ roots,
                                                               u32* __restrict__ out) {
  __shared__ u32 lds[SHA_QUAD_ROWS * SHA_QUAD_MAXBLK * 8];
  const int q = threadIdx.x & 3, rl = threadIdx.x >> 2;
  const long r = (long)blockIdx.x * SHA_QUAD_ROWS + rl;
  const bool live = r < nrows;  // no early return: the lanes of a quad stay together
  u32* lv = lds + rl * SHA_QUAD_MAXBLK * 8;
  if (live)
    for (int w = q; w < nblk * 8; w += 4) lv[w] = leaves[r * nblk * 8 + w];
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS writes are done
  __builtin_amdgcn_wave_barrier();
  int n = nblk;
  while (n > 1) {
    const int half = n >> 1;
    for (int i0 = 0; i0 < half; i0 += 4) {
      const int i = i0 + q;
      u32 h[8];
      if (live && i < half) {
        sha_node(lv + 16 * i, lv + 16 * i + 8, h);
#pragma unroll
        for (int k = 0; k < 8; k++) lv[8 * i + k] = h[k];
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
    }
    if (n & 1) {  // the odd last node moves up: words q and q + 4 by lane q
      u32 c0 = 0, c1 = 0;
      if (live) { c0 = lv[8 * (n - 1) + q]; c1 = lv[8 * (n - 1) + 4 + q]; }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
      if (live) { lv[8 * half + q] = c0; lv[8 * half + 4 + q] = c1; }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __builtin_amdgcn_wave_barrier();
    }
    n = half + (n & 1);
  }
  if (!live || q != 0) return;
  u32 root[8];
#pragma unroll
  for (int k = 0; k < 8; k++) root[k] = lv[k];
  if (roots) {
#pragma unroll
    for (int k = 0; k < 8; k++) roots[r * 8 + k] = root[k];
  }
  if (out) {
    u32 idx = base + (u32)r;
    if (mod) idx %= mod;
    u32 z[10];
    z[0] = tag;
    z[1] = __builtin_bswap32(idx);  // u32 little-endian bytes as a big-endian word
#pragma unroll
    for (int k = 0; k < 8; k++) z[2 + k] = root[k];
    u32 h[8];
    sha_short<10>(0u, z, h);
#pragma unroll
    for (int k = 0; k < 8; k++) out[r * 8 + k] = h[k];
  }
}

// One 256-thread workgroup per row for rows of SHA_QUAD_MAXBLK .. SHA_ROWTREE_MAXBLK blocks (e.g.
// the int32 logits rows of a 151,936-entry vocabulary: 594 blocks): the row's block leaves in LDS,
// each level's parents computed in parallel into a second LDS buffer (an odd last node moves up),
// then the tagged leaf. A thread per row would run its 2 (nblk - 1) compressions one after another.
#define SHA_ROWTREE_MAXBLK 1024
__global__ void __launch_bounds__(256) sha_row_tree_kernel(const u32* __restrict__ leaves, long nrows, int nblk,
                                                           u32 tag, u32 base, u32 mod, u32* __restrict__ roots,
                                                           u32* __restrict__ out) {
  extern __shared__ u32 rt_lds[];  // two buffers of nblk x 8 words
  const long r = blockIdx.x;
  u32* cur = rt_lds;
  u32* nxt = rt_lds + nblk * 8;
  const u32* src = leaves + r * nblk * 8;
  for (int i = threadIdx.x; i < nblk * 8; i += blockDim.x) cur[i] = src[i];
  __syncthreads();
  int n = nblk;
  while (n > 1) {
    const int half = n >> 1;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      u32 h[8];
      sha_node(cur + 16 * i, cur + 16 * i + 8, h);
#pragma unroll
      for (int k = 0; k < 8; k++) nxt[8 * i + k] = h[k];
    }
    if ((n & 1) && threadIdx.x < 8) nxt[8 * half + threadIdx.x] = cur[8 * (n - 1) + threadIdx.x];
    __syncthreads();
    u32* t = cur;
    cur = nxt;
    nxt = t;
    n = half + (n & 1);
  }
  if (threadIdx.x != 0) return;
  u32 root[8];
#pragma unroll
  for (int k = 0; k < 8; k++) root[k] = cur[k];
  if (roots) {
#pragma unroll
    for (int k = 0; k < 8; k++) roots[r * 8 + k] = root[k];
  }
  if (out) {
    u32 idx = base + (u32)r;
    if (mod) idx %= mod;
    u32 z[10];
    z[0] = tag;
    z[1] = __builtin_bswap32(idx);  // u32 little-endian bytes as a big-endian word
#pragma unroll
    for (int k = 0; k < 8; k++) z[2 + k] = root[k];
    u32 h[8];
    sha_short<10>(0u, z, h);
#pragma unroll
    for (int k = 0; k < 8; k++) out[r * 8 + k] = h[k];
  }
}

// One workgroup per tree of n leaves: the Merkle root, bottom-up through scratch.
__global__ void __launch_bounds__(256) sha_tree_kernel(const u32* __restrict__ leaves, int n0, u32* __restrict__ a,
                                                       u32* __restrict__ b, u32* __restrict__ roots) {
  const long t0 = (long)blockIdx.x * n0 * 8;
  const u32* src = leaves + t0;
  u32* dst = a + t0;
  u32* other = b + t0;
  int n = n0;
  if (n == 1) {
    if (threadIdx.x < 8) roots[blockIdx.x * 8 + threadIdx.x] = src[threadIdx.x];
    return;
  }
  while (n > 1) {
    const int half = n >> 1;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      u32 h[8];
      sha_node(src + 16 * i, src + 16 * i + 8, h);
#pragma unroll
      for (int k = 0; k < 8; k++) dst[8 * i + k] = h[k];
    }
    if ((n & 1) && threadIdx.x < 8) dst[8 * half + threadIdx.x] = src[8 * (n - 1) + threadIdx.x];
    __syncthreads();
    src = dst;
    u32* t = other;
    other = dst;
    dst = t;
    n = half + (n & 1);
  }
  if (threadIdx.x < 8) roots[blockIdx.x * 8 + threadIdx.x] = src[threadIdx.x];
}

// One workgroup per aligned group of up to SHA_GROUP leaves of a tree: the group's bottom-up root
// (8 pairing levels). Pairs never cross an aligned power-of-two boundary and a trailing partial
// group is the tail of every level, so the tree of the group roots, built the same way, has the
// same root as the whole tree.
#define SHA_GROUP 256
__global__ void __launch_bounds__(256) sha_group_kernel(const u32* __restrict__ leaves, int n0, int groups,
                                                        u32* __restrict__ out) {
  __shared__ u32 lv[SHA_GROUP * 8];
  const int t = blockIdx.x / groups, gi = blockIdx.x % groups;
  const int base = gi * SHA_GROUP, cnt = min(SHA_GROUP, n0 - base);
  const u32* src = leaves + ((long)t * n0 + base) * 8;
  for (int i = threadIdx.x; i < cnt * 8; i += blockDim.x) lv[i] = src[i];
  __syncthreads();
  int n = cnt;
  while (n > 1) {
    const int half = n >> 1;
    u32 h[8];
    if (threadIdx.x < half) sha_node(lv + 16 * threadIdx.x, lv + 16 * threadIdx.x + 8, h);
    __syncthreads();
    if (threadIdx.x < half) {
#pragma unroll
      for (int k = 0; k < 8; k++) lv[8 * threadIdx.x + k] = h[k];
    }
    if ((n & 1) && threadIdx.x < 8) lv[8 * half + threadIdx.x] = lv[8 * (n - 1) + threadIdx.x];
    __syncthreads();
    n = half + (n & 1);
  }
  if (threadIdx.x < 8) out[((long)t * groups + gi) * 8 + threadIdx.x] = lv[threadIdx.x];
}

extern "C" int uwc_sha_row_leaves(const uint32_t* rows, int64_t nrows, int row_words, uint32_t* scratch,
                                  int64_t scratch_words, uint32_t tag, uint32_t index_base, uint32_t index_mod,
                                  uint32_t* row_roots, uint32_t* leaves_out, hipStream_t stream) {
  const char* fn = "uwc_sha_row_leaves";
  if ((!rows && row_words > 0) || !scratch || nrows < 0 || row_words < 0) return uwc_fail("%s: bad arguments", fn);
  if (!row_roots && !leaves_out) return uwc_fail("%s: nothing to write", fn);
  if (rows && ((uintptr_t)rows & 3)) return uwc_fail("%s: rows must be 4-byte aligned", fn);
  if (nrows == 0) return UWC_OK;
  const int nblk = row_words == 0 ? 1 : (row_words + SHA_BLOCK_WORDS - 1) / SHA_BLOCK_WORDS;
  if (scratch_words < nrows * nblk * 8)
    return uwc_fail("%s: scratch has %lld words, needs %lld", fn, (long long)scratch_words, (long long)(nrows * nblk * 8));
  const long nt = nrows * nblk;
  const dim3 grid((unsigned)((nt + 127) / 128));
  if (row_words % 4 == 0 && ((uintptr_t)rows & 15) == 0)
    hipLaunchKernelGGL(sha_block_leaves_kernel<true>, grid, dim3(128), 0, stream, rows, (long)nrows, row_words, nblk, scratch);
  else
    hipLaunchKernelGGL(sha_block_leaves_kernel<false>, grid, dim3(128), 0, stream, rows, (long)nrows, row_words, nblk, scratch);
  int st = uwc_launch_status("sha_block_leaves");
  if (st) return st;
  if (nblk <= SHA_QUAD_MAXBLK)
    hipLaunchKernelGGL(sha_row_leaf_quad_kernel, dim3((unsigned)((nrows + SHA_QUAD_ROWS - 1) / SHA_QUAD_ROWS)), dim3(64),
                       0, stream, scratch, (long)nrows, nblk, tag, index_base, index_mod, row_roots, leaves_out);
  else if (nblk <= SHA_ROWTREE_MAXBLK && nrows <= 0x7FFFFFFFL)
    hipLaunchKernelGGL(sha_row_tree_kernel, dim3((unsigned)nrows), dim3(256), (size_t)nblk * 64, stream, scratch,
                       (long)nrows, nblk, tag, index_base, index_mod, row_roots, leaves_out);
  else
    hipLaunchKernelGGL(sha_row_leaf_kernel, dim3((unsigned)((nrows + 63) / 64)), dim3(64), 0, stream, scratch,
                       (long)nrows, nblk, tag, index_base, index_mod, row_roots, leaves_out);
  return uwc_launch_status("sha_row_leaf");
}

extern "C" int uwc_sha_merkle_roots(const uint32_t* leaves, int ntrees, int n, uint32_t* scratch, int64_t scratch_words,
                                    uint32_t* roots, hipStream_t stream) {
  const char* fn = "uwc_sha_merkle_roots";
  if (!leaves || !scratch || !roots || ntrees < 0 || n <= 0) return uwc_fail("%s: bad arguments", fn);
  if (ntrees == 0) return UWC_OK;
  const long need = 2L * ntrees * n * 8;
  if (scratch_words < need) return uwc_fail("%s: scratch has %lld words, needs %ld", fn, (long long)scratch_words, need);
  if (n > 2 * SHA_GROUP) {  // group roots first, in parallel, into the second half of scratch
    const int groups = (n + SHA_GROUP - 1) / SHA_GROUP;
    u32* gr = scratch + (long)ntrees * n * 8;
    hipLaunchKernelGGL(sha_group_kernel, dim3((unsigned)(ntrees * groups)), dim3(256), 0, stream, leaves, n, groups, gr);
    int st = uwc_launch_status("sha_group");
    if (st) return st;
    hipLaunchKernelGGL(sha_tree_kernel, dim3((unsigned)ntrees), dim3(256), 0, stream, gr, groups, scratch,
                       scratch + (long)ntrees * groups * 8, roots);
    return uwc_launch_status(fn);
  }
  hipLaunchKernelGGL(sha_tree_kernel, dim3((unsigned)ntrees), dim3(256), 0, stream, leaves, n, scratch,
                     scratch + (long)ntrees * n * 8, roots);
  return uwc_launch_status(fn);
}
