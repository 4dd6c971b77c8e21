/*
 * CPU oracle for the int8 x int8 -> int32 hot path of useful-work-coin.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product path links, loads or calls this
 * library: it is the checker that tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg compare the HIP kernels against.
 *
 * Every function restates the reference algorithm it names (paths relative to the
 * reference repository root). Build: see oracle/build.sh (gcc -O2 -fopenmp
 * -ffp-contract=off): IEEE-754 binary32 arithmetic on x86-64 SSE is correctly rounded
 * and, with contraction off, no multiply-add is fused, which is exactly the
 * "emulated fp32" contract of runtime/detrt/core.py:1-17.
 *
 * Pinning (what checks each function; the tests live in tests/test_oracle.py):
 *   or_igemm_i32        L1 known answer sha256[:20] = bf9394d180bda5b0412c
 *                       (results/xc_cpu.json:4, miner/ampere/bench/crosscheck.py:62-76)
 *                       and the Go-referee linear fixtures (int accumulators).
 *   or_b3_*             the BLAKE3 team's published test vectors (unkeyed 0..102400 bytes,
 *                       keyed 0, 1, 1024 and 2048 bytes: one block, a chunk chain, parent
 *                       nodes, 31- and 100-chunk trees), plus agreement with an independent
 *                       pure-Python restatement (oracle/blake3_py.py) over every tree shape
 *                       up to 129 chunks, keyed and plain, and ragged lengths.
 *   or_noise_*          structural invariants (range [-32,31], first != second < r) and the
 *                       rules' distributions (E uniform on [-32,31]; P's first index uniform, its
 *                       XOR distance uniform on [1,r-1]), byte layout against a pure-Python
 *                       random_hash. PARITY UNPINNED: the values rest on the pinned keyed BLAKE3
 *                       and the restated message layout (reference.py:67-93); the reference stores
 *                       no vectors of them, nor of the seeds or tile digests built the same way.
 *   or_transcript_*     brute-force per-tile recomputation on tiny shapes (explicit
 *                       cumulative sums over each tile's 128 elements).
 *   or_quant_act_f32    Go-referee fixtures N1->QA1, O->QA2, N2->QA3, SM->QA4 bit-exact.
 *   or_dequant_f32      Go-referee fixtures QA1 x W -> QKV etc. bit-exact
 *                       (chain/patches/0003-*.patch:618-634 linearElem).
 *   or_scale_bf16       torch's fp32 -> bf16 conversion (round to nearest even) of the same fp32
 *                       products, random values and exact ties of both kept-bit parities.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------ BLAKE3
 * Restated from the BLAKE3 specification (blake3==1.0.11 is the reference's dependency,
 * dist/requirements.txt:6; GPU use in miner/ampere/uwc_ampere/kernels.cu:41-244). */
#define B3_CHUNK_START 1u
#define B3_CHUNK_END 2u
#define B3_PARENT 4u
#define B3_ROOT 8u
#define B3_KEYED 16u

static const uint32_t B3IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                 0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
static const int B3PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static inline uint32_t ror32(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static inline void b3_g(uint32_t* v, int a, int b, int c, int d, uint32_t x, uint32_t y) {
  v[a] = v[a] + v[b] + x; v[d] = ror32(v[d] ^ v[a], 16);
  v[c] = v[c] + v[d];     v[b] = ror32(v[b] ^ v[c], 12);
  v[a] = v[a] + v[b] + y; v[d] = ror32(v[d] ^ v[a], 8);
  v[c] = v[c] + v[d];     v[b] = ror32(v[b] ^ v[c], 7);
}

/* Full 16-word compression output. */
EXPORT void or_b3_compress(const uint32_t cv[8], const uint32_t msg[16], uint64_t counter, uint32_t blen,
                           uint32_t flags, uint32_t out[16]) {
  uint32_t v[16], m[16], t[16];
  for (int i = 0; i < 8; i++) v[i] = cv[i];
  for (int i = 0; i < 4; i++) v[8 + i] = B3IV[i];
  v[12] = (uint32_t)counter; v[13] = (uint32_t)(counter >> 32); v[14] = blen; v[15] = flags;
  memcpy(m, msg, sizeof m);
  for (int r = 0; r < 7; r++) {
    b3_g(v, 0, 4, 8, 12, m[0], m[1]);
    b3_g(v, 1, 5, 9, 13, m[2], m[3]);
    b3_g(v, 2, 6, 10, 14, m[4], m[5]);
    b3_g(v, 3, 7, 11, 15, m[6], m[7]);
    b3_g(v, 0, 5, 10, 15, m[8], m[9]);
    b3_g(v, 1, 6, 11, 12, m[10], m[11]);
    b3_g(v, 2, 7, 8, 13, m[12], m[13]);
    b3_g(v, 3, 4, 9, 14, m[14], m[15]);
    for (int i = 0; i < 16; i++) t[i] = m[B3PERM[i]];
    memcpy(m, t, sizeof m);
  }
  for (int i = 0; i < 8; i++) { out[i] = v[i] ^ v[i + 8]; out[i + 8] = v[i + 8] ^ cv[i]; }
}

static inline uint32_t ld32(const uint8_t* p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Chaining value of one chunk (len <= 1024 bytes); if `root` the last block carries ROOT
 * and the first 8 output words are the digest. */
static void b3_chunk(const uint8_t* p, size_t len, const uint32_t key[8], uint32_t kflag, uint64_t chunk_idx,
                     int root, uint32_t cv_out[8]) {
  uint32_t cv[8], m[16], out[16];
  memcpy(cv, key, 32);
  size_t nblk = len == 0 ? 1 : (len + 63) / 64;
  for (size_t b = 0; b < nblk; b++) {
    uint8_t blk[64] = {0};
    size_t off = b * 64, bl = len - off < 64 ? len - off : 64;
    if (len) memcpy(blk, p + off, bl);
    for (int i = 0; i < 16; i++) m[i] = ld32(blk + 4 * i);
    uint32_t fl = kflag | (b == 0 ? B3_CHUNK_START : 0u) | (b == nblk - 1 ? B3_CHUNK_END : 0u);
    if (root && b == nblk - 1) fl |= B3_ROOT;
    or_b3_compress(cv, m, chunk_idx, (uint32_t)bl, fl, out);
    memcpy(cv, out, 32);
  }
  memcpy(cv_out, cv, 32);
}

/* Subtree over chunks [c0, c0 + n) of the input: left-complete tree (the left child holds the
 * largest power of two of chunks that leaves at least one byte on the right). */
static void b3_subtree(const uint8_t* data, size_t len, uint64_t c0, uint64_t n, const uint32_t key[8],
                       uint32_t kflag, int root, uint32_t cv_out[8]) {
  if (n == 1) {
    size_t off = (size_t)c0 * 1024, cl = len - off < 1024 ? len - off : 1024;
    b3_chunk(data + off, cl, key, kflag, c0, root, cv_out);
    return;
  }
  uint64_t left = 1;
  while (left * 2 < n) left *= 2;
  uint32_t m[16], out[16];
  b3_subtree(data, len, c0, left, key, kflag, 0, m);
  b3_subtree(data, len, c0 + left, n - left, key, kflag, 0, m + 8);
  or_b3_compress(key, m, 0, 64, B3_PARENT | kflag | (root ? B3_ROOT : 0u), out);
  memcpy(cv_out, out, 32);
}

/* BLAKE3 of `len` bytes; key = NULL for the plain hash, else the 8-word key (keyed mode).
 * digest = first 32 output bytes, as 8 little-endian words. */
EXPORT void or_b3_hash(const uint8_t* data, uint64_t len, const uint32_t* key, uint32_t digest[8]) {
  uint32_t kflag = key ? B3_KEYED : 0u;
  const uint32_t* k = key ? key : B3IV;
  uint64_t n = len == 0 ? 1 : (len + 1023) / 1024;
  b3_subtree(data, (size_t)len, 0, n, k, kflag, 1, digest);
}

/* get_random_hash(index, label, key, prepend): a keyed one-block hash of the 64-byte message
 * with word `prepend` = 1 + index and words 8..15 = label.
 * miner/ampere/uwc_ampere/reference.py:67-71; kernels.cu:247-257. */
static void random_hash(uint32_t index, const uint32_t label[8], const uint32_t key[8], int prepend, uint32_t h[8]) {
  uint32_t msg[16], out[16];
  for (int i = 0; i < 8; i++) { msg[i] = 0; msg[8 + i] = label[i]; }
  msg[prepend] = 1u + index;
  or_b3_compress(key, msg, 0, 64, B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, out);
  memcpy(h, out, 32);
}

/* rows x r int8 in [-32, 31]: byte j of hash block b -> (byte & 63) - 32.
 * reference.py:74-79 (uniform_matrix); kernels.cu:259-282. */
EXPORT void or_noise_uniform(int8_t* out, uint32_t nblocks, const uint32_t label[8], const uint32_t key[8]) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < (int64_t)nblocks; b++) {
    uint32_t h[8];
    random_hash((uint32_t)b, label, key, 0, h);
    for (int i = 0; i < 8; i++)
      for (int j = 0; j < 4; j++) out[b * 32 + 4 * i + j] = (int8_t)((int)((h[i] >> (8 * j)) & 63u) - 32);
  }
}

/* k noise pairs packed (first | second << 16); first = u & (r-1),
 * second = first ^ (1 + floor((r-1) u / 2^32)). reference.py:82-93; kernels.cu:284-301. */
EXPORT void or_noise_perm(uint32_t* out, uint32_t k, uint32_t r, const uint32_t label[8], const uint32_t key[8]) {
  uint32_t nh = (k + 7) / 8;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)nh; i++) {
    uint32_t h[8];
    random_hash((uint32_t)i, label, key, 1, h);
    for (int j = 0; j < 8; j++) {
      uint64_t l = (uint64_t)i * 8 + j;
      if (l >= k) break;
      uint32_t u = h[j], first = u & (r - 1);
      uint32_t second = first ^ (1u + (uint32_t)(((uint64_t)(r - 1) * u) >> 32));
      out[l] = first | (second << 16);
    }
  }
}

/* dst = int8(src + E[row][P.first] - E[row][P.second]) (two's-complement wrap).
 * reference.py:96-104 (noise_a / noise_bt); kernels.cu:303-345. */
EXPORT void or_noise_apply(const int8_t* src, int64_t rows, int64_t k, int64_t r, const int8_t* E, const uint32_t* P,
                           int8_t* dst) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows; i++) {
    const int8_t* e = E + i * r;
    for (int64_t l = 0; l < k; l++) {
      int v = src[i * k + l] + e[P[l] & 0xFFFF] - e[P[l] >> 16];
      dst[i * k + l] = (int8_t)(uint8_t)(v & 0xFF);
    }
  }
}

/* proj[row][j] = sum_l src[row][l] ([P.first(l) == j] - [P.second(l) == j]): src * S^T.
 * kernels.cu:339-343 (the projection half of noise_rows); test_kernels.py:73-76. */
EXPORT void or_project(const int8_t* src, int64_t rows, int64_t k, int64_t r, const uint32_t* P, int32_t* proj) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < rows; i++) {
    int32_t* pr = proj + i * r;
    for (int64_t j = 0; j < r; j++) pr[j] = 0;
    for (int64_t l = 0; l < k; l++) {
      int x = src[i * k + l];
      pr[P[l] & 0xFFFF] += x;
      pr[P[l] >> 16] -= x;
    }
  }
}

/* Balanced base-128 limbs: corr[li][row][off + j], row stride 2r, d = ((v + 64) & 127) - 64,
 * v = (v - d) >> 7. kernels.cu:348-361 (noise_rows tail), :374-395 (proj_corr). */
EXPORT void or_limbs(const int32_t* proj, int64_t rows, int64_t r, int lmax, int8_t* corr, int64_t corr_off) {
  const int64_t limb_stride = rows * 2 * r;
  for (int64_t i = 0; i < rows; i++)
    for (int64_t j = 0; j < r; j++) {
      int32_t v = proj[i * r + j];
      for (int li = 0; li < lmax; li++) {
        int32_t d = ((v + 64) & 127) - 64;
        corr[li * limb_stride + i * 2 * r + corr_off + j] = (int8_t)d;
        v = (v - d) >> 7;
      }
    }
}

/* C = A * B^T, A m x k, B n x k int8 (k contiguous), int32 wrapping accumulation.
 * The exact integer product of miner/ampere/bench/crosscheck.py:75 and
 * runtime/detrt/qwen3.py:109-110 (values fit int32 for k <= 133k). */
EXPORT void or_igemm_i32(const int8_t* A, const int8_t* B, int64_t m, int64_t n, int64_t k, int32_t* C) {
  const int64_t TB = 64;
  int64_t nbn = (n + TB - 1) / TB;
#pragma omp parallel
  {
    int32_t* bt = (int32_t*)malloc(sizeof(int32_t) * TB * 256);  /* k-slice x TB, int32 */
#pragma omp for schedule(dynamic)
    for (int64_t jb = 0; jb < nbn; jb++) {
      int64_t j0 = jb * TB, jn = n - j0 < TB ? n - j0 : TB;
      for (int64_t i = 0; i < m; i++)
        for (int64_t j = 0; j < jn; j++) C[i * n + j0 + j] = 0;
      for (int64_t l0 = 0; l0 < k; l0 += 256) {
        int64_t ln = k - l0 < 256 ? k - l0 : 256;
        for (int64_t l = 0; l < ln; l++)
          for (int64_t j = 0; j < TB; j++) bt[l * TB + j] = j < jn ? B[(j0 + j) * k + l0 + l] : 0;
        for (int64_t i = 0; i < m; i++) {
          uint32_t acc[64];
          for (int64_t j = 0; j < TB; j++) acc[j] = (uint32_t)C[i * n + j0 + (j < jn ? j : 0)];
          const int8_t* a = A + i * k + l0;
          for (int64_t l = 0; l < ln; l++) {
            uint32_t av = (uint32_t)(int32_t)a[l];
            const int32_t* b = bt + l * TB;
            for (int64_t j = 0; j < TB; j++) acc[j] += av * (uint32_t)b[j];
          }
          for (int64_t j = 0; j < jn; j++) C[i * n + j0 + j] = (int32_t)acc[j];
        }
      }
    }
    free(bt);
  }
}

/* ------------------------------------------------------------------ mining transcript
 * Hash tile pattern of the Ampere miner (miner/ampere/uwc_ampere/pearl_glue.py:14-15,
 * kernels.cu:8-11): inside each 64 x 64 block, tile (g, t) holds rows g + 8i (i < 8) and
 * cols 2t + e + 8j (e < 2, j < 8): 128 int32 values. After every r-chunk c of k the tile's
 * cumulative accumulators are XOR-folded, x = XOR_u32(acc), and msg[c % 16] =
 * rotl13(msg[c % 16]) ^ x (reference.py:111-121, kernels.cu:558-570).
 * msgs layout: [m/64][8 (g)][n/64][4 (t)][16] u32, as reference.py:138-165. */
static inline uint32_t rotl32(uint32_t x, int s) { return (x << s) | (x >> (32 - s)); }

EXPORT void or_transcript(const int8_t* Ap, const int8_t* Bp, int64_t m, int64_t n, int64_t k, int64_t r,
                          uint32_t* msgs) {
  const int64_t MB = m / 64, NB = n / 64;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t rb = 0; rb < MB; rb++)
    for (int64_t cb = 0; cb < NB; cb++) {
      uint32_t acc[64][64];
      uint32_t msg[8][4][16];
      int32_t bt[64][64];
      memset(acc, 0, sizeof acc);
      memset(msg, 0, sizeof msg);
      for (int64_t c = 0; c < k / r; c++) {
        for (int64_t l0 = c * r; l0 < (c + 1) * r; l0 += 64) {
          for (int64_t l = 0; l < 64; l++)
            for (int64_t j = 0; j < 64; j++) bt[l][j] = Bp[(cb * 64 + j) * k + l0 + l];
          for (int64_t i = 0; i < 64; i++) {
            const int8_t* a = Ap + (rb * 64 + i) * k + l0;
            for (int64_t l = 0; l < 64; l++) {
              uint32_t av = (uint32_t)(int32_t)a[l];
              for (int64_t j = 0; j < 64; j++) acc[i][j] += av * (uint32_t)bt[l][j];
            }
          }
        }
        const int slot = (int)(c % 16);
        for (int g = 0; g < 8; g++)
          for (int t = 0; t < 4; t++) {
            uint32_t x = 0;
            for (int i = 0; i < 8; i++)
              for (int j = 0; j < 8; j++) x ^= acc[g + 8 * i][2 * t + 8 * j] ^ acc[g + 8 * i][2 * t + 1 + 8 * j];
            msg[g][t][slot] = rotl32(msg[g][t][slot], 13) ^ x;
          }
      }
      for (int g = 0; g < 8; g++)
        for (int t = 0; t < 4; t++)
          memcpy(msgs + ((((rb * 8 + g) * NB + cb) * 4 + t) * 16), msg[g][t], 64);
    }
}

/* digest = keyed BLAKE3(key, 16 LE words of msg) for every tile (reference.py:124-125,
 * kernels.cu:574-578); win if digest <= target as little-endian U256 (kernels.cu:579-585). */
EXPORT void or_tile_hashes(const uint32_t* msgs, int64_t ntiles, const uint32_t key[8], uint32_t* digests) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < ntiles; i++) {
    uint32_t out[16];
    or_b3_compress(key, msgs + i * 16, 0, 64, B3_CHUNK_START | B3_CHUNK_END | B3_ROOT | B3_KEYED, out);
    memcpy(digests + i * 8, out, 32);
  }
}

EXPORT int or_hash_le(const uint32_t h[8], const uint32_t target[8]) {
  for (int i = 7; i >= 0; i--)
    if (h[i] != target[i]) return h[i] < target[i];
  return 1;
}

/* ------------------------------------------------------------------ detrt requant / dequant
 * quant_act = fwht (stages h = 1, 2, 4, ..., pairs (i, i + h) -> (a + b, a - b)) then
 * quant_sym(qmax = 64): s = max(max|y|, f32(1e-8)) / 64, q = clamp(rint(y / s), -64, 64),
 * returned scale s * (1 / sqrt(bs)) when bs > 1.
 * runtime/detrt/core.py:162-195; Go mirror chain/patches/0003-*.patch:119-160. */
static void fwht_row(float* v, int64_t k, int bs) {
  if (bs <= 1) return;
  for (int64_t h = 1; h < bs; h <<= 1)
    for (int64_t blk = 0; blk < k; blk += 2 * h)
      for (int64_t j = 0; j < h; j++) {
        float a = v[blk + j], b = v[blk + h + j];
        v[blk + j] = a + b;
        v[blk + h + j] = a - b;
      }
}

EXPORT void or_quant_act_f32(const float* x, int64_t rows, int64_t k, int bs, int qmax, int8_t* q, float* scale) {
  const float tiny = (float)1e-8;
#pragma omp parallel
  {
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
    for (int64_t i = 0; i < rows; i++) {
      memcpy(v, x + i * k, sizeof(float) * (size_t)k);
      fwht_row(v, k, bs);
      float amax = 0.0f;
      for (int64_t l = 0; l < k; l++) {
        float a = fabsf(v[l]);
        if (a > amax) amax = a;
      }
      float s = (amax > tiny ? amax : tiny) / (float)qmax;
      for (int64_t l = 0; l < k; l++) {
        float t = rintf(v[l] / s);
        if (t < -(float)qmax) t = -(float)qmax;
        if (t > (float)qmax) t = (float)qmax;
        q[i * k + l] = (int8_t)(int)t;
      }
      float sc = s;
      if (bs > 1) {
        float rs = 1.0f / sqrtf((float)bs);
        sc = s * rs;
      }
      scale[i] = sc;
    }
    free(v);
  }
}

/* y[i][j] = (f32(acc[i][j]) * sx[i]) * sw[j], each product rounded once.
 * runtime/detrt/qwen3.py:125; chain/patches/0003-*.patch:618-634 (linearElem). */
EXPORT void or_dequant_f32(const int32_t* acc, const float* sx, const float* sw, int64_t m, int64_t n, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      float t = (float)acc[i * n + j] * sx[i];
      y[i * n + j] = t * sw[j];
    }
}

/* bf16(f32(acc) * a_scale[i] * b_scale[j]) with round-to-nearest-even on the bit pattern
 * (kernels.cu:440-445, :687-704: the OUT_BF16 epilogue). */
EXPORT void or_scale_bf16(const int32_t* acc, const float* as, const float* bsc, int64_t m, int64_t n, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; i++)
    for (int64_t j = 0; j < n; j++) {
      float t = (float)acc[i * n + j] * as[i];
      float f = t * bsc[j];
      uint32_t u;
      memcpy(&u, &f, 4);
      out[i * n + j] = (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
    }
}
