/*
 * uwc.h - C-ABI of libuwc_hip.so, the MI355X (gfx950) int8 x int8 -> int32 GEMM hot path of
 * useful-work-coin: the cuPOW NoisyGEMM miner and the detrt deterministic integer linear, with
 * the decoder-layer ops and stage commitments around detrt's GEMMs.
 *
 * Conventions (all entry points):
 *   - every pointer is device memory unless stated otherwise, allocated by the caller;
 *   - launches are asynchronous on `stream` (hipStream_t; NULL = the null stream), no entry
 *     point synchronizes or allocates;
 *   - return 0 on success, UWC_EINVAL (-1) for rejected arguments (nothing launched), or a
 *     positive hipError_t if a launch failed; uwc_last_error() then describes the failure
 *     (thread-local, valid until the next failing call on the thread);
 *   - 32-byte values (keys, seeds, roots, labels, salts, targets) are 8 little-endian u32 words.
 *
 * Reference paths below are relative to the reference repository root.
 */
#ifndef UWC_H
#define UWC_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UWC_EINVAL (-1)

/* gemm flags and output modes: miner/ampere/uwc_ampere/ops.py:26-29 (OUT_F32 is new: the
 * fused detrt dequant epilogue fmul(fmul(f32(acc), a_scale[i]), b_scale[j])). */
#define UWC_FLAG_HASH 1
#define UWC_FLAG_DENOISE 2
#define UWC_FLAG_TILE128 0x100  /* force the 128 x 128 tiling (identical results) */
/* force configuration c (0: 128 x 128 tiles, 4-step ring; 1: 128 x 256, 3 steps; 2: 128 x 128,
 * 2 steps; 3: 128 x 256, 2 steps; c + 4: the same with each step's DMA spread over the next
 * step's passes) of the DMA-pipelined plain kernel: UWC_FLAG_PLAIN_CFG(c).
 * Plain GEMMs only (no HASH / DENOISE / TILE128); m, n multiples of the tile, k % 128 == 0, out
 * and (for BF16 / F32) b_scale 16-byte aligned, n % 4 == 0; identical results. */
#define UWC_FLAG_PLAIN 0x200
#define UWC_FLAG_PLAIN_CFG(c) (UWC_FLAG_PLAIN | ((c) << 12))
#define UWC_OUT_NONE 0
#define UWC_OUT_I32 1
#define UWC_OUT_BF16 2
#define UWC_OUT_F32 3
#define UWC_WIN_WORDS 10     /* win record: row_off, col_off, digest[8] */
#define UWC_DUMP_WORDS 24    /* tile dump: message[16], digest[8] */

/* Library version (1) and the message of the last failing call on this thread. */
int uwc_version(void);
const char* uwc_last_error(void);
/* The first 16 hex digits of the SHA-256 of the include/uwc.h the library was built from: a
 * binding compares it with the header it was written against, so a library left over from an
 * earlier header (changed argument lists) is refused instead of called with the wrong layout.
 * No counterpart in the reference (its kernels are compiled at import, kernels.cu via CuPy). */
const char* uwc_header_sha(void);

/*
 * C = A * B^T (A m x k, B n x k, int8, k contiguous, 16-byte aligned; k % 64 == 0), optionally:
 *   UWC_FLAG_HASH     fold every tile's cumulative int32 accumulators every r along k into the
 *                     16-word jackpot message (hash tile = rows g+8i, cols 2t+e+8j of each 64x64
 *                     block), digest it with keyed BLAKE3 (key = a_seed) and append
 *                     [row_off, col_off, digest] to wins (wins[0] = count, records capped at
 *                     max_wins) when digest <= target (little-endian U256). Needs m, n % 128 == 0,
 *                     r a power of two, r % 64 == 0, k % r == 0. tile_dump (optional, else NULL)
 *                     receives every tile's message and digest, layout
 *                     [m/64][8][n/64][4][UWC_DUMP_WORDS].
 *   UWC_FLAG_DENOISE  subtract sum_li 128^li [X_li | EAL] [EBRt | Y_li]^T exactly; corrA
 *                     (lmax, m, 2r), corrB (lmax, n, 2r) int8; limbs used from maxabs[0..1].
 * out_mode: UWC_OUT_NONE, UWC_OUT_I32 (int32 m x n), UWC_OUT_BF16 (bf16 of
 * f32(acc) * a_scale[i] * b_scale[j], RNE), UWC_OUT_F32 (fp32 of the same, each product
 * rounded once). Without flags any m, n >= 1 are accepted (edges masked).
 * Replaces ops.gemm -> noisy_gemm: miner/ampere/uwc_ampere/ops.py:185-198,
 * miner/ampere/uwc_ampere/kernels.cu:482-715.
 */
int uwc_noisy_gemm(const int8_t* A, const int8_t* B, int m, int n, int k, int r, const int8_t* corrA,
                   const int8_t* corrB, const int32_t* maxabs, int lmax, const uint32_t* key, const uint32_t* target,
                   uint32_t* wins, int max_wins, const float* a_scale, const float* b_scale, void* out, int out_mode,
                   int flags, uint32_t* tile_dump, hipStream_t stream);

/*
 * `count` GEMMs sharing B (and target, scales, out_mode, flags), item i equal to
 * uwc_noisy_gemm(A[i], B, ..., corrA[i], corrB[i], maxabs[i], ..., key[i], target, wins[i], ...,
 * out[i], ..., tile_dump[i]). A, corrA, corrB, maxabs, key, wins, out and tile_dump are HOST
 * arrays of `count` device pointers (corrA/corrB/maxabs may be NULL without UWC_FLAG_DENOISE, key
 * without UWC_FLAG_HASH, wins and tile_dump entirely). With HASH | DENOISE, UWC_OUT_I32, m, n % 256 == 0 and
 * count >= 2 the items run up to 32 per launch on the same tiles, the output stores of one item draining
 * while the next computes; otherwise one launch per item. The reference mines one nonce per
 * ops.gemm call (ops.py:185-198 from MinedWeight._forward, ops.py:339-347); this form serves a
 * sweep of nonces whose operands are all prepared up front.
 */
int uwc_noisy_gemm_many(int count, const int8_t* const* A, const int8_t* B, int m, int n, int k, int r,
                        const int8_t* const* corrA, const int8_t* const* corrB, const int32_t* const* maxabs, int lmax,
                        const uint32_t* const* key, const uint32_t* target, uint32_t* const* wins, int max_wins,
                        const float* a_scale, const float* b_scale, void* const* out, int out_mode, int flags,
                        uint32_t* const* tile_dump, hipStream_t stream);

/* Exact int32 C = A * B^T for any m, n (k % 64 == 0).
 * Replaces DetLinear.int_gemm's GPU path (torch._int_mm / MinedWeight.forward OUT_I32):
 * runtime/detrt/qwen3.py:106-119. */
int uwc_igemm_i32(const int8_t* A, const int8_t* B, int m, int n, int k, int32_t* C, hipStream_t stream);

/* Y = fmul(fmul(f32(A * B^T), sx[i]), sw[j]) fused in the GEMM epilogue (fp32 m x n).
 * Replaces DetLinear.__call__'s int_gemm + dequant: runtime/detrt/qwen3.py:121-126. */
int uwc_igemm_dequant_f32(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx, const float* sw,
                          float* Y, hipStream_t stream);

/* Y = fadd(x, fmul(fmul(f32(A * B^T), sx[i]), sw[j])) (fp32 m x n, rows of stride n): the exact
 * GEMM with the dequant and the residual add in its epilogue where the 256 x 256 tiles take the
 * shape, else the dequantized product followed by the residual pass; the same bits either way.
 * Y must not overlap x.
 * Replaces DetLinear.int_gemm + detgpu kernels.dequant_residual of the o and down projections:
 * runtime/detrt/qwen3.py:106-126, runtime/detgpu/kernels.py:805-813, runtime/detrt/stage.py:217, 224. */
int uwc_igemm_dequant_residual_f32(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx,
                                   const float* sw, const float* x, float* Y, hipStream_t stream);

/* Scratch words uwc_b3_root_and_seed needs for an input of nbytes (host-side, no GPU work). */
int uwc_b3_scratch_words(uint64_t nbytes);

/* Keyed BLAKE3 tree root of data (nbytes a positive multiple of 1024) into root_out, and if
 * seed_out is given: seed = BLAKE3(prefix || keyed_BLAKE3(salt, root || dim_le32 || 0^28)).
 * root_out and seed_out may each be NULL.
 * Replaces ops.b3_root_and_seed: miner/ampere/uwc_ampere/ops.py:99-118, kernels.cu:138-244. */
int uwc_b3_root_and_seed(const uint8_t* data, uint64_t nbytes, const uint32_t* key, const uint32_t* prefix,
                         const uint32_t* salt, uint32_t dim, uint32_t* root_out, uint32_t* seed_out,
                         uint32_t* scratch, uint64_t scratch_words, hipStream_t stream);

/* uwc_b3_root_and_seed over `count` (1..32) inputs of nbytes each, in one set of launches:
 * data, root_out and seed_out are HOST arrays of `count` device pointers (root_out / seed_out
 * may be NULL arrays; their entries may not be NULL). Item i uses scratch words
 * [i * s, (i + 1) * s) with s = uwc_b3_scratch_words(nbytes). Results equal `count` separate
 * calls. The reference commits one operand per call (ops.py:99-118 from MinedWeight._forward,
 * ops.py:322-324); this form serves a sweep of nonces whose activations are all known up front,
 * where one commitment alone leaves the latency-bound chunk chains at one wave per SIMD. */
int uwc_b3_root_and_seed_many(const uint8_t* const* data, int count, uint64_t nbytes, const uint32_t* key,
                              const uint32_t* prefix, const uint32_t* salt, uint32_t dim, uint32_t* const* root_out,
                              uint32_t* const* seed_out, uint32_t* scratch, uint64_t scratch_words,
                              hipStream_t stream);

/* uwc_b3_root_and_seed without a scratch argument: the same root and seed, for inputs of at most
 * 1 GiB (2^30 bytes; larger inputs are rejected with UWC_EINVAL), with the workspace in a static
 * device array of 131,200 words (513 KiB) that every GPU the library runs on holds until the
 * process ends. No counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). It allocates nothing; its first call
 * on a device looks up that device's workspace address (make it before a capture). Calls that
 * overlap on one GPU share the workspace and race; calls ordered on one stream do not. */
int uwc_b3_root_and_seed_static(const uint8_t* data, uint64_t nbytes, const uint32_t* key, const uint32_t* prefix,
                                const uint32_t* salt, uint32_t dim, uint32_t* root_out, uint32_t* seed_out,
                                hipStream_t stream);

/* out (nblocks x 32 int8) = (bytes of keyed_BLAKE3(key, msg(index, label)) & 63) - 32; also
 * zeroes zero_me[0..zero_n) (may be NULL with zero_n = 0).
 * Replaces ops.noise_uniform: ops.py:122-125, kernels.cu:259-282. */
int uwc_noise_uniform(int8_t* out, uint32_t nblocks, const uint32_t* label, const uint32_t* key, int32_t* zero_me,
                      int zero_n, hipStream_t stream);

/* k noise pairs packed first | second << 16 (r a power of two).
 * Replaces ops.noise_perm: ops.py:128-131, kernels.cu:284-301. */
int uwc_noise_perm(uint32_t* out, uint32_t k, uint32_t r, const uint32_t* label, const uint32_t* key,
                   hipStream_t stream);

/* One launch for a nonce's noise: E (rows x r) as uwc_noise_uniform, P (k pairs) as
 * uwc_noise_perm with the same label and key, St (r x k, optional) as uwc_proj_matrix(P), SpT
 * (optional, r <= 64, 16-byte aligned) = St transposed as k rows of 64 bytes, zero past r,
 * and zeroes zero0[0..n0) and zero1[0..n1) (n <= 256 each, pointers may be NULL with n = 0).
 * Fuses ops.noise_uniform + ops.noise_perm + ops.proj_matrix of MinedWeight._forward
 * (ops.py:328-336). */
int uwc_nonce_noise(int8_t* E, int rows, int r, uint32_t* P, int k, int8_t* St, int8_t* SpT, const uint32_t* label,
                    const uint32_t* key, int32_t* zero0, int n0, int32_t* zero1, int n1, hipStream_t stream);

/* uwc_nonce_noise for `count` (1..32) nonces in one launch: E, P, St, SpT, key, zero0, zero1 are
 * HOST arrays of `count` device pointers (St, SpT, zero0, zero1 may be NULL arrays; entries of a
 * given array may not be NULL). Same label for every item. Results equal `count` separate calls.
 * Batches the per-nonce noise of ops.py:328-336 over a sweep of nonces. */
int uwc_nonce_noise_many(int count, int8_t* const* E, int rows, int r, uint32_t* const* P, int k, int8_t* const* St,
                         int8_t* const* SpT, const uint32_t* label, const uint32_t* const* key, int32_t* const* zero0,
                         int n0, int32_t* const* zero1, int n1, hipStream_t stream);

/* For rows (multiple of 8) x k (multiple of 4) int8 src, each part optional (NULL = skip):
 *   dst = int8(src + E[row][Pn.first] - E[row][Pn.second]);
 *   projection src * S^T (S from Pp) in lmax base-128 limbs at corr[li][row][corr_off + j];
 *   E rows copied to corr[li][row][ecopy_off + j]; max |projection| atomically into *maxabs.
 * corr is (lmax, rows, 2r) int8; corr_off / ecopy_off are 0, r or -1 (skip).
 * Replaces ops.noise_rows: ops.py:134-142, kernels.cu:303-372. */
int uwc_noise_rows(const int8_t* src, int rows, int k, int r, const int8_t* E, const uint32_t* Pn, int8_t* dst,
                   const uint32_t* Pp, int8_t* corr, int corr_off, int ecopy_off, int32_t* maxabs, int lmax,
                   hipStream_t stream);

/* St (r x k int8, k % 16 == 0) = the selection matrix of a noise permutation:
 * St[j][l] = [P.first(l) == j] - [P.second(l) == j].
 * Replaces ops.proj_matrix: ops.py:152-158, kernels.cu:397-404. */
int uwc_proj_matrix(const uint32_t* P, int k, int r, int8_t* St, hipStream_t stream);

/* Projection src * St^T (rows x r, exact int32 on the matrix cores) written as lmax balanced
 * base-128 limbs to corr[li][row][corr_off + j] (corr_off 0 or r), max |projection| into *maxabs
 * (atomic max; may be NULL). rows % 16 == 0, k % 64 == 0, r % 16 == 0, r <= 128.
 * Replaces ops.project (torch._int_mm + proj_corr): ops.py:161-168, kernels.cu:374-395. */
int uwc_project(const int8_t* src, int rows, int k, int r, const int8_t* St, int8_t* corr, int corr_off,
                int32_t* maxabs, int lmax, hipStream_t stream);

/* One pass over src: dst = int8(src + E[row][Pn.first] - E[row][Pn.second]); if St is given the
 * projection src * St^T in limbs at corr_off (as uwc_project); E rows copied to
 * corr[li][row][ecopy_off + j] if ecopy_off >= 0. Shapes as uwc_project; Pn and dst 16-byte aligned.
 * Fuses noise_rows' noising (kernels.cu:303-345) with ops.project (ops.py:332-334). */
int uwc_noise_project(const int8_t* src, int rows, int k, int r, const int8_t* E, const uint32_t* Pn, int8_t* dst,
                      const int8_t* St, int8_t* corr, int corr_off, int ecopy_off, int32_t* maxabs, int lmax,
                      hipStream_t stream);

/* The per-nonce operand side of a mined forward in one launch:
 *   ApEA = int8(A + EA[row][P.first] - EA[row][P.second]), given as A + (SpA * EA^T)^T with
 *   SpA (k x 64) = uwc_nonce_noise's SpT of those pairs;
 *   X = A * StB^T -> lmax limbs at corrA[li][row][corr_a_off + j], EA rows copied to
 *   corrA[li][row][ecopy_off + j] (if ecopy_off >= 0), maxabs[0] = max(maxabs[0], max |X|);
 *   Y = Bp * StA^T -> lmax limbs at corrB[li][col][corr_b_off + j], maxabs[1] likewise.
 * A m x k, Bp n x k, StA/StB r x k selection matrices (uwc_proj_matrix / uwc_nonce_noise);
 * m % 32 == 0, n % 32 == 0, k % 256 == 0, r in {16, 32, 64}, lmax 1..4; A, ApEA, Bp, StA,
 * StB, SpA, EA 16-byte aligned.
 * Replaces MinedWeight._forward's noise_rows(A) + project(A) + project(BpEBt) (ops.py:331-336; the
 * operand noising, both projections and their limbs, kernels.cu:303-404). */
int uwc_side_project(const int8_t* A, int m, const int8_t* EA, const int8_t* SpA, int8_t* ApEA, const int8_t* StB,
                     int8_t* corrA, int corr_a_off, int ecopy_off, const int8_t* Bp, int n, const int8_t* StA,
                     int8_t* corrB, int corr_b_off, int k, int r, int32_t* maxabs, int lmax, hipStream_t stream);

/* uwc_side_project for `count` (1..32) nonces sharing the block side (StB, Bp) in one launch:
 * item i as uwc_side_project(A[i], m, EA[i], SpA[i], ApEA[i], StB, corrA[i], corr_a_off, ecopy_off,
 * Bp, n, StA[i], corrB[i], corr_b_off, k, r, maxabs[i], lmax). A, EA, SpA, ApEA, corrA, StA, corrB
 * and maxabs are HOST arrays of `count` device pointers. m % 128 == 0, n % 128 == 0,
 * k % 128 == 0, r in {16, 32, 64}; corr offsets 0 or r (ecopy_off may be -1); A, EA, SpA, ApEA,
 * StA, StB, Bp (and corrA for the E copy) 16-byte aligned.
 * Batches the per-nonce operand side of MinedWeight._forward (ops.py:331-336) over a sweep's
 * group of nonces. */
int uwc_side_project_many(int count, const int8_t* const* A, const int8_t* const* EA, const int8_t* const* SpA,
                          int8_t* const* ApEA, const int8_t* StB, int8_t* const* corrA, int corr_a_off, int ecopy_off,
                          const int8_t* Bp, const int8_t* const* StA, int8_t* const* corrB, int corr_b_off, int m,
                          int n, int k, int r, int32_t* const* maxabs, int lmax, hipStream_t stream);

/* detrt quant_act per row of x (rows x k fp32): q = clamp(rint(fwht_bs(x) / s), -qmax, qmax),
 * s = max(max|y|, 1e-8) / qmax, scale = s * (1 / sqrt(bs)) if bs > 1 else s (bs a power of two
 * dividing k, or 0/1 for none; k % 512 == 0 with bs <= 512, else k <= 40960).
 * Replaces core.quant_act / detgpu quant_act_f32: runtime/detrt/core.py:162-195,
 * runtime/detgpu/kernels.py:75-114. */
int uwc_quant_act_f32(const float* x, int rows, int k, int bs, int qmax, int8_t* q, float* scale, hipStream_t stream);

/* The miner's fused activation quantizer on bf16 rows (x: rows x k bf16 bit patterns, k % 8 == 0):
 * exactly uwc_quant_act_f32 with qmax = 64 on the rows widened to fp32 (block FWHT of size bs,
 * q = clamp(rint(y / s), -64, 64), s = max(max|y|, 1e-8) / 64, scale = s * (1 / sqrt(bs))).
 * Replaces ops.quant_rows_had: miner/ampere/uwc_ampere/ops.py:172-181, kernels.cu:717-778. */
int uwc_quant_rows_had(const uint16_t* x, int rows, int k, int bs, int8_t* q, float* scale, hipStream_t stream);

/* y = fmul(fmul(f32(acc), sx[i]), sw[j]) for an int32 m x n accumulator.
 * Replaces the dequant of runtime/detrt/qwen3.py:125 (detgpu deq, runtime/detgpu/kernels.py:35). */
int uwc_dequant_f32(const int32_t* acc, const float* sx, const float* sw, int m, int n, float* y, hipStream_t stream);

/* ======================================================================== decoder layer
 * detrt's deterministic decoder-layer ops around the exact GEMMs (the fused GPU layer of
 * runtime/detgpu/stages.py:154-168), bit-identical to the CPU reference runtime/detrt
 * (core.py, stage.py:146-233). Row-major fp32 / int8 / int32 buffers; N = B * T tokens of
 * B sequences, token n at position n % T. inv_d = float32(1 / k), eps = float32(rms_norm_eps).
 * A row must fit in LDS (k <= 40960 floats). */

/* q, scale = quant_act(det_rmsnorm(x, w, eps), bs) per row of x (rows x k).
 * Replaces detgpu kernels.rmsnorm_quant: runtime/detgpu/kernels.py:712-728, :117-195. */
int uwc_rmsnorm_quant_f32(const float* x, const float* w, int rows, int k, int bs, float inv_d, float eps, int8_t* q,
                          float* scale, hipStream_t stream);

/* y = det_rmsnorm(x, w, eps) per row (the final-norm hidden state, qwen3.py:300).
 * Replaces core.det_rmsnorm: runtime/detrt/core.py:149-156. */
int uwc_rmsnorm_f32(const float* x, const float* w, int rows, int k, float inv_d, float eps, float* y,
                    hipStream_t stream);

/* From the qkv GEMM's int32 rows (N x (H + 2 Hkv) hd): dequant with s1[n] and sw[col] (or, with
 * s1 = sw = NULL, acc holds the already dequantized fp32 rows), per-head
 * det_rmsnorm with qnw / knw (qknorm != 0: Qwen3; 0: Llama / Mistral), rope from the cos / sin
 * tables (max_pos x hd, row = position), and quant_sym(127) per head: qq (N, H, hd) int8, qs
 * (N, H), kq / vq (N, Hkv, hd), ks / vs (N, Hkv). vt (optional, NULL to skip) receives V
 * transposed per (sequence, kv head) in the attention kernel's key order, (B, Hkv, hd,
 * uwc_vt_tokens(T)) int8. hd in {32, 64, 128}; acc, sw, qnw, knw, the tables, qq, kq, vq 16-byte
 * aligned.
 * Replaces detgpu kernels.qkv_post: runtime/detgpu/kernels.py:788-802, :356-398. */
int uwc_qkv_post(const void* acc, const float* s1, const float* sw, const float* qnw, const float* knw,
                 const float* cos_tab, const float* sin_tab, int B, int T, int H, int Hkv, int hd, float eps, int qknorm,
                 int8_t* qq, float* qs, int8_t* kq, float* ks, int8_t* vq, float* vs, int8_t* vt, hipStream_t stream);

/* Padded key count of the transposed V (T rounded up to 64). Host-side, no GPU work. */
int uwc_vt_tokens(int T);

/* vt = V (N x Hkv x hd int8) in the attention kernel's transposed layout (see uwc_qkv_post). */
int uwc_v_transpose(const int8_t* vq, int B, int T, int Hkv, int hd, int8_t* vt, hipStream_t stream);

/* Exact causal attention per sequence from quantized heads (qq, qs, kq, ks as uwc_qkv_post;
 * vt from uwc_qkv_post / uwc_v_transpose; vs (N, Hkv)): o (N, H * hd) fp32, the O rows.
 * Scores are exact int8 dot products, softmax uses det_exp and an exact fixed-point sum, P is
 * quantized to 14 bits and multiplied as two 7-bit limbs with an exact integer sum.
 * T <= 131072, H % Hkv == 0, hd in {32, 64, 128}; qq, kq, vt, o 16-byte aligned.
 * Replaces detgpu kernels.attention: runtime/detgpu/kernels.py:731-770 (stage.py:171-196). */
int uwc_attention(const int8_t* qq, const float* qs, const int8_t* kq, const float* ks, const int8_t* vt,
                  const float* vs, int B, int T, int H, int Hkv, int hd, float inv_sqrt_hd, float* o,
                  hipStream_t stream);

/* Bytes of the scratch of uwc_attention_ws for B sequences of T tokens and H heads: the
 * exponentials, 4 KiB per 16 queries x 64 keys of the causal triangle (2.2 GB at B = 1,
 * T = 8192, H = 16), then the row maxima, 4 bytes per query and head from a 256-byte boundary;
 * 0 for empty shapes. Host-side, no GPU work. No counterpart in the reference (its kernel keeps
 * nothing between passes). */
uint64_t uwc_attention_scratch_bytes(int B, int T, int H);

/* uwc_attention that keeps every e_ij = det_exp(s_ij - max) it computes for the exact row sum in
 * escratch (at least uwc_attention_scratch_bytes(B, T, H) bytes, 16-byte aligned) and reads it
 * back for the P x V pass instead of recomputing scores and exponentials, in two launches: the
 * row maxima (left in the same scratch), then the sums and P x V. Identical output, about half
 * the VALU work, 8 bytes of HBM traffic per score (each exponential written and read once).
 * Replaces the same reference as uwc_attention. */
int uwc_attention_ws(const int8_t* qq, const float* qs, const int8_t* kq, const float* ks, const int8_t* vt,
                     const float* vs, int B, int T, int H, int Hkv, int hd, float inv_sqrt_hd, float* o,
                     float* escratch, uint64_t escratch_bytes, hipStream_t stream);

/* q, scale = quant_act(fmul(det_silu(g), u), bs) per row, g and u the dequantized halves of the
 * gate_up GEMM's int32 row (rows x 2I; s3[row], sw[col]), or with s3 = sw = NULL its fp32 row.
 * Replaces detgpu kernels.swiglu_quant: runtime/detgpu/kernels.py:816-826. */
int uwc_swiglu_quant(const void* acc, const float* s3, const float* sw, int rows, int I, int bs, int8_t* q,
                     float* scale, hipStream_t stream);

/* out = fadd(x, fmul(fmul(f32(acc), s[row]), sw[col])) (rows x n): R1 and R2; with s = sw = NULL,
 * acc holds the fp32 term and out = fadd(x, acc).
 * Replaces detgpu kernels.dequant_residual: runtime/detgpu/kernels.py:805-813. */
int uwc_dequant_residual(const void* acc, const float* s, const float* sw, const float* x, int rows, int n,
                         float* out, hipStream_t stream);

/* out[t] = table[ids[t]] (V x D fp32); an id outside [0, V) gives a zero row and increments *bad
 * (optional). Replaces the embedding lookup m.embed[tokens] (stage.py:141, detgpu/stages.py:185). */
int uwc_embed_rows(const float* table, int64_t V, int D, const int64_t* ids, int N, float* out, int* bad,
                   hipStream_t stream);

/* out[i] = op(x[i], y[i]) for one of detrt's elementwise fp32 ops exactly as the layer kernels
 * compute it (y unused for SQRT, EXP, SILU): the per-op check that native gfx950 fp32 equals
 * detrt's emulated fp32. Replaces runtime/tests/test_fp32_native.py's per-op GPU check
 * (core.py:45-63 fadd/fsub/fmul/fdiv/fsqrt, :108-146 det_exp, det_silu). */
#define UWC_OP_ADD 0
#define UWC_OP_SUB 1
#define UWC_OP_MUL 2
#define UWC_OP_DIV 3
#define UWC_OP_SQRT 4
#define UWC_OP_EXP 5
#define UWC_OP_SILU 6
int uwc_det_elementwise(int op, const float* x, const float* y, float* out, int64_t n, hipStream_t stream);

/* ======================================================================== stage commitments
 * SHA-256 / RFC 6962 trees as runtime/detrt/stage.py:33-77: a row is little-endian 4-byte
 * words cut into 1 KiB blocks, row_root = MerkleRoot(H(0x00 || block)); a tagged leaf is
 * H(0x00 || tag || u32le index || row_root) with tag "leaf" (trace) or "sout" (stage outputs,
 * spec/stage-program.md:82-88). Digests are 8 SHA-256 state words (big-endian bytes). */

/* For nrows rows of row_words words each: row roots (optional, nrows x 8) and tagged leaves
 * (optional, nrows x 8) with index (index_base + row) % index_mod (index_mod 0: no modulus);
 * tag is the 4 tag bytes as a big-endian word. scratch: nrows * ceil(row_words / 256) * 8 words.
 * Replaces detgpu sha.sout_leaves / _leaf_words: runtime/detgpu/sha.py:139-200. */
int uwc_sha_row_leaves(const uint32_t* rows, int64_t nrows, int row_words, uint32_t* scratch, int64_t scratch_words,
                       uint32_t tag, uint32_t index_base, uint32_t index_mod, uint32_t* row_roots, uint32_t* leaves,
                       hipStream_t stream);

/* roots[t] = MerkleRoot(leaves[t * n .. t * n + n)) for ntrees trees; scratch 2 * ntrees * n * 8 words.
 * Replaces detgpu sha.tree_roots / stage_roots_gpu: runtime/detgpu/sha.py:117-136, :203-215. */
int uwc_sha_merkle_roots(const uint32_t* leaves, int ntrees, int n, uint32_t* scratch, int64_t scratch_words,
                         uint32_t* roots, hipStream_t stream);

/* Measurement aid (no reference counterpart): iters x 8 v_mfma_i32_32x32x32_i8 per wave in a
 * register-only loop, 8 waves on every CU, with constant (random_operands = 0) or seeded random
 * operands; each MFMA is 65,536 int8 ops. Timing it gives the part's sustained int8 MFMA rate,
 * which is lower with switching operands (power-limited clock): the practical ceiling of an int8
 * GEMM on real data. sink: uwc CU count x 512 words. */
int uwc_mfma_rate_probe(int iters, int random_operands, uint32_t* sink, int64_t sink_words, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* UWC_H */
