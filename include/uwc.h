/*
 * uwc.h - C-ABI of libuwc_hip.so, the MI355X (gfx950) int8 x int8 -> int32 GEMM hot path of
 * useful-work-coin: the cuPOW NoisyGEMM miner and the detrt deterministic integer linear.
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
#define UWC_OUT_NONE 0
#define UWC_OUT_I32 1
#define UWC_OUT_BF16 2
#define UWC_OUT_F32 3
#define UWC_WIN_WORDS 10     /* win record: row_off, col_off, digest[8] */
#define UWC_DUMP_WORDS 24    /* tile dump: message[16], digest[8] */

/* Library version (1) and the message of the last failing call on this thread. */
int uwc_version(void);
const char* uwc_last_error(void);

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

/* Exact int32 C = A * B^T for any m, n (k % 64 == 0).
 * Replaces DetLinear.int_gemm's GPU path (torch._int_mm / MinedWeight.forward OUT_I32):
 * runtime/detrt/qwen3.py:106-119. */
int uwc_igemm_i32(const int8_t* A, const int8_t* B, int m, int n, int k, int32_t* C, hipStream_t stream);

/* Y = fmul(fmul(f32(A * B^T), sx[i]), sw[j]) fused in the GEMM epilogue (fp32 m x n).
 * Replaces DetLinear.__call__'s int_gemm + dequant: runtime/detrt/qwen3.py:121-126. */
int uwc_igemm_dequant_f32(const int8_t* A, const int8_t* B, int m, int n, int k, const float* sx, const float* sw,
                          float* Y, hipStream_t stream);

/* Scratch words uwc_b3_root_and_seed needs for an input of nbytes (host-side, no GPU work). */
int uwc_b3_scratch_words(uint64_t nbytes);

/* Keyed BLAKE3 tree root of data (nbytes a positive multiple of 1024) into root_out, and if
 * seed_out is given: seed = BLAKE3(prefix || keyed_BLAKE3(salt, root || dim_le32 || 0^28)).
 * root_out and seed_out may each be NULL.
 * Replaces ops.b3_root_and_seed: miner/ampere/uwc_ampere/ops.py:99-118, kernels.cu:138-244. */
int uwc_b3_root_and_seed(const uint8_t* data, uint64_t nbytes, const uint32_t* key, const uint32_t* prefix,
                         const uint32_t* salt, uint32_t dim, uint32_t* root_out, uint32_t* seed_out,
                         uint32_t* scratch, uint64_t scratch_words, hipStream_t stream);

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

#ifdef __cplusplus
}
#endif

#endif /* UWC_H */
