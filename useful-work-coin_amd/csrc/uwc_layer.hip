// detrt's decoder-layer row ops on gfx950, bit-identical to the CPU reference: the fused
// kernels around the exact int8 GEMMs of one layer (runtime/detgpu/stages.py:154-168 calls
// them; CUDA twins runtime/detgpu/kernels.py:117-353, CPU definitions runtime/detrt/core.py and
// runtime/detrt/stage.py:146-233):
//
//   rmsnorm_quant    N1 / N2 (and the final norm before lm_head) fused with the next quant_act
//   qkv_post         QKV dequant -> per-head RMSNorm (Qwen3) -> rope -> per-head int8 quant of
//                    q, k and v, plus V transposed into the attention kernel's key order
//   swiglu_quant     GU dequant -> SiLU(g) * u -> quant_act (SM, QA4)
//   dequant_residual x + dequant(acc) (R1, R2)
//   embed_rows       the embedding gather (EMBED)
//   rmsnorm          det_rmsnorm alone (the final-norm hidden state)
//
// Row kernels keep one row in LDS (one workgroup of 256 threads per row). qkv_post gives each
// head row to one wave (head_dim 32, 64 or 128; lane d holds elements d, d + 64, ...), so its
// reductions are wave shuffles. Every fp32 step is one correctly rounded op in the reference's
// order (uwc_rows.h).
#include "uwc_rows.h"

// ------------------------------------------------------------------ rmsnorm (+ quant_act)
template <bool QUANT>
__global__ void __launch_bounds__(256) rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w, int k,
                                                      int bs, float inv_d, float eps, i8* __restrict__ q,
                                                      float* __restrict__ scale, float* __restrict__ y) {
  extern __shared__ float dx_row[];
  __shared__ DxRed red;
  const long r = blockIdx.x;
  const float* xr = x + r * k;
  for (int i = threadIdx.x; i < k; i += 256) dx_row[i] = xr[i];
  __syncthreads();
  dx_rmsnorm_lds(dx_row, k, w, inv_d, eps, red);
  if constexpr (QUANT) {
    if (k % 512 == 0 && bs <= 512 && (bs <= 1 || (bs & (bs - 1)) == 0))
      dx_quant_lds_g(dx_row, k, bs > 1 ? __builtin_ctz(bs) : 0, 64, q + r * k, scale + r, red);
    else
      dx_quant_lds(dx_row, k, bs, 64, q + r * k, scale + r, red);
  } else {
    float* yr = y + r * k;
    for (int i = threadIdx.x; i < k; i += 256) yr[i] = dx_row[i];
  }
}

// quant_act (qmax 64, dx_quant_lds_g's ops) of one row held by a wave in the 8-per-lane layout of
// fwht512_rows (lane L: elements 8 L .. 8 L + 7 of each 512-element group): the transform, the
// row's max |y| by a wave reduction, one 8-byte store per group and lane, the scale by lane 0.
template <int G>
__device__ __forceinline__ void wave_quant_row(float (&y)[G][8], int lane, int lbs, i8* __restrict__ qrow,
                                               float* __restrict__ srow) {
  const bool neg = fwht512_rows<G>(y, G, lane, lbs);
  float m2 = 0.f;
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int j = 0; j < 8; j++) m2 = fmaxf(m2, fabsf(y[g][j]));
  m2 = wave_max(m2);
  const float fq = 64.0f;
  const float sc = __fdiv_rn(fmaxf(m2, 1e-8f), fq);
  const double rs = neg ? -1.0 / (double)sc : 1.0 / (double)sc;  // the lane holds y or -y
  i8* qr = qrow + lane * 8;
#pragma unroll
  for (int g = 0; g < G; g++) {
    u64 packed = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float t = fminf(fmaxf(rintf(uwc_div_rd(y[g][j], rs)), -fq), fq);
      packed |= (u64)(u8)(i8)(int)t << (8 * j);
    }
    *reinterpret_cast<u64*>(qr + g * 512) = packed;
  }
  if (lane == 0) *srow = lbs > 0 ? __fmul_rn(sc, __fdiv_rn(1.0f, uwc_sqrt_rn((float)(1 << lbs)))) : sc;
}

// rmsnorm + quant_act with one wave per row and the row in registers, for k = 512 G (G <= 8) and
// bs = 2^lbs <= 512: lane L holds elements 8 L .. 8 L + 7 of each 512-element group (the layout of
// fwht512_rows), the max square and the exact fixed-point sum are wave reductions (a max and an
// int64 sum: any order gives the same value), then the same per-element ops as dx_rmsnorm_lds and
// dx_quant_lds_g. No LDS and no barrier: the 256-thread row kernel's five workgroup reductions
// and LDS passes made it latency-bound (54 us per 8192 x 2048 call against 15 us of traffic).
template <int G>
__global__ void __launch_bounds__(256) rmsnorm_quant_wave_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                                 int rows, int lbs, float inv_d, float eps,
                                                                 i8* __restrict__ q, float* __restrict__ scale) {
  constexpr int K = 512 * G;
  const int lane = threadIdx.x & 63;
  const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves only; no barriers below
  const float* xr = x + r * K + lane * 8;
  float y[G][8];
#pragma unroll
  for (int g = 0; g < G; g++) {
    const float4 a = *reinterpret_cast<const float4*>(xr + g * 512), b = *reinterpret_cast<const float4*>(xr + g * 512 + 4);
    y[g][0] = a.x; y[g][1] = a.y; y[g][2] = a.z; y[g][3] = a.w;
    y[g][4] = b.x; y[g][5] = b.y; y[g][6] = b.z; y[g][7] = b.w;
  }
  float mx = 0.f;
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int j = 0; j < 8; j++) mx = fmaxf(mx, __fmul_rn(y[g][j], y[g][j]));
  mx = wave_max(mx);
  const int sh = dx_shift(mx, dx_log2ceil(K));
  long long acc = 0;
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int j = 0; j < 8; j++) acc += dx_fix(__fmul_rn(y[g][j], y[g][j]), sh);
  acc = wave_sum64(acc);
  const float ss = dx_unfix(acc, sh);
  const float rr = __fdiv_rn(1.0f, uwc_sqrt_rn(__fadd_rn(__fmul_rn(ss, inv_d), eps)));
  const float* wr = w + lane * 8;
#pragma unroll
  for (int g = 0; g < G; g++) {
    const float4 a = *reinterpret_cast<const float4*>(wr + g * 512), b = *reinterpret_cast<const float4*>(wr + g * 512 + 4);
    const float wv[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; j++) y[g][j] = __fmul_rn(__fmul_rn(y[g][j], rr), wv[j]);
  }
  wave_quant_row<G>(y, lane, lbs, q + r * K, scale + r);
}

// ------------------------------------------------------------------ swiglu + quant_act
// swiglu_quant from int32 gate | up rows with one wave per row and the row in registers, for
// I = 512 G (G <= 12) and bs <= 512: element i = fmul(silu(deq(g_i)), deq(u_i)) as in the row
// kernel below, then wave_quant_row. No LDS and no barrier.
template <int G>
__global__ void __launch_bounds__(256) swiglu_quant_wave_kernel(const i32* __restrict__ acc, const float* __restrict__ s3,
                                                                const float* __restrict__ sw, int rows, int lbs,
                                                                i8* __restrict__ q, float* __restrict__ scale) {
  constexpr int I = 512 * G;
  const int lane = threadIdx.x & 63;
  const long r = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= rows) return;  // whole waves only; no barriers below
  const i32* ar = acc + r * 2L * I + lane * 8;
  const float* swr = sw + lane * 8;
  const float sx = s3[r];
  float y[G][8];
#pragma unroll
  for (int g = 0; g < G; g++) {
    const v4i g0 = *reinterpret_cast<const v4i*>(ar + g * 512), g1 = *reinterpret_cast<const v4i*>(ar + g * 512 + 4);
    const v4i u0 = *reinterpret_cast<const v4i*>(ar + I + g * 512), u1 = *reinterpret_cast<const v4i*>(ar + I + g * 512 + 4);
    const float4 wg0 = *reinterpret_cast<const float4*>(swr + g * 512), wg1 = *reinterpret_cast<const float4*>(swr + g * 512 + 4);
    const float4 wu0 = *reinterpret_cast<const float4*>(swr + I + g * 512),
                 wu1 = *reinterpret_cast<const float4*>(swr + I + g * 512 + 4);
    const int gv[8] = {g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
    const int uv[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
    const float wgv[8] = {wg0.x, wg0.y, wg0.z, wg0.w, wg1.x, wg1.y, wg1.z, wg1.w};
    const float wuv[8] = {wu0.x, wu0.y, wu0.z, wu0.w, wu1.x, wu1.y, wu1.z, wu1.w};
#pragma unroll
    for (int j = 0; j < 8; j++) y[g][j] = __fmul_rn(dx_silu(dx_deq(gv[j], sx, wgv[j])), dx_deq(uv[j], sx, wuv[j]));
  }
  wave_quant_row<G>(y, lane, lbs, q + r * (long)I, scale + r);
}

// acc: rows x 2I (gate | up), int32 accumulators dequantized with s3[row], sw[col], or with FP
// already fp32; row value i = fmul(silu(g_i), u_i) (stage.py:220-221).
template <bool FP>
__global__ void __launch_bounds__(256) swiglu_quant_kernel(const void* __restrict__ acc, const float* __restrict__ s3,
                                                           const float* __restrict__ sw, int I, int bs,
                                                           i8* __restrict__ q, float* __restrict__ scale) {
  extern __shared__ float dx_row[];
  __shared__ DxRed red;
  const long r = blockIdx.x;
  for (int i = threadIdx.x; i < I; i += 256) {
    float g, u;
    if constexpr (FP) {
      const float* ar = static_cast<const float*>(acc) + r * 2L * I;
      g = ar[i];
      u = ar[I + i];
    } else {
      const i32* ar = static_cast<const i32*>(acc) + r * 2L * I;
      const float sx = s3[r];
      g = dx_deq(ar[i], sx, sw[i]);
      u = dx_deq(ar[I + i], sx, sw[I + i]);
    }
    dx_row[i] = __fmul_rn(dx_silu(g), u);
  }
  __syncthreads();
  if (I % 512 == 0 && bs <= 512 && (bs <= 1 || (bs & (bs - 1)) == 0))
    dx_quant_lds_g(dx_row, I, bs > 1 ? __builtin_ctz(bs) : 0, 64, q + r * (long)I, scale + r, red);
  else
    dx_quant_lds(dx_row, I, bs, 64, q + r * (long)I, scale + r, red);
}

// ------------------------------------------------------------------ residual
// out = fadd(x, fmul(fmul(f32(acc), s[row]), sw[col])) (stage.py:217, 224); with FP acc is the
// already dequantized fp32 term.
template <bool FP>
__global__ void dequant_residual_kernel(const void* __restrict__ acc, const float* __restrict__ s,
                                        const float* __restrict__ sw, const float* __restrict__ x, int n, u64 total,
                                        float* __restrict__ out) {
  for (u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (u64)gridDim.x * blockDim.x) {
    float y;
    if constexpr (FP) {
      y = static_cast<const float*>(acc)[i];
    } else {
      const u64 r = i / (u64)n;
      const int c = (int)(i - r * n);
      y = dx_deq(static_cast<const i32*>(acc)[i], s[r], sw[c]);
    }
    out[i] = __fadd_rn(x[i], y);
  }
}

// ------------------------------------------------------------------ embedding gather
// out[t] = table[ids[t]]; an id outside [0, V) yields a zero row and bumps *bad (never read out
// of bounds).
__global__ void embed_kernel(const float* __restrict__ table, long V, int D, const int64_t* __restrict__ ids, int N,
                             float* __restrict__ out, int* __restrict__ bad) {
  const int t = blockIdx.x;
  if (t >= N) return;
  const int64_t id = ids[t];
  const bool ok = id >= 0 && id < V;
  if (!ok && threadIdx.x == 0 && bad) atomicAdd(bad, 1);
  const float* src = table + (ok ? id : 0) * (long)D;
  float* dst = out + (long)t * D;
  for (int i = threadIdx.x; i < D; i += blockDim.x) dst[i] = ok ? src[i] : 0.0f;
}

// ------------------------------------------------------------------ qkv_post
// Position of key j inside its 64-key block in the transposed V the attention kernel reads:
// key 16 kb + 4 kg + ki sits at 16 kg + 4 kb + ki (the order in which a 16x16 score block's
// C registers hand keys to the P x V MFMA's k slots).
__host__ __device__ __forceinline__ int vt_pos(int j) {
  return (j & ~63) | (((j >> 2) & 3) << 4) | (((j >> 4) & 3) << 2) | (j & 3);
}

// Four heads per wave: each 16-lane row of a wave holds one head, a lane NV = HD / 16 adjacent
// dims, so the per-head work that does not grow with the head's size (the row maxima and the
// exact sum of squares as 4-step DPP reductions inside the row, the shift, the correctly rounded
// square root and divisions, the float64 reciprocal) runs once per four heads, and every load
// and store of a lane is one contiguous vector. The rope's partner of dim d is d +- HD / 2, the
// same register of lane l ^ 8 in the row (DPP row_ror:8); rot's sign rides on sin (fl(-a b) is
// -fl(a b)). Heads 16 p + 4 w + r for pass p, wave w, row r, so a row's head is one kind (q, k
// or v) and a branch on it splits rows, never a row.
//
// One workgroup takes QP_TOKENS consecutive tokens, each pass of a wave its tokens in turn; the
// column scales of a pass are loaded once for the four. A V head's quantized bytes of the 4
// tokens stay in the row's registers, so when the tokens are positions 4a .. 4a + 3 of one
// sequence (vt_pos keeps those 4 adjacent) each transposed row gets one 4-byte store instead of 4
// byte stores to rows Tp bytes apart.
#define QP_TOKENS 4
template <int HD, bool FP>
__global__ void __launch_bounds__(256) qkv_post_kernel(
    const void* __restrict__ acc, const float* __restrict__ s1, const float* __restrict__ sw,
    const float* __restrict__ qnw, const float* __restrict__ knw, const float* __restrict__ cosb,
    const float* __restrict__ sinb, long N, int T, int H, int Hkv, float inv_hd, float eps, int qknorm,
    i8* __restrict__ qq, float* __restrict__ qs, i8* __restrict__ kq, float* __restrict__ ks, i8* __restrict__ vq,
    float* __restrict__ vs, i8* __restrict__ vt, int Tp) {
  constexpr int NV = HD / 16;  // dims per lane
  constexpr int L = HD == 32 ? 5 : HD == 64 ? 6 : 7;  // log2(HD)
  constexpr int TK = QP_TOKENS;
  static_assert(TK == 4, "a transposed row's 4-byte store holds the bytes of exactly 4 tokens");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, row = lane >> 4, sl = lane & 15;
  const int d0 = NV * sl;
  const long n0 = (long)blockIdx.x * TK;
  const int nt = (int)min((long)TK, N - n0);  // tokens of this workgroup (>= 1)
  const int NH = H + 2 * Hkv;
  const long W = (long)NH * HD;
  int pos[TK], bs[TK];
  float sx[TK];
#pragma unroll
  for (int t = 0; t < TK; t++) {
    const long n = n0 + min(t, nt - 1);
    pos[t] = (int)(n % T);
    bs[t] = (int)(n / T);
    sx[t] = FP ? 1.0f : s1[n];
  }
  const bool packed = nt == TK && bs[0] == bs[TK - 1] && (pos[0] & 3) == 0 && ((uintptr_t)vt & 3) == 0;
  // NV consecutive floats, 16-byte aligned for NV >= 4 (8-byte for NV = 2): the host checks the
  // bases, and every offset used here is a multiple of NV
  auto ldv = [](const float* p, float (&v)[NV]) {
    if constexpr (NV % 4 == 0) {
#pragma unroll
      for (int j = 0; j < NV; j += 4) {
        const float4 x = *reinterpret_cast<const float4*>(p + j);
        v[j] = x.x, v[j + 1] = x.y, v[j + 2] = x.z, v[j + 3] = x.w;
      }
    } else {
      const float2 x = *reinterpret_cast<const float2*>(p);
      v[0] = x.x, v[1] = x.y;
    }
  };
  float qn[NV], kn[NV];
  if (qknorm) {
    ldv(qnw + d0, qn);
    ldv(knw + d0, kn);
  }
  const bool low = sl < 8;  // the row's lanes holding the first half of the head
  for (int p = 0; p * 16 < NH; p++) {
    const int hh = 16 * p + 4 * wave + row;  // this row's head
    const bool live = hh < NH;
    const int hc = min(hh, NH - 1);
    const bool isq = hc < H, isv = hc >= H + Hkv;
    const int col = hc * HD + d0;
    float swv[NV];
    if constexpr (!FP) ldv(sw + col, swv);
    u32 pk[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) pk[j] = 0;
#pragma unroll
    for (int t = 0; t < TK; t++) {
      if (t >= nt) break;
      const long n = n0 + t;
      float v[NV];
      if constexpr (FP) {
        ldv(static_cast<const float*>(acc) + n * W + col, v);
      } else {
        const i32* a = static_cast<const i32*>(acc) + n * W + col;
        int av[NV];
        if constexpr (NV % 4 == 0) {
#pragma unroll
          for (int j = 0; j < NV; j += 4) {
            const int4 x = *reinterpret_cast<const int4*>(a + j);
            av[j] = x.x, av[j + 1] = x.y, av[j + 2] = x.z, av[j + 3] = x.w;
          }
        } else {
          const int2 x = *reinterpret_cast<const int2*>(a);
          av[0] = x.x, av[1] = x.y;
        }
#pragma unroll
        for (int j = 0; j < NV; j++) v[j] = dx_deq(av[j], sx[t], swv[j]);
      }
      if (!isv) {
        if (qknorm) {  // det_rmsnorm over the head (qwen3.py:214-216)
          float mx = 0.f;
#pragma unroll
          for (int j = 0; j < NV; j++) mx = fmaxf(mx, __fmul_rn(v[j], v[j]));
          const int sh = dx_shift(row16_max(mx), L);
          long long sq = 0;
#pragma unroll
          for (int j = 0; j < NV; j++) sq += dx_fix(__fmul_rn(v[j], v[j]), sh);
          const float ss = dx_unfix(row16_sum64(sq), sh);
          const float r = __fdiv_rn(1.0f, uwc_sqrt_rn(__fadd_rn(__fmul_rn(ss, inv_hd), eps)));
#pragma unroll
          for (int j = 0; j < NV; j++) v[j] = __fmul_rn(__fmul_rn(v[j], r), isq ? qn[j] : kn[j]);
        }
        // rope: fadd(fmul(z, cos), fmul(rot(z), sin)), rot(z) = cat(-z[half:], z[:half])
        float cs[NV], sn[NV];
        ldv(cosb + (long)pos[t] * HD + d0, cs);
        ldv(sinb + (long)pos[t] * HD + d0, sn);
        float part[NV];
#pragma unroll
        for (int j = 0; j < NV; j++) part[j] = qa_dpp<0x128>(v[j]);  // row_ror:8: lane l ^ 8 of the row
#pragma unroll
        for (int j = 0; j < NV; j++) v[j] = __fadd_rn(__fmul_rn(v[j], cs[j]), __fmul_rn(part[j], low ? -sn[j] : sn[j]));
      }
      // quant_sym(qmax = 127) over the head (core.py:160-166)
      float am = 0.f;
#pragma unroll
      for (int j = 0; j < NV; j++) am = fmaxf(am, fabsf(v[j]));
      const float s = __fdiv_rn(fmaxf(row16_max(am), 1e-8f), 127.0f);
      const double rs = 1.0 / (double)s;
      u32 qb[NV / 2];  // the lane's NV quantized bytes, 2 per 16-bit half (NV >= 2)
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const int qv = (int)fminf(fmaxf(rintf(uwc_div_rd(v[j], rs)), -127.f), 127.f);
        const u32 b = (u32)qv & 0xffu;
        if (j % 2 == 0) qb[j / 2] = b;
        else qb[j / 2] |= b << 8;
        if (packed) pk[j] |= b << (8 * t);
      }
      if (live) {
        i8* qo;
        float* so;
        if (isq) {
          qo = qq + (n * H + hh) * HD;
          so = qs + n * H + hh;
        } else if (!isv) {
          qo = kq + (n * Hkv + (hh - H)) * HD;
          so = ks + n * Hkv + (hh - H);
        } else {
          qo = vq + (n * Hkv + (hh - H - Hkv)) * HD;
          so = vs + n * Hkv + (hh - H - Hkv);
        }
        if constexpr (NV == 2) {
          *reinterpret_cast<unsigned short*>(qo + d0) = (unsigned short)qb[0];
        } else {
#pragma unroll
          for (int j = 0; j < NV / 4; j++)
            *reinterpret_cast<u32*>(qo + d0 + 4 * j) = qb[2 * j] | (qb[2 * j + 1] << 16);
        }
        if (sl == 0) *so = s;
        if (vt && isv && !packed) {
          const int hk = hh - H - Hkv;
#pragma unroll
          for (int j = 0; j < NV; j++)
            vt[((long)(bs[t] * Hkv + hk) * HD + d0 + j) * Tp + vt_pos(pos[t])] = (i8)((qb[j / 2] >> (8 * (j % 2))) & 0xff);
        }
      }
    }
    if (live && vt && isv && packed) {
      const int hk = hh - H - Hkv;
#pragma unroll
      for (int j = 0; j < NV; j++)
        *reinterpret_cast<u32*>(vt + ((long)(bs[0] * Hkv + hk) * HD + d0 + j) * Tp + vt_pos(pos[0])) = pk[j];
    }
  }
}

// V (N x Hkv x HD int8) transposed per (sequence, kv head) into the attention kernel's layout.
__global__ void v_transpose_kernel(const i8* __restrict__ vq, int T, int Hkv, int HD, int Tp, i8* __restrict__ vt) {
  const int n = blockIdx.x, bseq = n / T, pos = n % T;
  for (int i = threadIdx.x; i < Hkv * HD; i += blockDim.x) {
    const int hk = i / HD, d = i % HD;
    vt[((long)(bseq * Hkv + hk) * HD + d) * Tp + vt_pos(pos)] = vq[(long)n * Hkv * HD + i];
  }
}

// ------------------------------------------------------------------ per-op conformance
// out[i] = op(x[i], y[i]) for one of detrt's elementwise fp32 ops, as the kernels above compute
// it: the per-op check of native fp32 against detrt's emulation (runtime/tests/test_fp32_native.py).
__global__ void det_elementwise_kernel(int op, const float* __restrict__ x, const float* __restrict__ y,
                                       float* __restrict__ out, u64 n) {
  for (u64 i = (u64)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (u64)gridDim.x * blockDim.x) {
    const float a = x[i], b = y ? y[i] : 0.0f;
    float r;
    switch (op) {
      case UWC_OP_ADD: r = __fadd_rn(a, b); break;
      case UWC_OP_SUB: r = __fsub_rn(a, b); break;
      case UWC_OP_MUL: r = __fmul_rn(a, b); break;
      case UWC_OP_DIV: r = __fdiv_rn(a, b); break;
      case UWC_OP_SQRT: r = uwc_sqrt_rn(a); break;
      case UWC_OP_EXP: r = dx_exp(a); break;
      default: r = dx_silu(a); break;
    }
    out[i] = r;
  }
}

// ------------------------------------------------------------------ C-ABI
extern "C" int uwc_det_elementwise(int op, const float* x, const float* y, float* out, int64_t n, hipStream_t stream) {
  const char* fn = "uwc_det_elementwise";
  if (op < UWC_OP_ADD || op > UWC_OP_SILU) return uwc_fail("%s: unknown op %d", fn, op);
  if (!x || !out || n < 0 || (op <= UWC_OP_DIV && !y)) return uwc_fail("%s: null or empty arguments", fn);
  if (n == 0) return UWC_OK;
  const u64 blocks = ((u64)n + 255) / 256;
  hipLaunchKernelGGL(det_elementwise_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, stream,
                     op, x, y, out, (u64)n);
  return uwc_launch_status(fn);
}

static int row_lds(const char* fn, const void* kern, int k, size_t& smem) {
  smem = (size_t)k * 4;
  if (smem > 160 * 1024) return uwc_fail("%s: a row of %d floats exceeds LDS", fn, k);
  if (smem > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) return uwc_fail("%s: cannot raise LDS to %zu bytes: %s", fn, smem, hipGetErrorString(e));
  }
  return UWC_OK;
}

static int check_bs(const char* fn, int bs, int k) {
  if (bs > 1 && ((bs & (bs - 1)) || k % bs)) return uwc_fail("%s: bs=%d must be a power of two dividing %d", fn, bs, k);
  return UWC_OK;
}

extern "C" int uwc_rmsnorm_quant_f32(const float* x, const float* w, int rows, int k, int bs, float inv_d, float eps,
                                     int8_t* q, float* scale, hipStream_t stream) {
  const char* fn = "uwc_rmsnorm_quant_f32";
  if (!x || !w || !q || !scale || rows < 0 || k <= 0) return uwc_fail("%s: null or empty arguments", fn);
  int st = check_bs(fn, bs, k);
  if (st) return st;
  if (rows == 0) return UWC_OK;
  const int bse = bs > 1 ? bs : 1;
  if (k % 512 == 0 && k <= 4096 && bse <= 512 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)w & 15) == 0 &&
      ((uintptr_t)q & 7) == 0) {
    const int lbs = __builtin_ctz((unsigned)bse);
    const dim3 grid((unsigned)((rows + 3) / 4));
    switch (k / 512) {
      case 1: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<1>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 2: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<2>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 3: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<3>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 4: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<4>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 5: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<5>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 6: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<6>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      case 7: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<7>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
      default: hipLaunchKernelGGL(rmsnorm_quant_wave_kernel<8>, grid, dim3(256), 0, stream, x, w, rows, lbs, inv_d, eps, q, scale); break;
    }
    return uwc_launch_status(fn);
  }
  size_t smem;
  if ((st = row_lds(fn, (const void*)rmsnorm_kernel<true>, k, smem))) return st;
  hipLaunchKernelGGL(rmsnorm_kernel<true>, dim3(rows), dim3(256), smem, stream, x, w, k, bs, inv_d, eps, q, scale,
                     (float*)nullptr);
  return uwc_launch_status(fn);
}

extern "C" int uwc_rmsnorm_f32(const float* x, const float* w, int rows, int k, float inv_d, float eps, float* y,
                               hipStream_t stream) {
  const char* fn = "uwc_rmsnorm_f32";
  if (!x || !w || !y || rows < 0 || k <= 0) return uwc_fail("%s: null or empty arguments", fn);
  if (rows == 0) return UWC_OK;
  size_t smem;
  int st = row_lds(fn, (const void*)rmsnorm_kernel<false>, k, smem);
  if (st) return st;
  hipLaunchKernelGGL(rmsnorm_kernel<false>, dim3(rows), dim3(256), smem, stream, x, w, k, 0, inv_d, eps,
                     (i8*)nullptr, (float*)nullptr, y);
  return uwc_launch_status(fn);
}

extern "C" int uwc_swiglu_quant(const void* acc, const float* s3, const float* sw, int rows, int I, int bs,
                                int8_t* q, float* scale, hipStream_t stream) {
  const char* fn = "uwc_swiglu_quant";
  if (!acc || !q || !scale || rows < 0 || I <= 0) return uwc_fail("%s: null or empty arguments", fn);
  if (!s3 != !sw) return uwc_fail("%s: give both scales (int32 acc) or neither (fp32 rows)", fn);
  int st = check_bs(fn, bs, I);
  if (st) return st;
  if (rows == 0) return UWC_OK;
  const int bse = bs > 1 ? bs : 1;
  if (s3 && I % 512 == 0 && I <= 512 * 12 && bse <= 512 && ((uintptr_t)acc & 15) == 0 && ((uintptr_t)sw & 15) == 0 &&
      ((uintptr_t)q & 7) == 0) {
    const int lbs = __builtin_ctz((unsigned)bse);
    const dim3 grid((unsigned)((rows + 3) / 4));
    const i32* a = static_cast<const i32*>(acc);
#define SWQ(G)                                                                                                        \
  case G: hipLaunchKernelGGL(swiglu_quant_wave_kernel<G>, grid, dim3(256), 0, stream, a, s3, sw, rows, lbs, q, scale); break;
    switch (I / 512) {
      SWQ(1) SWQ(2) SWQ(3) SWQ(4) SWQ(5) SWQ(6) SWQ(7) SWQ(8) SWQ(9) SWQ(10) SWQ(11)
      default: hipLaunchKernelGGL(swiglu_quant_wave_kernel<12>, grid, dim3(256), 0, stream, a, s3, sw, rows, lbs, q, scale); break;
    }
#undef SWQ
    return uwc_launch_status(fn);
  }
  size_t smem;
  if (s3) {
    if ((st = row_lds(fn, (const void*)swiglu_quant_kernel<false>, I, smem))) return st;
    hipLaunchKernelGGL(swiglu_quant_kernel<false>, dim3(rows), dim3(256), smem, stream, acc, s3, sw, I, bs, q, scale);
  } else {
    if ((st = row_lds(fn, (const void*)swiglu_quant_kernel<true>, I, smem))) return st;
    hipLaunchKernelGGL(swiglu_quant_kernel<true>, dim3(rows), dim3(256), smem, stream, acc, s3, sw, I, bs, q, scale);
  }
  return uwc_launch_status(fn);
}

extern "C" int uwc_dequant_residual(const void* acc, const float* s, const float* sw, const float* x, int rows, int n,
                                    float* out, hipStream_t stream) {
  const char* fn = "uwc_dequant_residual";
  if (!acc || !x || !out || rows < 0 || n <= 0) return uwc_fail("%s: null or empty arguments", fn);
  if (!s != !sw) return uwc_fail("%s: give both scales (int32 acc) or neither (fp32 rows)", fn);
  const u64 total = (u64)rows * n;
  if (total == 0) return UWC_OK;
  const u64 blocks = (total + 255) / 256;
  const dim3 grid((unsigned)(blocks < 65536 ? blocks : 65536));
  if (s)
    hipLaunchKernelGGL(dequant_residual_kernel<false>, grid, dim3(256), 0, stream, acc, s, sw, x, n, total, out);
  else
    hipLaunchKernelGGL(dequant_residual_kernel<true>, grid, dim3(256), 0, stream, acc, s, sw, x, n, total, out);
  return uwc_launch_status(fn);
}

extern "C" int uwc_embed_rows(const float* table, int64_t V, int D, const int64_t* ids, int N, float* out, int* bad,
                              hipStream_t stream) {
  const char* fn = "uwc_embed_rows";
  if (!table || !ids || !out || V <= 0 || D <= 0 || N < 0) return uwc_fail("%s: null or empty arguments", fn);
  if (N == 0) return UWC_OK;
  hipLaunchKernelGGL(embed_kernel, dim3(N), dim3(256), 0, stream, table, (long)V, D, ids, N, out, bad);
  return uwc_launch_status(fn);
}

extern "C" int uwc_vt_tokens(int T) { return T <= 0 ? 0 : ((T + 63) / 64) * 64; }

extern "C" int uwc_qkv_post(const void* acc, const float* s1, const float* sw, const float* qnw, const float* knw,
                            const float* cosb, const float* sinb, int B, int T, int H, int Hkv, int hd, float eps,
                            int qknorm, int8_t* qq, float* qs, int8_t* kq, float* ks, int8_t* vq, float* vs, int8_t* vt,
                            hipStream_t stream) {
  const char* fn = "uwc_qkv_post";
  if (!acc || !cosb || !sinb || !qq || !qs || !kq || !ks || !vq || !vs) return uwc_fail("%s: null arguments", fn);
  if (!s1 != !sw) return uwc_fail("%s: give both scales (int32 acc) or neither (fp32 rows)", fn);
  if (qknorm && (!qnw || !knw)) return uwc_fail("%s: q/k norm weights are needed with qknorm", fn);
  if (B < 0 || T <= 0 || H <= 0 || Hkv <= 0 || H % Hkv) return uwc_fail("%s: bad B=%d T=%d H=%d Hkv=%d", fn, B, T, H, Hkv);
  if (hd != 32 && hd != 64 && hd != 128) return uwc_fail("%s: head_dim %d not in {32, 64, 128}", fn, hd);
  if (((uintptr_t)acc | (uintptr_t)sw | (uintptr_t)qnw | (uintptr_t)knw | (uintptr_t)cosb | (uintptr_t)sinb |
       (uintptr_t)qq | (uintptr_t)kq | (uintptr_t)vq) & 15)
    return uwc_fail("%s: acc, sw, qnw, knw, cos, sin, qq, kq, vq must be 16-byte aligned", fn);
  const long N = (long)B * T;
  if (N == 0) return UWC_OK;
  if (N > 0x7fffffff) return uwc_fail("%s: too many tokens", fn);
  const float inv_hd = (float)(1.0 / (double)hd);
  const int Tp = uwc_vt_tokens(T);
  const dim3 grid((unsigned)((N + QP_TOKENS - 1) / QP_TOKENS));
#define QKV_LAUNCH(HD)                                                                                               \
  do {                                                                                                               \
    if (s1)                                                                                                          \
      hipLaunchKernelGGL((qkv_post_kernel<HD, false>), grid, dim3(256), 0, stream, acc, s1, sw, qnw, knw, cosb,      \
                         sinb, N, T, H, Hkv, inv_hd, eps, qknorm, qq, qs, kq, ks, vq, vs, vt, Tp);                    \
    else                                                                                                             \
      hipLaunchKernelGGL((qkv_post_kernel<HD, true>), grid, dim3(256), 0, stream, acc, s1, sw, qnw, knw, cosb,       \
                         sinb, N, T, H, Hkv, inv_hd, eps, qknorm, qq, qs, kq, ks, vq, vs, vt, Tp);                    \
  } while (0)
  if (hd == 32) QKV_LAUNCH(32);
  else if (hd == 64) QKV_LAUNCH(64);
  else QKV_LAUNCH(128);
#undef QKV_LAUNCH
  return uwc_launch_status(fn);
}

extern "C" int uwc_v_transpose(const int8_t* vq, int B, int T, int Hkv, int hd, int8_t* vt, hipStream_t stream) {
  const char* fn = "uwc_v_transpose";
  if (!vq || !vt || B < 0 || T <= 0 || Hkv <= 0 || hd <= 0) return uwc_fail("%s: null or empty arguments", fn);
  const long N = (long)B * T;
  if (N == 0) return UWC_OK;
  hipLaunchKernelGGL(v_transpose_kernel, dim3((unsigned)N), dim3(256), 0, stream, vq, T, Hkv, hd, uwc_vt_tokens(T), vt);
  return uwc_launch_status(fn);
}
