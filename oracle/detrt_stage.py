"""CPU restatement of detrt's deterministic decoder layer, its stage program and the SHA-256
stage commitments (numpy float32 / int64 / hashlib).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this module, and only as the checker: the product path
(useful-work-coin_amd/uwc_amd) never imports it.

Arithmetic: detrt evaluates every fp32 + - * / sqrt as one correctly rounded IEEE binary32
operation (runtime/detrt/core.py:1-17). numpy's float32 ufuncs are exactly that (one rounding,
never contracted into a fused multiply-add), so each f* helper below is the plain float32 op.
Integer sums are int64 and exact; int -> float conversions round to nearest even.

Pinned by (tests/test_detrt_stage_oracle.py): every leaf row of the reference's Go-referee
stage fixtures (tiny Qwen3 and tiny Llama stages of 12 tokens through both layers, all 26 op
kinds; the real Qwen3-1.7B stages at 8 tokens for every non-GEMM op), and the three
committed stage trace roots of each tiny fixture (SHA-256 over every row, in program order).
hashlib's SHA-256 is the standard; the tree shapes are RFC 6962's (runtime/detrt/stage.py:33-52).
"""
from __future__ import annotations

import hashlib
import math
import struct

import numpy as np

F32, F64, I64 = np.float32, np.float64, np.int64

# runtime/detrt/core.py:101-105: 2**f on [0, 1) (degree-7 least squares), log2(e)
EXP2 = [1.0, 0.6931471824645996, 0.2402263879776001, 0.055505119264125824, 0.00961404386907816,
        0.001342222560197115, 0.0001435537706129253, 2.1489791834028438e-05]
LOG2E = 1.4426950408889634
# runtime/detrt/qwen3.py:36-38
MAX_KEYS = 1 << 20
P_LEVELS = 16383
BLOCK = 1024  # runtime/detrt/stage.py:25

# op codes and names of the stage program (runtime/detrt/stage.py:27-30)
OPS = ["EMBED", "N1", "QA1", "QKV", "QN", "KN", "QR", "KR", "KQ", "VQ", "QQ", "VT", "VS", "S", "P", "O",
       "QA2", "OP", "R1", "N2", "QA3", "GU", "SM", "QA4", "DN", "R2"]


def c32(v: float) -> np.float32:
    """A float constant rounded once to float32 (core.py:37-43)."""
    return np.float32(v)


# ------------------------------------------------------------------ exact row sums, exp, norms
def exact_rowsum(x: np.ndarray, max_terms: int) -> np.ndarray:
    """core.py:77-97: each term rounded once (half-even) to int64 fixed point at scale 2**shift,
    shift = (62 - L) - e with 2**(e-1) <= max|x| < 2**e, L = ceil(log2(max_terms)); exact
    int64 sum, then to float64 (rounded) and float32."""
    L = max(1, math.ceil(math.log2(max_terms)))
    x = np.asarray(x, F32)
    amax = np.abs(x).max(axis=-1, keepdims=True)
    _, e = np.frexp(amax)
    shift = np.clip((62 - L) - e.astype(I64), -1000, 1000)
    q = np.rint(np.ldexp(x.astype(F64), shift)).astype(I64)
    s = q.sum(axis=-1, keepdims=True)
    return np.ldexp(s.astype(F64), -shift).astype(F32)[..., 0]


def pow2_f32(n: np.ndarray) -> np.ndarray:
    """core.py:66-68: exactly 2**n from the bit pattern."""
    return ((n.astype(np.int32) + 127) << 23).view(F32)


def det_exp(z: np.ndarray) -> np.ndarray:
    """core.py:108-126."""
    z = np.asarray(z, F32)
    with np.errstate(invalid="ignore", over="ignore"):
        t = z * c32(LOG2E)
        under = t < c32(-126.0)
        over = t >= c32(128.0)
        t = np.where(under | over | np.isnan(t), F32(0), t).astype(F32)
        n = np.floor(t)
        f = t - n
        p = np.full_like(f, c32(EXP2[7]))
        for cf in reversed(EXP2[:7]):
            p = p * f + c32(cf)  # two roundings: the product, then the sum
        r = p * pow2_f32(n)
    r = np.where(under, F32(0), r)
    r = np.where(over, F32(np.inf), r)
    return np.where(np.isnan(z), z, r).astype(F32)


def det_silu(x: np.ndarray) -> np.ndarray:
    """core.py:144-146."""
    x = np.asarray(x, F32)
    return x / (c32(1.0) + det_exp(-x))


def det_rmsnorm(x: np.ndarray, w: np.ndarray, eps32: np.float32) -> np.ndarray:
    """core.py:149-156: x * (1 / sqrt(mean(x^2) + eps)) * w with an exact sum of squares."""
    x = np.asarray(x, F32)
    d = x.shape[-1]
    ss = exact_rowsum(x * x, d)
    mean = ss * c32(1.0 / d)
    r = c32(1.0) / np.sqrt(mean + eps32)
    return (x * r[..., None]) * np.asarray(w, F32)


# ------------------------------------------------------------------ quantization
def quant_sym(x: np.ndarray, qmax: int):
    """core.py:160-166: s = max(max|x|, 1e-8) / qmax, q = round_half_even(x / s) clamped."""
    x = np.asarray(x, F32)
    amax = np.abs(x).max(axis=-1, keepdims=True)
    s = np.maximum(amax, c32(1e-8)) / c32(float(qmax))
    q = np.clip(np.rint(x / s), -qmax, qmax)
    return q.astype(np.int32), s


def fwht(x: np.ndarray, bs: int) -> np.ndarray:
    """core.py:169-183: unnormalized block Walsh-Hadamard, stages h = 1, 2, 4, ..."""
    x = np.asarray(x, F32)
    if bs <= 1:
        return x
    shp = x.shape
    k = shp[-1]
    v = x.reshape(-1, k)
    h = 1
    while h < bs:
        v = v.reshape(v.shape[0], k // (2 * h), 2, h)
        a, b = v[:, :, 0, :], v[:, :, 1, :]
        v = np.stack([a + b, a - b], axis=2).reshape(-1, k)
        h *= 2
    return v.reshape(shp)


def quant_act(x: np.ndarray, bs: int, qmax: int = 64):
    """core.py:186-193: (int8-valued q, fp32 scale with the 1/sqrt(bs) fold)."""
    y = fwht(x, bs)
    q, s = quant_sym(y, qmax)
    if bs > 1:
        s = s * (c32(1.0) / np.sqrt(c32(float(bs))))
    return q.astype(np.int8), s[..., 0]


def lin_bs(hadamard_block: int, k: int) -> int:
    """DetLinear's block size (qwen3.py:75)."""
    return min(hadamard_block, k & -k) if hadamard_block else 0


def int_gemm(q: np.ndarray, Wq: np.ndarray) -> np.ndarray:
    """Exact q @ Wq^T as the reference's CPU path computes it, a float64 GEMM (qwen3.py:106-110):
    every product is an integer below 2**14 and every partial sum below 2**53 for k < 2**39, so
    any summation order is exact."""
    return (np.asarray(q, F64) @ np.asarray(Wq, F64).T).astype(I64)


def dequant(acc: np.ndarray, s: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """fmul(fmul(f32(acc), s_x), s_w) (qwen3.py:125)."""
    return (acc.astype(F32) * s[:, None].astype(F32)) * sw[None, :].astype(F32)


def linear(x: np.ndarray, Wq: np.ndarray, sw: np.ndarray, bs: int):
    """DetLinear.__call__ (qwen3.py:121-126): (q, s, y)."""
    q, s = quant_act(x, bs)
    return q, s, dequant(int_gemm(q, Wq), s, sw)


def rope(z: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """qwen3.py:232-237 / stage.py:157-158: fadd(fmul(z, cos), fmul(rot(z), sin)),
    rot(z) = cat(-z[half:], z[:half])."""
    half = z.shape[-1] // 2
    rot = np.concatenate([-z[..., half:], z[..., :half]], axis=-1)
    return z * cos + rot * sin


def inv_sqrt_hd(hd: int) -> np.float32:
    """qwen3.py:197: float32 of 1 / sqrt(hd) computed in float64."""
    return np.float32(1.0 / np.sqrt(hd))


# ------------------------------------------------------------------ attention
def attention(qq, qs, kq, ks, vq, vs, inv_sqrt: np.float32):
    """Causal attention of one sequence from quantized heads (stage.py:171-196, qwen3.py:255-282).

    qq (T, H, hd), kq / vq (T, Hkv, hd) integer-valued; qs (T, H, 1), ks / vs (T, Hkv, 1) fp32.
    Returns (sc (H, T, T) with -inf above the diagonal, pi (H, T, T) int32, sp (H, T, 1), o (H, T, hd))."""
    return _attend(qq, qs, kq, ks, vq, vs, inv_sqrt, np.arange(qq.shape[0]))


def attention_rows(qq, qs, kq, ks, vq, vs, inv_sqrt: np.float32, rows):
    """attention() for the query positions `rows` only (every key of the sequence is used): the
    same computation restricted to those rows, without the (H, T, T) arrays, for long sequences.
    Returns (sc, pi, sp, o) with the row axis of length len(rows)."""
    rows = np.asarray(rows, np.int64)
    return _attend(qq[rows], qs[rows], kq, ks, vq, vs, inv_sqrt, rows)


def _attend(qq, qs, kq, ks, vq, vs, inv_sqrt, qpos):
    """Query rows qq (R, H, hd) at positions qpos (R) against all T keys of kq / vq."""
    H = qq.shape[1]
    T, Hkv = kq.shape[0], kq.shape[1]
    rep = H // Hkv
    # float64 products are exact here: |q . k| < 2**24 and |sum p v| < 16383 * 127 * T < 2**53
    K = np.repeat(kq.transpose(1, 0, 2), rep, axis=0).astype(F64)   # (H, T, hd)
    SK = np.repeat(ks.transpose(1, 0, 2), rep, axis=0)               # (H, T, 1)
    V = np.repeat(vq.transpose(1, 0, 2), rep, axis=0).astype(F64)
    SV = np.repeat(vs.transpose(1, 0, 2), rep, axis=0)
    Q, QS = qq.transpose(1, 0, 2).astype(F64), qs.transpose(1, 0, 2)
    sc_int = (Q @ K.transpose(0, 2, 1)).astype(F32)                 # exact: |s| < 2**24
    sc = ((sc_int * QS) * SK.transpose(0, 2, 1)) * inv_sqrt
    mask = np.arange(T)[None, :] <= np.asarray(qpos)[:, None]
    sc = np.where(mask[None], sc, F32(-np.inf)).astype(F32)
    mx = sc.max(axis=-1, keepdims=True)
    with np.errstate(invalid="ignore"):
        e = det_exp(sc - mx)
    den = exact_rowsum(e, MAX_KEYS)
    Pr = e / den[..., None]
    Pv = Pr * SV.transpose(0, 2, 1)
    pmax = Pv.max(axis=-1, keepdims=True)
    sp = np.maximum(pmax, c32(1e-30)) / c32(float(P_LEVELS))
    pi = np.clip(np.rint(Pv / sp), 0, P_LEVELS).astype(np.int32)
    acc = (pi.astype(F64) @ V).astype(I64)                            # = sum over key chunks of (hi << 7) + lo
    o = acc.astype(F32) * sp
    return sc, pi, sp, o


# ------------------------------------------------------------------ model and stage program
class Model:
    """The deterministic model's parameters as detrt holds them (qwen3.py:165-199): fp32 embedding,
    norms and rope tables; linears as (Wq int8 n x k, sw fp32 n) with the Hadamard block bs."""

    def __init__(self, cfg: dict, embed, norms: list[dict], lins: list[dict], cos, sin, lm_head=None, final_norm=None):
        self.cfg = cfg
        self.embed, self.norms, self.lins, self.cos, self.sin = embed, norms, lins, cos, sin
        self.lm_head, self.final_norm = lm_head, final_norm

    @property
    def eps32(self) -> np.float32:
        return np.array([self.cfg["eps_bits"]], np.uint32).view(F32)[0]

    def bs(self, k: int) -> int:
        return lin_bs(self.cfg["Bs"], k)


def program(H: int, Hkv: int, hd: int, T: int, l0: int, l1: int) -> list[tuple]:
    """Leaf list (op, layer, t, h) in the canonical order (stage.py:89-110)."""
    out = []
    if l0 == 0:
        out += [("EMBED", 0, t, -1) for t in range(T)]
    for l in range(l0, l1):
        per_t = lambda op: [(op, l, t, -1) for t in range(T)]
        per_th = lambda op, nh: [(op, l, t, h) for t in range(T) for h in range(nh)]
        out += per_t("N1") + per_t("QA1") + per_t("QKV")
        out += per_th("QN", H) + per_th("KN", Hkv) + per_th("QR", H) + per_th("KR", Hkv)
        out += per_th("KQ", Hkv) + per_th("VQ", Hkv) + per_th("QQ", H)
        out += [("VT", l, d, h) for h in range(Hkv) for d in range(hd)]
        out += [("VS", l, -1, h) for h in range(Hkv)]
        out += per_th("S", H) + per_th("P", H) + per_th("O", H)
        for op in ("QA2", "OP", "R1", "N2", "QA3", "GU", "SM", "QA4", "DN", "R2"):
            out += per_t(op)
    return out


def _qrow(q, s) -> np.ndarray:
    return np.concatenate([np.asarray(q, np.int32).ravel(), np.asarray([s], F32).view(np.int32)])


def layer(m: Model, l: int, x: np.ndarray, put=None) -> np.ndarray:
    """One decoder layer over a T-token sequence (stage.py:146-233); put(op, l, t, h, row) receives
    every leaf row when given. Returns the layer output R2 (T, D)."""
    cfg = m.cfg
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    T = x.shape[0]
    nrm, lin = m.norms[l], m.lins[l]
    eps = m.eps32
    h1 = det_rmsnorm(x, nrm["in_norm"], eps)
    q1, s1, qkv = linear(h1, *lin["qkv"], m.bs(h1.shape[1]))
    q, k, v = qkv[:, :H * hd], qkv[:, H * hd:(H + Hkv) * hd], qkv[:, (H + Hkv) * hd:]
    if cfg["arch"] == 0:
        qn = det_rmsnorm(q.reshape(T, H, hd), nrm["q_norm"], eps)
        kn = det_rmsnorm(k.reshape(T, Hkv, hd), nrm["k_norm"], eps)
    else:
        qn, kn = q.reshape(T, H, hd), k.reshape(T, Hkv, hd)
    cos, sin = m.cos[:T][:, None, :], m.sin[:T][:, None, :]
    qr, kr = rope(qn, cos, sin), rope(kn, cos, sin)
    kq, ks = quant_sym(kr, 127)
    vq, vs = quant_sym(v.reshape(T, Hkv, hd), 127)
    qq, qs = quant_sym(qr, 127)
    sc, pi, sp, o = attention(qq, qs, kq, ks, vq, vs, inv_sqrt_hd(hd))
    oc = o.transpose(1, 0, 2).reshape(T, H * hd)
    q2, s2, op = linear(oc, *lin["o"], m.bs(oc.shape[1]))
    r1 = x + op
    h2 = det_rmsnorm(r1, nrm["post_norm"], eps)
    q3, s3, gu = linear(h2, *lin["gu"], m.bs(h2.shape[1]))
    I_ = gu.shape[1] // 2
    sm = det_silu(gu[:, :I_]) * gu[:, I_:]
    q4, s4, dn = linear(sm, *lin["down"], m.bs(sm.shape[1]))
    r2 = r1 + dn
    if put is not None:
        for t in range(T):
            put("N1", l, t, -1, h1[t])
            put("QA1", l, t, -1, _qrow(q1[t], s1[t]))
            put("QKV", l, t, -1, qkv[t])
            for hh in range(H):
                put("QN", l, t, hh, qn[t, hh])
                put("QR", l, t, hh, qr[t, hh])
                put("QQ", l, t, hh, _qrow(qq[t, hh], qs[t, hh, 0]))
                put("S", l, t, hh, sc[hh, t, :t + 1])
                put("P", l, t, hh, _qrow(pi[hh, t, :t + 1], sp[hh, t, 0]))
                put("O", l, t, hh, o[hh, t])
            for hh in range(Hkv):
                put("KN", l, t, hh, kn[t, hh])
                put("KR", l, t, hh, kr[t, hh])
                put("KQ", l, t, hh, _qrow(kq[t, hh], ks[t, hh, 0]))
                put("VQ", l, t, hh, _qrow(vq[t, hh], vs[t, hh, 0]))
            for op_, row in (("QA2", _qrow(q2[t], s2[t])), ("OP", op[t]), ("R1", r1[t]), ("N2", h2[t]),
                             ("QA3", _qrow(q3[t], s3[t])), ("GU", gu[t]), ("SM", sm[t]),
                             ("QA4", _qrow(q4[t], s4[t])), ("DN", dn[t]), ("R2", r2[t])):
                put(op_, l, t, -1, row)
        for hh in range(Hkv):
            for d in range(hd):
                put("VT", l, d, hh, np.ascontiguousarray(vq[:, hh, d]).astype(np.int32))
            put("VS", l, -1, hh, vs[:, hh, 0])
    return r2.astype(F32)


def layer_rows(m: Model, l: int, x: np.ndarray, rows) -> np.ndarray:
    """layer(m, l, x)[rows] without the other rows' outputs: the keys and values of every position
    (rmsnorm, the k / v columns of the qkv linear, k norm, rope, int8 quant) and everything else for
    the query rows only. Rows are independent in every step but attention (stage.py:146-233), so
    this is the same arithmetic restricted to the rows; for long sequences. Returns (len(rows), D)."""
    cfg = m.cfg
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    T = x.shape[0]
    rows = np.asarray(rows, np.int64)
    nrm, lin = m.norms[l], m.lins[l]
    eps = m.eps32
    Wq, sw = lin["qkv"]
    h1 = det_rmsnorm(x, nrm["in_norm"], eps)
    q1, s1 = quant_act(h1, m.bs(h1.shape[1]))
    kv = slice(H * hd, (H + 2 * Hkv) * hd)
    kvo = dequant(int_gemm(q1, Wq[kv]), s1, sw[kv])                  # (T, 2 Hkv hd)
    k, v = kvo[:, :Hkv * hd], kvo[:, Hkv * hd:]
    qo = dequant(int_gemm(q1[rows], Wq[:H * hd]), s1[rows], sw[:H * hd])  # (R, H hd)
    if cfg["arch"] == 0:
        qn = det_rmsnorm(qo.reshape(len(rows), H, hd), nrm["q_norm"], eps)
        kn = det_rmsnorm(k.reshape(T, Hkv, hd), nrm["k_norm"], eps)
    else:
        qn, kn = qo.reshape(len(rows), H, hd), k.reshape(T, Hkv, hd)
    qr = rope(qn, m.cos[rows][:, None, :], m.sin[rows][:, None, :])
    kr = rope(kn, m.cos[:T][:, None, :], m.sin[:T][:, None, :])
    kq, ks = quant_sym(kr, 127)
    vq, vs = quant_sym(v.reshape(T, Hkv, hd), 127)
    qq, qs = quant_sym(qr, 127)
    *_, o = _attend(qq, qs, kq, ks, vq, vs, inv_sqrt_hd(hd), rows)
    oc = o.transpose(1, 0, 2).reshape(len(rows), H * hd)
    _, _, op = linear(oc, *lin["o"], m.bs(oc.shape[1]))
    r1 = x[rows] + op
    h2 = det_rmsnorm(r1, nrm["post_norm"], eps)
    _, _, gu = linear(h2, *lin["gu"], m.bs(h2.shape[1]))
    I_ = gu.shape[1] // 2
    sm = det_silu(gu[:, :I_]) * gu[:, I_:]
    _, _, dn = linear(sm, *lin["down"], m.bs(sm.shape[1]))
    return (r1 + dn).astype(F32)


def final_logits(m: Model, x: np.ndarray):
    """lm_head(det_rmsnorm(x, norm)) (qwen3.py:300, :306): (int32 accumulators, fp32 logits)."""
    h = det_rmsnorm(x, m.final_norm, m.eps32)
    Wq, sw = m.lm_head
    q, s = quant_act(h, m.bs(h.shape[1]))
    acc = int_gemm(q, Wq)
    return acc.astype(np.int32), dequant(acc, s, sw)


def run_stage(m: Model, tokens, x_in, l0: int, l1: int, keep_rows: bool = True):
    """stage.py:136-234: layers [l0, l1) of one sequence. Returns (leaf rows in program order
    or None, output (T, D))."""
    cfg = m.cfg
    rows: dict = {}
    put = (lambda op, l, t, h, row: rows.__setitem__((op, l, t, h), np.asarray(row))) if keep_rows else None
    if l0 == 0:
        x = m.embed[np.asarray(tokens)].astype(F32)
        if put:
            for t in range(x.shape[0]):
                put("EMBED", 0, t, -1, x[t])
    else:
        x = np.asarray(x_in, F32)
    T = x.shape[0]
    for l in range(l0, l1):
        x = layer(m, l, x, put)
    if not keep_rows:
        return None, x
    leaves = program(cfg["H"], cfg["Hkv"], cfg["hd"], T, l0, l1)
    return [rows[lf] for lf in leaves], x


# ------------------------------------------------------------------ SHA-256 commitments
def _leaf(data: bytes) -> bytes:
    return hashlib.sha256(b"\x00" + data).digest()


def _node(l: bytes, r: bytes) -> bytes:
    return hashlib.sha256(b"\x01" + l + r).digest()


def merkle_root(leaves: list[bytes]) -> bytes:
    """RFC 6962 tree, split at the largest power of two below n (stage.py:42-52)."""
    if not leaves:
        return hashlib.sha256(b"").digest()
    if len(leaves) == 1:
        return leaves[0]
    k = 1
    while k << 1 < len(leaves):
        k <<= 1
    return _node(merkle_root(leaves[:k]), merkle_root(leaves[k:]))


def row_bytes(row: np.ndarray) -> bytes:
    """A leaf row as little-endian 4-byte words (stage.py:63-65)."""
    row = np.asarray(row)
    assert row.dtype in (np.float32, np.int32) and row.ndim == 1, row.dtype
    return row.astype("<f4" if row.dtype == np.float32 else "<i4").tobytes()


def row_root(row: np.ndarray) -> bytes:
    """Merkle root of sha256(0x00 || block) over the row's 1 KiB blocks (stage.py:68-73)."""
    b = row_bytes(row)
    return merkle_root([_leaf(b[i:i + BLOCK]) for i in range(0, max(len(b), 1), BLOCK)])


def tagged_leaf(tag: bytes, index: int, rroot: bytes) -> bytes:
    """sha256(0x00 || tag || u32le index || row_root): "leaf" (trace, stage.py:76-77) or "sout"
    (stage outputs, spec/stage-program.md:82-88)."""
    return _leaf(tag + struct.pack("<I", index) + rroot)


def trace_root(rows: list[np.ndarray]) -> bytes:
    return merkle_root([tagged_leaf(b"leaf", i, row_root(r)) for i, r in enumerate(rows)])


def stage_output_root(out: np.ndarray) -> bytes:
    """StageOutputRoot over the T output rows (spec/stage-program.md:82-88; detgpu/sha.py:1-10)."""
    return merkle_root([tagged_leaf(b"sout", t, row_root(out[t].astype(F32))) for t in range(out.shape[0])])


# ------------------------------------------------------------------ fixtures
def model_from_fixture(d) -> Model:
    """A Model from a tests/golden/stage_*.npz fixture with full weights."""
    D, H, Hkv, hd, I, L, V, eps_bits, Bs, max_pos, arch = (int(v) for v in d["cfg"])
    cfg = dict(D=D, H=H, Hkv=Hkv, hd=hd, I=I, L=L, V=V, eps_bits=eps_bits, Bs=Bs, max_pos=max_pos, arch=arch)
    emb = np.zeros((V, D), F32)
    emb[d["w_embed_rows"]] = d["w_embed"]
    cos = np.zeros((max_pos, hd), F32)
    sin = np.zeros((max_pos, hd), F32)
    cos[d["w_rope_cos_rows"]] = d["w_rope_cos"]
    sin[d["w_rope_sin_rows"]] = d["w_rope_sin"]
    norms, lins = [], []
    for l in range(L):
        key = f"w_in_norm_{l}"
        if key not in d:
            break
        norms.append({nm: d[f"w_{nm}_{l}"] for nm in ("in_norm", "post_norm", "q_norm", "k_norm")})
        ls = {}
        for lin in ("qkv", "o", "gu", "down"):
            p = f"w_{lin}_{l}"
            ls[lin] = (d[p + "_q"], d[p + "_s"])
        lins.append(ls)
    return Model(cfg, emb, norms, lins, cos, sin)


def fixture_rows(d, si: int) -> list[np.ndarray]:
    """The u32 rows of stage si (program order)."""
    w, off = d[f"s{si}_words"], d[f"s{si}_offs"]
    return [w[off[i]:off[i + 1]] for i in range(len(off) - 1)]
