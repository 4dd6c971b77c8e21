"""detrt's deterministic decoder layer and stage commitments on MI355X: the call surface of the
reference's GPU engine runtime/detgpu (kernels.py, sha.py, stages.py), over libuwc_hip.so.

Bit-identical to the CPU reference runtime/detrt: every fp32 step is one correctly rounded IEEE
op in detrt's order, every sum is exact (int32 / int64 / fixed point), and max is exact, so no
batching, tiling or key split changes a bit.

  kernels   quant_act, rmsnorm_quant, rmsnorm, qkv_post, attention, dequant_residual,
            swiglu_quant, embed                     (runtime/detgpu/kernels.py:699-826)
  sha       sout_leaves, stage_roots_gpu, digest_bytes, stage_output_roots, row_roots,
            trace_root                              (runtime/detgpu/sha.py:139-236)
  stages    layer_fused, stage_outputs, job_outputs, final_logits
                                                    (runtime/detgpu/stages.py:154-219)
  DetModel  the attributes of detrt.qwen3.DetQwen3 that the stages read (qwen3.py:165-199),
            built from quantized weight tables or from a seeded random init.

Everything runs on torch's current HIP stream; buffers are torch tensors on the caller's GPU.
"""
from __future__ import annotations

import hashlib

import numpy as np
import torch

from . import _lib
from .detrt import DetLinear, hadamard_bs
from .detrt import quant_act as _quant_act

F32 = torch.float32
TAG_LEAF = int.from_bytes(b"leaf", "big")
TAG_SOUT = int.from_bytes(b"sout", "big")
BLOCK = 1024  # bytes per committed row block (runtime/detrt/stage.py:25)


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _f32(v: float) -> float:
    """A Python float rounded once to float32 (detrt's c32)."""
    return float(np.float32(v))


def _inv(k: int) -> float:
    return float(np.float32(1.0 / k))


# ================================================================== kernels
def quant_act(x: torch.Tensor, bs: int) -> tuple[torch.Tensor, torch.Tensor]:
    """detrt.core.quant_act(x, bs) for float32 x (rows, k): (int8 q, float32 scale)."""
    return _quant_act(x, bs)


def rmsnorm_quant(x: torch.Tensor, w: torch.Tensor, eps: float, bs: int) -> tuple[torch.Tensor, torch.Tensor]:
    """quant_act(det_rmsnorm(x, w, eps), bs) for float32 x (rows, k) (detgpu/kernels.py:712-728)."""
    x = x.contiguous()
    rows, k = x.shape
    if x.dtype != F32 or w.dtype != F32 or (bs > 1 and k % bs):
        raise AssertionError("rmsnorm_quant: float32 x and w, bs dividing k")
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=F32, device=x.device)
    _lib.call("uwc_rmsnorm_quant_f32", x.data_ptr(), w.contiguous().data_ptr(), rows, k, bs, _inv(k), _f32(eps),
              q.data_ptr(), s.data_ptr(), _stream())
    return q, s


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """detrt.core.det_rmsnorm along the last dim of float32 x."""
    shp = x.shape
    x2 = x.reshape(-1, shp[-1]).contiguous()
    rows, k = x2.shape
    y = torch.empty_like(x2)
    _lib.call("uwc_rmsnorm_f32", x2.data_ptr(), w.contiguous().data_ptr(), rows, k, _inv(k), _f32(eps), y.data_ptr(),
              _stream())
    return y.reshape(shp)


def vt_tokens(T: int) -> int:
    return _lib.lib().uwc_vt_tokens(T)


def qkv_post_vt(acc, s1, sw, qnw, knw, cos, sin, T: int, H: int, Hkv: int, eps: float, qknorm: bool = True):
    """qkv_post plus V transposed for attention(): (qq, qs, kq, ks, vq, vs, vt). acc is the int32
    GEMM output (with s1, sw), or already dequantized float32 rows (s1 = sw = None)."""
    acc = acc.contiguous()
    N = acc.shape[0]
    hd = acc.shape[1] // (H + 2 * Hkv)
    fp = acc.dtype == F32
    if (acc.dtype != torch.int32 and not fp) or acc.shape[1] != (H + 2 * Hkv) * hd or N % T:
        raise AssertionError(f"qkv_post: acc must be int32 or float32 (B*T, (H + 2 Hkv) hd), got {tuple(acc.shape)}")
    if fp != (s1 is None) or (s1 is None) != (sw is None):
        raise AssertionError("qkv_post: int32 acc needs s1 and sw; float32 rows take neither")
    B = N // T
    dev = acc.device
    e = lambda *shape, dt=torch.int8: torch.empty(shape, dtype=dt, device=dev)
    qq, qs, kq, ks, vq, vs = e(N, H, hd), e(N, H, 1, dt=F32), e(N, Hkv, hd), e(N, Hkv, 1, dt=F32), e(N, Hkv, hd), e(N, Hkv, 1, dt=F32)
    # qkv_post writes every key below T; the pad keys T .. Tp - 1 (their positions are spread over
    # the last 64-key tile, which vt_pos permutes) only meet zero probabilities in attention, and
    # that tile is zeroed first so that vt is defined everywhere
    vt = torch.empty((B, Hkv, hd, vt_tokens(T)), dtype=torch.int8, device=dev)
    if T % 64:
        vt[..., T // 64 * 64:].zero_()
    qn = qnw.contiguous() if qknorm else None
    kn = knw.contiguous() if qknorm else None
    cos, sin = cos.contiguous(), sin.contiguous()
    if cos.shape[0] < T or cos.shape[1] != hd:
        raise AssertionError("qkv_post: the rope tables need T rows of head_dim")
    _lib.call("uwc_qkv_post", acc.data_ptr(), None if fp else s1.contiguous().data_ptr(),
              None if fp else sw.contiguous().data_ptr(),
              qn.data_ptr() if qn is not None else None, kn.data_ptr() if kn is not None else None,
              cos.data_ptr(), sin.data_ptr(), B, T, H, Hkv, hd, _f32(eps), int(bool(qknorm)),
              qq.data_ptr(), qs.data_ptr(), kq.data_ptr(), ks.data_ptr(), vq.data_ptr(), vs.data_ptr(), vt.data_ptr(),
              _stream())
    return qq, qs, kq, ks, vq, vs, vt


def qkv_post(acc, s1, sw, qnw, knw, cos, sin, T: int, H: int, Hkv: int, eps: float, qknorm: bool = True):
    """Quantized q, k, v from the qkv GEMM's int32 output: (qq (N,H,hd) int8, qs (N,H,1), kq, ks,
    vq, vs) (detgpu/kernels.py:788-802). qknorm False (Llama, Mistral): no per-head RMSNorm."""
    return qkv_post_vt(acc, s1, sw, qnw, knw, cos, sin, T, H, Hkv, eps, qknorm)[:6]


# The exponentials scratch of the stored-exp attention is allocated per call from torch's caching
# allocator on the current stream: stream-ordered (two calls on two streams never share it, and a
# buffer freed after a call is reused only by work queued after that call) and, after the first
# call of a size, without a device allocation. Calls whose scratch would exceed ATTN_SCRATCH_MAX
# bytes recompute the exponentials instead.
ATTN_SCRATCH_MAX = 16 << 30


def attention(qq, qs, kq, ks, vq, vs, B: int, T: int, H: int, Hkv: int, inv_sqrt_hd_f32: float, vt=None,
              stored_exp=None):
    """detrt's attention from quantized q, k, v: qq (N, H, hd), kq and vq (N, Hkv, hd) int8, qs
    (N, H, 1), ks and vs (N, Hkv, 1). Returns o as (N, H*hd) float32 (detgpu/kernels.py:731-770).
    vt (from qkv_post_vt) skips the transpose of vq. stored_exp: keep the softmax exponentials in
    a device scratch between the kernel's passes (uwc_attention_ws) instead of recomputing them;
    None takes it when the scratch is at most ATTN_SCRATCH_MAX bytes. Either way the same bits."""
    N, _, hd = qq.shape
    if N != B * T or kq.shape != (N, Hkv, hd) or vq.shape != (N, Hkv, hd):
        raise AssertionError("attention: shapes (B*T, H, hd) / (B*T, Hkv, hd)")
    i8 = lambda z: z.to(torch.int8).contiguous()
    f = lambda z: z.contiguous().to(F32)
    qq, kq, vq = i8(qq), i8(kq), i8(vq)
    qs, ks, vs = f(qs), f(ks), f(vs)
    if vt is None:
        vt = torch.zeros((B, Hkv, hd, vt_tokens(T)), dtype=torch.int8, device=qq.device)
        _lib.call("uwc_v_transpose", vq.data_ptr(), B, T, Hkv, hd, vt.data_ptr(), _stream())
    o = torch.empty((N, H * hd), dtype=F32, device=qq.device)
    nbytes = int(_lib.lib().uwc_attention_scratch_bytes(B, T, H))
    if stored_exp is None:
        stored_exp = 0 < nbytes <= ATTN_SCRATCH_MAX
    args = (qq.data_ptr(), qs.data_ptr(), kq.data_ptr(), ks.data_ptr(), vt.data_ptr(), vs.data_ptr(), B, T, H, Hkv,
            hd, float(np.float32(inv_sqrt_hd_f32)), o.data_ptr())
    if stored_exp and nbytes > 0:
        es = torch.empty((nbytes + 3) // 4, dtype=F32, device=qq.device)
        _lib.call("uwc_attention_ws", *args, es.data_ptr(), es.numel() * 4, _stream())
    else:
        _lib.call("uwc_attention", *args, _stream())
    return o


def _scales(acc, *scales):
    fp = acc.dtype == F32
    if fp != all(s is None for s in scales) or any(s is None for s in scales) != fp:
        raise AssertionError("int32 accumulators need their scales; float32 rows take none")
    return [None if fp else s.contiguous().data_ptr() for s in scales]


def dequant_residual(acc, s, sw, x, out=None):
    """x + fmul(fmul(f32(acc), s), sw) (detgpu/kernels.py:805-813); x + acc for float32 acc (s = sw = None).
    out: an optional contiguous (N, k) float32 destination that does not overlap x or acc."""
    acc, x = acc.contiguous(), x.contiguous()
    N, k = acc.shape
    if out is None:
        out = torch.empty((N, k), dtype=F32, device=acc.device)
    elif out.shape != (N, k) or out.dtype != F32 or not out.is_contiguous():
        raise AssertionError(f"dequant_residual: out must be a contiguous float32 {N} x {k} tensor")
    ps, psw = _scales(acc, s, sw)
    _lib.call("uwc_dequant_residual", acc.data_ptr(), ps, psw, x.data_ptr(), N, k, out.data_ptr(), _stream())
    return out


def linear_residual(lin, q, s, x, out=None):
    """x + fmul(fmul(f32(q @ lin.Wq^T), s), lin.sw): a DetLinear's exact GEMM on pre-quantized rows
    q (N, k) with the dequant and the residual x (N, n) added in one call
    (uwc_igemm_dequant_residual_f32: in the GEMM's epilogue where its 256 x 256 tiles take the
    shape), the same bits as dequant_residual(lin.int_gemm(q), s, lin.sw, x). out: an optional
    contiguous (N, n) float32 destination that does not overlap x."""
    if lin.mine and lin.mw is not None:
        return dequant_residual(lin.int_gemm(q), s, lin.sw, x, out=out)
    q, x = q.contiguous(), x.contiguous()
    N = q.shape[0]
    if out is None:
        out = torch.empty((N, lin.n), dtype=F32, device=q.device)
    elif out.shape != (N, lin.n) or out.dtype != F32 or not out.is_contiguous():
        raise AssertionError(f"linear_residual: out must be a contiguous float32 {N} x {lin.n} tensor")
    if x.shape != (N, lin.n) or x.dtype != F32:
        raise AssertionError(f"linear_residual: x must be float32 {N} x {lin.n}")
    _lib.call("uwc_igemm_dequant_residual_f32", q.data_ptr(), lin.Wq.data_ptr(), N, lin.n, lin.k, s.data_ptr(),
              lin.sw.data_ptr(), x.data_ptr(), out.data_ptr(), _stream())
    return out


def swiglu_quant(acc, s3, sw, bs: int):
    """quant_act(silu(g) * u, bs) from the gate_up GEMM's int32 rows (detgpu/kernels.py:816-826),
    or from float32 GU rows (s3 = sw = None)."""
    acc = acc.contiguous()
    N, two_i = acc.shape
    I = two_i // 2
    if bs > 1 and I % bs:
        raise AssertionError("swiglu_quant: bs must divide I")
    q = torch.empty((N, I), dtype=torch.int8, device=acc.device)
    sc = torch.empty(N, dtype=F32, device=acc.device)
    ps3, psw = _scales(acc, s3, sw)
    _lib.call("uwc_swiglu_quant", acc.data_ptr(), ps3, psw, N, I, bs, q.data_ptr(), sc.data_ptr(), _stream())
    return q, sc


def embed(table: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """table[ids] for float32 table (V, D); ids outside [0, V) raise (checked on the host)."""
    ids64 = ids.reshape(-1).to(device=table.device, dtype=torch.int64).contiguous()
    V, D = table.shape
    if ids64.numel() and (int(ids64.min()) < 0 or int(ids64.max()) >= V):
        raise IndexError(f"embed: token id outside [0, {V})")
    out = torch.empty((ids64.numel(), D), dtype=F32, device=table.device)
    _lib.call("uwc_embed_rows", table.contiguous().data_ptr(), V, D, ids64.data_ptr(), ids64.numel(), out.data_ptr(),
              None, _stream())
    return out


OPS = {"add": 0, "sub": 1, "mul": 2, "div": 3, "sqrt": 4, "exp": 5, "silu": 6}


def elementwise(op: str, x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    """One of detrt's fp32 ops (fadd, fsub, fmul, fdiv, fsqrt, det_exp, det_silu) elementwise, as the
    layer kernels compute it (the native-fp32 check of runtime/tests/test_fp32_native.py)."""
    x = x.contiguous().to(F32)
    y = y.contiguous().to(F32) if y is not None else None
    out = torch.empty_like(x)
    _lib.call("uwc_det_elementwise", OPS[op], x.data_ptr(), y.data_ptr() if y is not None else None, out.data_ptr(),
              x.numel(), _stream())
    return out


# ================================================================== sha
def _row_leaf_words(rows: torch.Tensor, tag: int, base: int, mod: int, want_roots: bool = False):
    """(n, 8) int32 tagged leaves (and row roots) of the rows of a 2-D float32 / int32 tensor."""
    rows = rows.contiguous()
    n, w = rows.shape
    nblk = max(1, -(-w // (BLOCK // 4)))
    scratch = torch.empty(n * nblk * 8, dtype=torch.int32, device=rows.device)
    leaves = torch.empty((n, 8), dtype=torch.int32, device=rows.device)
    roots = torch.empty((n, 8), dtype=torch.int32, device=rows.device) if want_roots else None
    _lib.call("uwc_sha_row_leaves", rows.data_ptr() if rows.numel() else None, n, w, scratch.data_ptr(),
              scratch.numel(), tag, base, mod, roots.data_ptr() if roots is not None else None, leaves.data_ptr(),
              _stream())
    return (leaves, roots) if want_roots else leaves


def _leaf_words(out: torch.Tensor) -> torch.Tensor:
    """(B * T, 8) int32: the stage-output leaves H(0x00 || "sout" || u32 t || row_root) as words."""
    B, T, D = out.shape
    return _row_leaf_words(out.reshape(B * T, D).to(F32), TAG_SOUT, 0, T)


def merkle_roots(words: torch.Tensor, ntrees: int) -> torch.Tensor:
    """(ntrees, 8) roots of ntrees consecutive trees of equal size over (ntrees * n, 8) leaf words."""
    n = words.shape[0] // ntrees
    scratch = torch.empty(2 * words.numel(), dtype=torch.int32, device=words.device)
    roots = torch.empty((ntrees, 8), dtype=torch.int32, device=words.device)
    _lib.call("uwc_sha_merkle_roots", words.contiguous().data_ptr(), ntrees, n, scratch.data_ptr(), scratch.numel(),
              roots.data_ptr(), _stream())
    return roots


# sha256(cos bytes || sin bytes) of detrt's pinned fp32 rope tables (runtime/artifacts/*.npz, built
# by qwen3.py:49-68; the Qwen3-1.7B one is also recorded as rope_table_sha in
# results/step2/xdev_cpu.json:4): (theta, head_dim, positions) -> digest.
PINNED_ROPE_SHA = {
    (1e6, 128, 8192): "8ee66518240c0e045455c4ff8fb6cf1d959e22872c1e0dbba4bbc18985d3df26",
    (1e4, 64, 8192): "bfd2634ada10ea33214570446397a3749cf48de85eac0a0fba1531f18abaa79a",
    (1e4, 32, 64): "2ff462ac8583a2f5ef106fc4a9823cb845ece1243d83d73b5565c53ffee34bc7",
}


def rope_table(theta: float, head_dim: int, max_pos: int) -> tuple[np.ndarray, np.ndarray]:
    """detrt's fp32 rope tables (max_pos x head_dim): angle(p, i) = p / theta^(2 (i mod hd/2) / hd)
    in float64, cos and sin in float64 rounded once to float32 (qwen3.py:59-66). The reference
    loads them from pinned files; here they are computed on the host, and a table with a pinned
    digest is checked against it, so a host whose libm rounds differently fails loudly instead of
    silently changing every rotated query and key."""
    half = np.arange(0, head_dim, 2, dtype=np.float64) / head_dim
    freq = 1.0 / np.power(float(theta), half)
    ang = np.outer(np.arange(max_pos, dtype=np.float64), np.tile(freq, 2))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    want = PINNED_ROPE_SHA.get((float(theta), int(head_dim), int(max_pos)))
    if want is not None:
        got = hashlib.sha256(cos.tobytes() + sin.tobytes()).hexdigest()
        if got != want:
            raise RuntimeError(f"rope_table(theta={theta:g}, hd={head_dim}, pos={max_pos}): this host's table hashes to "
                               f"{got[:16]}..., not detrt's pinned {want[:16]}...")
    return cos, sin


def digest_bytes(words) -> np.ndarray:
    """SHA-256 digests as bytes: (..., 8) state words, torch or numpy, to (..., 32) uint8. A digest
    is its state words in big-endian byte order (FIPS 180-4)."""
    host = words.detach().to("cpu").numpy() if isinstance(words, torch.Tensor) else np.asarray(words)
    be = np.ascontiguousarray(host).astype(">u4", copy=False)
    return be.view(np.uint8).reshape(host.shape[:-1] + (32,))


def sout_leaves(out: torch.Tensor) -> np.ndarray:
    """Stage-output leaves of B stages: out (B, T, D) float32 on the GPU -> (B, T, 32) uint8 on the CPU."""
    B, T, _ = out.shape
    return digest_bytes(_leaf_words(out)).reshape(B, T, 32)


def stage_roots_gpu(out: torch.Tensor) -> torch.Tensor:
    """stage_output_root of each of the B stages in out (B, T, D), on the GPU: (B, 8) int32 words."""
    B = out.shape[0]
    return merkle_roots(_leaf_words(out), B)


def stage_output_roots(out: torch.Tensor) -> list[bytes]:
    """agent.proto.stage_output_root for each of the B stages in out (B, T, D)."""
    return [bytes(r) for r in digest_bytes(stage_roots_gpu(out))]


def row_roots(rows: torch.Tensor) -> torch.Tensor:
    """(n, 8) int32 row roots of the rows of a 2-D float32 / int32 tensor."""
    return _row_leaf_words(rows, TAG_LEAF, 0, 0, want_roots=True)[1]


def trace_root(rows: list[torch.Tensor]) -> bytes:
    """Stage trace root over leaf rows in program order (stage.py:120-133), hashed on the GPU:
    rows of equal length are hashed together; leaf i = H(0x00 || "leaf" || u32 i || row_root)."""
    dev = rows[0].device
    n = len(rows)
    leaves = torch.empty((n, 8), dtype=torch.int32, device=dev)
    by_len: dict = {}
    for i, r in enumerate(rows):
        by_len.setdefault(int(r.numel()), []).append(i)
    for w, idx in by_len.items():
        mat = torch.stack([rows[i].reshape(-1).view(torch.int32) for i in idx]) if w else \
            torch.empty((len(idx), 0), dtype=torch.int32, device=dev)
        idx_t = torch.tensor(idx, dtype=torch.int64, device=dev)
        # one call per run of consecutive indices, so that the leaf index is base + row
        runs, start = [], 0
        for j in range(1, len(idx) + 1):
            if j == len(idx) or idx[j] != idx[j - 1] + 1:
                runs.append((start, j))
                start = j
        for a, b in runs:
            leaves[idx_t[a:b]] = _row_leaf_words(mat[a:b], TAG_LEAF, idx[a], 0)
    return bytes(digest_bytes(merkle_roots(leaves, 1))[0])


# ================================================================== model and stages
class DetModel:
    """What detgpu's stages read from detrt.qwen3.DetQwen3 (qwen3.py:165-199): D, H, Hkv, hd, eps,
    qk_norm, inv_sqrt_hd, embed, cos, sin, layers[l] = dict(in_norm, post_norm, q_norm, k_norm,
    qkv, o, gu, down (DetLinear), dev, cos, sin), norm and lm_head. Weights are already quantized
    (int8 rows with their fp32 scales, as committed in the weights tree, stage.py:239-264)."""

    def __init__(self, cfg: dict, embed: torch.Tensor, layers: list[dict], cos: torch.Tensor, sin: torch.Tensor,
                 norm: torch.Tensor | None = None, lm_head: DetLinear | None = None):
        self.D, self.H, self.Hkv, self.hd = cfg["D"], cfg["H"], cfg["Hkv"], cfg["hd"]
        self.eps = float(np.array([cfg["eps_bits"]], np.uint32).view(np.float32)[0]) if "eps_bits" in cfg \
            else _f32(cfg["eps"])
        self.arch = cfg.get("arch", 0)
        self.qk_norm = self.arch == 0
        self.hadamard_block = cfg["Bs"]
        self.inv_sqrt_hd = float(np.float32(1.0 / np.sqrt(self.hd)))
        self.embed, self.cos, self.sin = embed, cos, sin
        self.device = embed.device
        self.layers = layers
        for L in layers:
            L.setdefault("dev", self.device)
            L.setdefault("cos", cos)
            L.setdefault("sin", sin)
        self.norm, self.lm_head = norm, lm_head

    def enter(self, dev):
        return dev

    @classmethod
    def from_tables(cls, cfg: dict, embed, norms: list[dict], lins: list[dict], cos, sin, device="cuda",
                    norm=None, lm_head=None) -> "DetModel":
        """From numpy tables: norms[l] = {in_norm, post_norm, q_norm, k_norm}, lins[l][name] = (Wq, sw)."""
        t = lambda a, dt=F32: torch.as_tensor(np.ascontiguousarray(a)).to(device=device, dtype=dt)
        layers = []
        for nrm, ls in zip(norms, lins):
            L = {nm: t(nrm[nm]) for nm in ("in_norm", "post_norm", "q_norm", "k_norm")}
            for name in ("qkv", "o", "gu", "down"):
                Wq, sw = ls[name]
                L[name] = DetLinear.from_quantized(t(Wq, torch.int8), t(sw), hadamard_bs(cfg["Bs"], Wq.shape[1]))
            layers.append(L)
        lm = None
        if lm_head is not None:
            lm = DetLinear.from_quantized(t(lm_head[0], torch.int8), t(lm_head[1]), hadamard_bs(cfg["Bs"], lm_head[0].shape[1]))
        return cls(cfg, t(embed), layers, t(cos), t(sin), t(norm) if norm is not None else None, lm)

    @classmethod
    def random(cls, cfg: dict, seed: int = 0, device="cuda", with_lm_head: bool = True) -> "DetModel":
        """A model of cfg's shape with seeded random weights, quantized on the GPU as DetLinear does
        (Wq = quant_sym(fwht(W, bs), 64) per row, N(0, 0.02) weights), N(0, 1) embedding rows,
        norm weights near 1, and the rope table of theta 1e6 built in float64 (qwen3.py:47-66)."""
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        D, H, Hkv, hd, I, V = cfg["D"], cfg["H"], cfg["Hkv"], cfg["hd"], cfg["I"], cfg["V"]
        bs = cfg["Bs"]

        def lin(n, k):
            W = torch.randn((n, k), generator=g, device=device) * 0.02
            q, s = _quant_act(W, hadamard_bs(bs, k))
            del W
            return DetLinear.from_quantized(q, s, hadamard_bs(bs, k))

        def nw(k):
            return 1.0 + 0.05 * torch.randn(k, generator=g, device=device)
        layers = []
        for _ in range(cfg["L"]):
            layers.append(dict(in_norm=nw(D), post_norm=nw(D), q_norm=nw(hd), k_norm=nw(hd),
                               qkv=lin((H + 2 * Hkv) * hd, D), o=lin(D, H * hd), gu=lin(2 * I, D), down=lin(D, I)))
        embed_t = torch.randn((V, D), generator=g, device=device)
        cos_np, sin_np = rope_table(cfg.get("theta", 1e6), hd, cfg.get("max_pos", 8192))
        cos, sin = torch.from_numpy(cos_np).to(device), torch.from_numpy(sin_np).to(device)
        lm = lin(V, D) if with_lm_head else None
        return cls(cfg, embed_t, layers, cos, sin, nw(D), lm)


def layer_fused(m, L, x: torch.Tensor, B: int, T: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """One decoder layer: x (N, D) float32 -> (N, D) float32, bit-identical to detrt
    (detgpu/stages.py:154-168); out: optional (N, D) float32 destination, not overlapping x."""
    H, Hkv = m.H, m.Hkv
    q1, s1 = rmsnorm_quant(x, L["in_norm"], m.eps, L["qkv"].bs)
    qq, qs, kq, ks, vq, vs, vt = qkv_post_vt(L["qkv"].int_gemm(q1), s1, L["qkv"].sw, L["q_norm"], L["k_norm"],
                                             L["cos"][:T], L["sin"][:T], T, H, Hkv, m.eps, m.qk_norm)
    oc = attention(qq, qs, kq, ks, vq, vs, B, T, H, Hkv, m.inv_sqrt_hd, vt=vt)
    q2, s2 = quant_act(oc, L["o"].bs)
    r1 = linear_residual(L["o"], q2, s2, x)
    q3, s3 = rmsnorm_quant(r1, L["post_norm"], m.eps, L["gu"].bs)
    q4, s4 = swiglu_quant(L["gu"].int_gemm(q3), s3, L["gu"].sw, L["down"].bs)
    return linear_residual(L["down"], q4, s4, r1, out=out)


@torch.no_grad()
def stage_outputs(m, tokens: torch.Tensor | None, x: torch.Tensor | None, l0: int, l1: int) -> torch.Tensor:
    """Layers l0..l1-1 for B sequences of T tokens: tokens (B, T) int64 when l0 == 0, else x
    (B, T, D) float32, the previous group's output. Returns (B, T, D) float32 on the GPU
    (detgpu/stages.py:172-214)."""
    if l0 == 0:
        B, T = tokens.shape
        x = embed(m.embed, tokens)
    else:
        B, T = x.shape[0], x.shape[1]
        x = x.to(m.device, F32).reshape(B * T, m.D)
    for l in range(l0, l1):
        x = layer_fused(m, m.layers[l], x, B, T)
    return x.reshape(B, T, m.D)


@torch.no_grad()
def forward_stage_roots(m, tokens: torch.Tensor, outs: torch.Tensor | None = None):
    """Every layer of one sequence (tokens (1, T)) with every layer's stage-output root: the layer
    outputs land in one (L, T, D) float32 buffer (outs, or a new one), and all L roots are then
    hashed by one batched set of launches, as stage_roots_gpu over L stages. Per layer, the 1 KiB
    SHA-256 chains of a stage output (8 per 8 KiB row: 65,536 at T = 8192) give every SIMD one
    wave, whose dependent rounds leave the VALU mostly idle; the L layers together give each SIMD
    L waves. Returns (the last layer's output (T, D), roots (L, 8) int32 words), the same roots as
    stage_roots_gpu of each layer's output."""
    B, T = tokens.shape
    if B != 1:
        raise AssertionError("forward_stage_roots: one sequence")
    nl = len(m.layers)
    if outs is None:
        outs = torch.empty((nl, T, m.D), dtype=F32, device=m.device)
    elif outs.shape != (nl, T, m.D) or outs.dtype != F32 or not outs.is_contiguous():
        raise AssertionError(f"forward_stage_roots: outs must be a contiguous float32 ({nl}, {T}, {m.D}) tensor")
    x = embed(m.embed, tokens)
    for l, L in enumerate(m.layers):
        x = layer_fused(m, L, x, 1, T, out=outs[l])
    return x, stage_roots_gpu(outs)


def job_outputs(m, tokens: torch.Tensor, groups: int, upto: int | None = None) -> list[torch.Tensor]:
    """The outputs of layer groups 0 .. upto (default: all) for a batch of sequences, each (B, T, D)
    on the GPU: the layers split into `groups` equal runs, each run continuing from the previous
    run's output (detgpu/stages.py:216-225)."""
    per = len(m.layers) // groups
    last = groups - 1 if upto is None else upto
    bounds = [(g * per, (g + 1) * per) for g in range(last + 1)]
    outs = []
    for l0, l1 in bounds:
        prev = outs[-1] if outs else None
        outs.append(stage_outputs(m, tokens if prev is None else None, prev, l0, l1))
    return outs


@torch.no_grad()
def final_logits(m, x: torch.Tensor):
    """lm_head(det_rmsnorm(x, norm)) for hidden rows x (N, D): (int32 logits accumulators, fp32
    logits), the rows DetQwen3.logprobs starts from (qwen3.py:300-311)."""
    q, s = rmsnorm_quant(x.reshape(-1, m.D), m.norm, m.eps, m.lm_head.bs)
    acc = m.lm_head.int_gemm(q)
    from .detrt import dequant
    return acc, dequant(acc, s, m.lm_head.sw)
