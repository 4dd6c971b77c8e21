"""GPU parity of the decoder-layer ops and stage commitments (uwc_amd.detgpu over libuwc_hip.so)
against the CPU oracle (oracle/detrt_stage.py) and the reference's referee fixtures, bit for bit.

  * every kernel vs the oracle on seeded inputs, including ragged sizes, zero and tiny rows;
  * whole stages of the tiny Qwen3 / Llama fixtures (12 tokens, both layers) through
    stage_outputs: the GPU's R2 rows and every leaf the fused kernels expose (QA1, QQ, KQ, VQ,
    O, QA2, R1, QA3, QA4) equal the committed rows;
  * the real Qwen3-1.7B fixture rows (hd 128): qkv_post, attention, dequant_residual,
    rmsnorm_quant and swiglu_quant from the fixture's own inputs;
  * SHA-256: row roots and stage-output roots vs hashlib, and the stage trace roots of the
    fixtures recomputed on the GPU from the committed rows.
"""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import detrt_stage as S

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _u32(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a).view(np.uint32)


def _t(a, dev, dt=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return t if dt is None else t.to(dt)


def _rows(rng, n, k, scale=1.0):
    x = (rng.standard_normal((n, k)) * scale).astype(np.float32)
    if n > 3:
        x[0] = 0
        x[1] *= np.float32(1e-30)       # subnormal squares
        x[2, ::7] = np.float32(3e4)     # large
    return x


def _fp32_sweep(rng, n):
    """Random bit patterns over every exponent (incl. subnormals), plus specials."""
    bits = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32).copy()
    x[~np.isfinite(x)] = np.float32(1.5)
    special = np.array([0.0, -0.0, 1.0, -1.0, 2.0, 0.5, 3.0, 1e-45, -1e-45, 1.17549435e-38, 3.4028235e38, -3.4028235e38,
                        np.inf, -np.inf, 64.0, 128.0, 512.0, 2048.0, 1e-6, 1e-5, -87.0, -88.5, -103.9, 88.7, 89.0],
                       np.float32)
    return np.concatenate([special, x, rng.standard_normal(n).astype(np.float32) * np.float32(30)])


def test_fp32_ops_match_ieee_and_detrt(dev):
    """Each elementwise op the kernels use, on bit patterns across every exponent, equals numpy's
    IEEE float32 op (add, sub, mul, div, sqrt) or the oracle's det_exp / det_silu bit for bit."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(2026)
    x = _fp32_sweep(rng, 200_000)
    y = _fp32_sweep(rng, 200_000)[::-1].copy()
    z = np.concatenate([x, rng.uniform(-110, 110, 200_000).astype(np.float32)])
    xt, yt, zt = _t(x, dev), _t(y, dev), _t(z, dev)
    with np.errstate(all="ignore"):
        ref = {"add": x + y, "sub": x - y, "mul": x * y, "div": x / y, "sqrt": np.sqrt(np.abs(x)),
               "exp": S.det_exp(z), "silu": S.det_silu(z)}
    args = {"sqrt": (_t(np.abs(x), dev),), "exp": (zt,), "silu": (zt,)}
    for op, r in ref.items():
        got = detgpu.elementwise(op, *args.get(op, (xt, yt))).cpu().numpy()
        same = (_u32(got) == _u32(r)) | (np.isnan(got) & np.isnan(r))
        assert same.all(), (op, np.nonzero(~same)[0][:5], got[~same][:3], r[~same][:3])


@pytest.mark.parametrize("k,bs", [(128, 64), (2048, 512), (6144, 512), (1024, 64), (512, 1), (1536, 0), (1000, 8), (96, 0),
                                  (4096, 128), (2560, 256), (3584, 32), (2048, 2)])
def test_rmsnorm_quant_and_rmsnorm(dev, k, bs):
    """k = 512 G up to 4096 run on the one-wave-per-row kernel (every G from 1 to 8 at some bs),
    the rest on the LDS row kernel."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(k + bs)
    x = _rows(rng, 37, k)
    w = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    eps = np.float32(1e-6)
    ref_h = S.det_rmsnorm(x, w, eps)
    ref_q, ref_s = S.quant_act(ref_h, bs)
    q, s = detgpu.rmsnorm_quant(_t(x, dev), _t(w, dev), float(eps), bs)
    assert np.array_equal(q.cpu().numpy(), ref_q)
    assert np.array_equal(_u32(s), _u32(ref_s))
    y = detgpu.rmsnorm(_t(x, dev), _t(w, dev), float(eps))
    assert np.array_equal(_u32(y), _u32(ref_h))


@pytest.mark.parametrize("I,bs", [(256, 64), (6144, 512), (1024, 8), (512, 2), (300, 4), (2560, 128), (3584, 256),
                                  (5632, 512), (4096, 1)])
def test_swiglu_quant(dev, I, bs):
    """I = 512 G up to 6144 run on the one-wave-per-row kernel, the rest on the LDS row kernel."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(I)
    n = 19
    acc = rng.integers(-3_000_000, 3_000_000, (n, 2 * I)).astype(np.int32)
    acc[0] = 0
    s3 = rng.uniform(1e-6, 1e-4, n).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-2, 2 * I).astype(np.float32)
    gu = S.dequant(acc, s3, sw)
    sm = S.det_silu(gu[:, :I]) * gu[:, I:]
    ref_q, ref_s = S.quant_act(sm, bs)
    q, s = detgpu.swiglu_quant(_t(acc, dev), _t(s3, dev), _t(sw, dev), bs)
    assert np.array_equal(q.cpu().numpy(), ref_q)
    assert np.array_equal(_u32(s), _u32(ref_s))


def test_dequant_residual_and_embed(dev):
    from uwc_amd import detgpu
    rng = np.random.default_rng(3)
    acc = rng.integers(-2**31, 2**31 - 1, (33, 257), dtype=np.int64).astype(np.int32)
    s = rng.uniform(1e-9, 1e-3, 33).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-1, 257).astype(np.float32)
    x = rng.standard_normal((33, 257)).astype(np.float32)
    out = detgpu.dequant_residual(_t(acc, dev), _t(s, dev), _t(sw, dev), _t(x, dev))
    assert np.array_equal(_u32(out), _u32(x + S.dequant(acc, s, sw)))
    table = rng.standard_normal((50, 24)).astype(np.float32)
    ids = np.array([[3, 0, 49, 7], [7, 7, 1, 2]], np.int64)
    e = detgpu.embed(_t(table, dev), _t(ids, dev))
    assert np.array_equal(_u32(e), _u32(table[ids.ravel()]))
    with pytest.raises(IndexError):
        detgpu.embed(_t(table, dev), _t(np.array([50]), dev))


@pytest.mark.parametrize("m,n,k", [(8192, 2048, 256), (8192, 2048, 2048), (2048, 2048, 512), (384, 256, 128)])
def test_linear_residual_fused(dev, m, n, k):
    """uwc_igemm_dequant_residual_f32 (the 256 x 256 GEMM with the dequant and the residual add in
    its epilogue where its tiles fill the CUs, 8192 x 2048; else the dequantized product and the
    residual pass) equals dequant_residual of the int32 product bit for bit, and the oracle on
    sampled rows."""
    from uwc_amd import detgpu, detrt, ops
    g = torch.Generator(device=dev)
    g.manual_seed(m + n + k)
    q = torch.randint(-127, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    W = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    s = torch.rand(m, device=dev, generator=g) * 1e-3 + 1e-6
    sw = torch.rand(n, device=dev, generator=g) * 1e-2 + 1e-6
    x = torch.randn((m, n), device=dev, generator=g)
    lin = detrt.DetLinear.from_quantized(W, sw, 0)
    y = detgpu.linear_residual(lin, q, s, x)
    ref = detgpu.dequant_residual(ops.igemm_i32(q, W), s, sw, x)
    assert torch.equal(y.view(torch.int32), ref.view(torch.int32))
    rows = [0, 1, m // 2 + 3, m - 1]
    acc = (q[rows].cpu().numpy().astype(np.int64) @ W.cpu().numpy().astype(np.int64).T).astype(np.int32)
    want = x[rows].cpu().numpy() + S.dequant(acc, s[rows].cpu().numpy(), sw.cpu().numpy())
    assert np.array_equal(_u32(y[rows]), _u32(want))
    out = torch.empty_like(x)
    assert detgpu.linear_residual(lin, q, s, x, out=out) is out and torch.equal(out, y)


def _qkv_ref(acc, s1, sw, qnw, knw, cos, sin, B, T, H, Hkv, hd, eps, qknorm):
    qkv = S.dequant(acc, s1, sw)
    N = B * T
    q, k, v = qkv[:, :H * hd], qkv[:, H * hd:(H + Hkv) * hd], qkv[:, (H + Hkv) * hd:]
    q, k = q.reshape(N, H, hd), k.reshape(N, Hkv, hd)
    if qknorm:
        q, k = S.det_rmsnorm(q, qnw, eps), S.det_rmsnorm(k, knw, eps)
    pos = np.arange(N) % T
    qr, kr = S.rope(q, cos[pos][:, None], sin[pos][:, None]), S.rope(k, cos[pos][:, None], sin[pos][:, None])
    return S.quant_sym(qr, 127), S.quant_sym(kr, 127), S.quant_sym(v.reshape(N, Hkv, hd), 127)


@pytest.mark.parametrize("B,T,H,Hkv,hd,qknorm", [(1, 12, 4, 2, 32, True), (2, 9, 4, 4, 64, False),
                                                  (1, 33, 16, 8, 128, True), (3, 7, 2, 1, 128, False)])
def test_qkv_post(dev, B, T, H, Hkv, hd, qknorm):
    from uwc_amd import detgpu
    rng = np.random.default_rng(B * 100 + T)
    N, W = B * T, (H + 2 * Hkv) * hd
    acc = rng.integers(-5_000_000, 5_000_000, (N, W)).astype(np.int32)
    acc[0, :hd] = 0  # an all-zero head
    s1 = rng.uniform(1e-6, 1e-4, N).astype(np.float32)
    sw = rng.uniform(1e-4, 1e-2, W).astype(np.float32)
    qnw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    knw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    ang = np.arange(T)[:, None] * (1.0 / 10000 ** (np.arange(0, hd, 2) / hd))[None]
    cos = np.cos(np.concatenate([ang, ang], 1)).astype(np.float32)
    sin = np.sin(np.concatenate([ang, ang], 1)).astype(np.float32)
    eps = np.float32(1e-6)
    (rq, rqs), (rk, rks), (rv, rvs) = _qkv_ref(acc, s1, sw, qnw, knw, cos, sin, B, T, H, Hkv, hd, eps, qknorm)
    out = detgpu.qkv_post_vt(_t(acc, dev), _t(s1, dev), _t(sw, dev), _t(qnw, dev), _t(knw, dev), _t(cos, dev),
                             _t(sin, dev), T, H, Hkv, float(eps), qknorm)
    qq, qs, kq, ks, vq, vs, vt = (o.cpu().numpy() for o in out)
    assert np.array_equal(qq, rq) and np.array_equal(_u32(qs), _u32(rqs))
    assert np.array_equal(kq, rk) and np.array_equal(_u32(ks), _u32(rks))
    assert np.array_equal(vq, rv) and np.array_equal(_u32(vs), _u32(rvs))
    # vt is V in the attention kernel's key order
    Tp = vt.shape[-1]
    for n in range(N):
        bseq, pos = divmod(n, T)
        j = (pos & ~63) | (((pos >> 2) & 3) << 4) | (((pos >> 4) & 3) << 2) | (pos & 3)
        assert np.array_equal(vt[bseq, :, :, j], rv[n]), n
    assert Tp % 64 == 0
    for pos in range(T, Tp):  # pad keys: zero
        j = (pos & ~63) | (((pos >> 2) & 3) << 4) | (((pos >> 4) & 3) << 2) | (pos & 3)
        assert not vt[:, :, :, j].any(), pos


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("B,T,H,Hkv,hd", [(1, 1, 1, 1, 32), (1, 12, 4, 2, 32), (2, 70, 4, 2, 64),
                                          (1, 300, 2, 1, 128), (1, 129, 16, 8, 128), (1, 100, 8, 2, 64),
                                          (2, 70, 8, 1, 128)])
def test_attention(dev, B, T, H, Hkv, hd, stored):
    """Both forms of the kernel (exponentials recomputed per pass, or kept in the scratch of
    uwc_attention_ws) against the oracle's attention, bit for bit; 1, 2, 4 and 8 heads per kv
    head (the stored form's row max takes 1, 2 or 4 heads per workgroup)."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(T * 7 + hd)
    N = B * T
    qq = rng.integers(-127, 128, (N, H, hd)).astype(np.int8)
    kq = rng.integers(-127, 128, (N, Hkv, hd)).astype(np.int8)
    vq = rng.integers(-127, 128, (N, Hkv, hd)).astype(np.int8)
    qs = rng.uniform(1e-3, 3e-2, (N, H, 1)).astype(np.float32)
    ks = rng.uniform(1e-3, 3e-2, (N, Hkv, 1)).astype(np.float32)
    vs = rng.uniform(1e-3, 3e-2, (N, Hkv, 1)).astype(np.float32)
    inv = S.inv_sqrt_hd(hd)
    o = detgpu.attention(_t(qq, dev), _t(qs, dev), _t(kq, dev), _t(ks, dev), _t(vq, dev), _t(vs, dev), B, T, H, Hkv,
                         float(inv), stored_exp=stored).cpu().numpy()
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        _, _, _, ref = S.attention(qq[sl].astype(np.int64), qs[sl], kq[sl].astype(np.int64), ks[sl],
                                   vq[sl].astype(np.int64), vs[sl], inv)
        np.testing.assert_array_equal(_u32(o[sl]), _u32(ref.transpose(1, 0, 2).reshape(T, H * hd)))


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("lo,hi,T,hd", [(0.1, 0.4, 300, 64), (0.5, 2.0, 200, 128), (0.2, 1.0, 150, 32),
                                        (0.05, 0.1, 260, 64), (0.03, 0.08, 260, 128)])
def test_attention_underflowing_exponentials(dev, lo, hi, T, hd, stored):
    """Large q and k scales spread the scores over hundreds of nats, so exponentials underflow
    (det_exp's t < -126 rule; 96-97% of them at the first three scale ranges, 38% and 7% at the
    last two): in tiles without masked keys the kernel leaves that rule out (a subnormal instead
    of 0), which no output can show; both forms against the oracle bit for bit."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(int(hi * 100) + T)
    H, Hkv = 4, 2
    qq = rng.integers(-127, 128, (T, H, hd)).astype(np.int8)
    kq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int8)
    vq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int8)
    qs = rng.uniform(lo, hi, (T, H, 1)).astype(np.float32)
    ks = rng.uniform(lo, hi, (T, Hkv, 1)).astype(np.float32)
    vs = rng.uniform(1e-3, 3e-2, (T, Hkv, 1)).astype(np.float32)
    inv = S.inv_sqrt_hd(hd)
    o = detgpu.attention(_t(qq, dev), _t(qs, dev), _t(kq, dev), _t(ks, dev), _t(vq, dev), _t(vs, dev), 1, T, H, Hkv,
                         float(inv), stored_exp=stored).cpu().numpy()
    _, _, _, ref = S.attention(qq.astype(np.int64), qs, kq.astype(np.int64), ks, vq.astype(np.int64), vs, inv)
    np.testing.assert_array_equal(_u32(o), _u32(ref.transpose(1, 0, 2).reshape(T, H * hd)))


@pytest.mark.parametrize("stored", [False, True])
@pytest.mark.parametrize("period,T,hd", [(7, 300, 64), (3, 200, 128), (64, 260, 32)])
def test_attention_repeated_keys(dev, period, T, hd, stored):
    """Keys, values and their scales repeating every `period` positions give exact ties in e * vs
    between keys (the case in which the kernel's candidate tracking for the row statistic pm
    must fall back to the full sweep), mixed with rows that have none (period 64 with 16-key lane
    groups): both forms against the oracle's attention, bit for bit."""
    from uwc_amd import detgpu
    rng = np.random.default_rng(period * 31 + T)
    H, Hkv = 4, 2
    qq = rng.integers(-127, 128, (T, H, hd)).astype(np.int8)
    base = lambda *shape: rng.integers(-127, 128, (period,) + shape).astype(np.int8)  # noqa: E731
    kq = np.resize(base(Hkv, hd), (T, Hkv, hd)).astype(np.int8)
    vq = np.resize(base(Hkv, hd), (T, Hkv, hd)).astype(np.int8)
    qs = rng.uniform(1e-3, 3e-2, (T, H, 1)).astype(np.float32)
    ks = np.resize(rng.uniform(1e-3, 3e-2, (period, Hkv, 1)).astype(np.float32), (T, Hkv, 1))
    vs = np.resize(rng.uniform(1e-3, 3e-2, (period, Hkv, 1)).astype(np.float32), (T, Hkv, 1))
    inv = S.inv_sqrt_hd(hd)
    o = detgpu.attention(_t(qq, dev), _t(qs, dev), _t(kq, dev), _t(ks, dev), _t(vq, dev), _t(vs, dev), 1, T, H, Hkv,
                         float(inv), stored_exp=stored).cpu().numpy()
    _, _, _, ref = S.attention(qq.astype(np.int64), qs, kq.astype(np.int64), ks, vq.astype(np.int64), vs, inv)
    np.testing.assert_array_equal(_u32(o), _u32(ref.transpose(1, 0, 2).reshape(T, H * hd)))


@pytest.mark.parametrize("B,T,H,Hkv,hd", [(1, 2048, 16, 8, 128), (2, 1000, 4, 4, 64), (1, 777, 8, 2, 32),
                                          (1, 1500, 16, 2, 128)])
def test_attention_stored_equals_recomputed(dev, B, T, H, Hkv, hd):
    """The stored-exponentials form equals the recomputing one bit for bit at sizes the oracle
    would take minutes for (the oracle comparison above covers both at small T)."""
    from uwc_amd import detgpu
    g = torch.Generator(device=dev)
    g.manual_seed(T + hd)
    N = B * T
    qq = torch.randint(-127, 128, (N, H, hd), dtype=torch.int8, device=dev, generator=g)
    kq = torch.randint(-127, 128, (N, Hkv, hd), dtype=torch.int8, device=dev, generator=g)
    vq = torch.randint(-127, 128, (N, Hkv, hd), dtype=torch.int8, device=dev, generator=g)
    qs = torch.rand((N, H, 1), device=dev, generator=g) * 3e-2 + 1e-3
    ks = torch.rand((N, Hkv, 1), device=dev, generator=g) * 3e-2 + 1e-3
    vs = torch.rand((N, Hkv, 1), device=dev, generator=g) * 3e-2 + 1e-3
    inv = float(S.inv_sqrt_hd(hd))
    a = detgpu.attention(qq, qs, kq, ks, vq, vs, B, T, H, Hkv, inv, stored_exp=False)
    b = detgpu.attention(qq, qs, kq, ks, vq, vs, B, T, H, Hkv, inv, stored_exp=True)
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_attention_stored_on_two_streams(dev):
    """Stored-exponentials attention calls queued on two streams at once, of different sizes, each
    equal to the recomputing form: every call has its own scratch (stream-ordered allocation)."""
    from uwc_amd import detgpu
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    H, Hkv, hd = 8, 4, 128
    inv = float(S.inv_sqrt_hd(hd))
    cases = []
    for T in (1500, 900):
        mk = lambda *s: torch.randint(-127, 128, s, dtype=torch.int8, device=dev, generator=g)  # noqa: E731
        sc = lambda *s: torch.rand(s, device=dev, generator=g) * 3e-2 + 1e-3  # noqa: E731
        cases.append((T, (mk(T, H, hd), sc(T, H, 1), mk(T, Hkv, hd), sc(T, Hkv, 1), mk(T, Hkv, hd), sc(T, Hkv, 1))))
    want = [detgpu.attention(*a, 1, T, H, Hkv, inv, stored_exp=False) for T, a in cases]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = []
    for _ in range(3):
        got = []
        for st, (T, a) in zip(streams, cases):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                got.append(detgpu.attention(*a, 1, T, H, Hkv, inv, stored_exp=True))
        outs.append(got)
    torch.cuda.synchronize()
    for got in outs:
        for x, y in zip(got, want):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))


def _fixture_model(name, dev):
    from uwc_amd import detgpu
    d = np.load(os.path.join(GOLDEN, name + ".npz"))
    m = S.model_from_fixture(d)
    gm = detgpu.DetModel.from_tables(m.cfg, m.embed, m.norms, m.lins, m.cos, m.sin, device=dev)
    return d, m, gm


@pytest.mark.parametrize("name", ["stage_tiny_qwen3", "stage_tiny_llama"])
def test_fixture_stages_on_gpu(dev, name):
    from uwc_amd import detgpu
    d, m, gm = _fixture_model(name, dev)
    cfg = m.cfg
    H, Hkv, hd = cfg["H"], cfg["Hkv"], cfg["hd"]
    for si in range(3):
        T, l0, l1 = (int(v) for v in d[f"s{si}_meta"])
        tokens = _t(d[f"s{si}_tokens"][None], dev) if l0 == 0 else None
        x = _t(d[f"s{si}_input"][None], dev) if l0 > 0 else None
        out = detgpu.stage_outputs(gm, tokens, x, l0, l1)
        rows, ref_out = S.run_stage(m, d[f"s{si}_tokens"] if l0 == 0 else None, d.get(f"s{si}_input"), l0, l1)
        assert np.array_equal(_u32(out[0]), _u32(ref_out)), f"{name} stage {si}: outputs differ"
        if f"s{si}_words" in d:  # the committed output rows themselves
            fr = S.fixture_rows(d, si)
            assert np.array_equal(_u32(out[0]), np.stack(fr[-T:]))
        # stage output root on the GPU vs hashlib
        assert detgpu.stage_output_roots(out)[0] == S.stage_output_root(ref_out)
    # the fused kernels' exposed leaves, layer 0 of stage 0
    T = int(d["s0_meta"][0])
    leaves = S.program(H, Hkv, hd, T, 0, 1)
    R = dict(zip(leaves, S.fixture_rows(d, 0)))
    L = gm.layers[0]
    x = detgpu.embed(gm.embed, _t(d["s0_tokens"], dev))
    q1, s1 = detgpu.rmsnorm_quant(x, L["in_norm"], gm.eps, L["qkv"].bs)
    qrow = lambda q, s: np.concatenate([q.astype(np.int32), np.asarray([s], np.float32).view(np.int32)]).view(np.uint32)
    q1n, s1n = q1.cpu().numpy(), s1.cpu().numpy()
    for t in range(T):
        assert np.array_equal(qrow(q1n[t], s1n[t]), R[("QA1", 0, t, -1)])
    qq, qs, kq, ks, vq, vs, vt = detgpu.qkv_post_vt(L["qkv"].int_gemm(q1), s1, L["qkv"].sw, L["q_norm"], L["k_norm"],
                                                    L["cos"][:T], L["sin"][:T], T, H, Hkv, gm.eps, gm.qk_norm)
    o = detgpu.attention(qq, qs, kq, ks, vq, vs, 1, T, H, Hkv, gm.inv_sqrt_hd, vt=vt)
    qqn, qsn, kqn, ksn, vqn, vsn, on = (a.cpu().numpy() for a in (qq, qs, kq, ks, vq, vs, o))
    for t in range(T):
        for h in range(H):
            assert np.array_equal(qrow(qqn[t, h], qsn[t, h, 0]), R[("QQ", 0, t, h)])
            assert np.array_equal(_u32(on[t, h * hd:(h + 1) * hd]), R[("O", 0, t, h)])
        for h in range(Hkv):
            assert np.array_equal(qrow(kqn[t, h], ksn[t, h, 0]), R[("KQ", 0, t, h)])
            assert np.array_equal(qrow(vqn[t, h], vsn[t, h, 0]), R[("VQ", 0, t, h)])


def test_forward_stage_roots_batched(dev):
    """forward_stage_roots (every layer's output kept, all stage-output roots hashed in one batched
    set of launches) gives each layer's output and root exactly as the layer-by-layer forward with
    stage_roots_gpu per layer does, and the fixture model's roots equal the oracle's."""
    from uwc_amd import detgpu
    d, m, gm = _fixture_model("stage_tiny_qwen3", dev)
    toks = d["s0_tokens"]
    x, roots = detgpu.forward_stage_roots(gm, _t(toks[None], dev))
    xo = m.embed[toks]
    for l in range(len(gm.layers)):
        xo = S.layer(m, l, xo)
        assert bytes(detgpu.digest_bytes(roots)[l]) == S.stage_output_root(xo), l
    assert np.array_equal(_u32(x), _u32(xo))
    # a random model of 5 layers at T = 300 (ragged trees), against the per-layer forward
    cfg = dict(D=256, H=4, Hkv=2, hd=64, I=512, L=5, V=1000, eps=1e-6, Bs=128, max_pos=512, theta=1e6, arch=0)
    rm = detgpu.DetModel.random(cfg, seed=3, device=dev, with_lm_head=False)
    T = 300
    tok = torch.from_numpy(np.random.default_rng(5).integers(0, cfg["V"], size=(1, T))).to(dev)
    xb, rb = detgpu.forward_stage_roots(rm, tok)
    xs = detgpu.embed(rm.embed, tok)
    for l, L in enumerate(rm.layers):
        xs = detgpu.layer_fused(rm, L, xs, 1, T)
        assert torch.equal(detgpu.stage_roots_gpu(xs.reshape(1, T, cfg["D"]))[0], rb[l]), l
    assert torch.equal(xb, xs)


def test_qwen3_1p7b_rows_on_gpu(dev):
    """The non-GEMM ops at the real shape (hd 128, 16 / 8 heads, I 6144) from the fixture's inputs."""
    from uwc_amd import detgpu
    d = np.load(os.path.join(GOLDEN, "stage_qwen3_1p7b.npz"))
    D, H, Hkv, hd, I, L_, V, eps_bits, Bs, max_pos, arch = (int(v) for v in d["cfg"])
    eps = float(np.array([eps_bits], np.uint32).view(np.float32)[0])
    cos, sin = _t(d["w_rope_cos"], dev), _t(d["w_rope_sin"], dev)
    f32 = lambda r: np.asarray(r).view(np.float32)
    qrow = lambda q, s: np.concatenate([q.astype(np.int32), np.asarray([s], np.float32).view(np.int32)]).view(np.uint32)
    for si in (0, 1):
        T, l0, l1 = (int(v) for v in d[f"s{si}_meta"])
        l = l0
        R = dict(zip(S.program(H, Hkv, hd, T, l0, l1), S.fixture_rows(d, si)))
        x = np.stack([f32(R[("EMBED", 0, t, -1)]) for t in range(T)]) if si == 0 else d["s1_input"]
        nw = {nm: _t(d[f"w_{nm}_{l}"], dev) for nm in ("in_norm", "post_norm", "q_norm", "k_norm")}
        # N1 + QA1
        q1, s1 = detgpu.rmsnorm_quant(_t(x, dev), nw["in_norm"], eps, min(Bs, D & -D))
        q1n, s1n = q1.cpu().numpy(), s1.cpu().numpy()
        for t in range(T):
            assert np.array_equal(qrow(q1n[t], s1n[t]), R[("QA1", l, t, -1)])
        # qkv_post from the fixture's fp32 QKV rows (the int32 path is pinned by the tiny stages)
        qkv = np.stack([f32(R[("QKV", l, t, -1)]) for t in range(T)])
        qq, qs, kq, ks, vq, vs, vt = detgpu.qkv_post_vt(_t(qkv, dev), None, None, nw["q_norm"], nw["k_norm"], cos, sin,
                                                        T, H, Hkv, eps, True)
        o = detgpu.attention(qq, qs, kq, ks, vq, vs, 1, T, H, Hkv, float(S.inv_sqrt_hd(hd)), vt=vt)
        qqn, qsn, kqn, ksn, vqn, vsn, on = (a.cpu().numpy() for a in (qq, qs, kq, ks, vq, vs, o))
        for t in range(T):
            for h in range(H):
                assert np.array_equal(qrow(qqn[t, h], qsn[t, h, 0]), R[("QQ", l, t, h)])
                assert np.array_equal(_u32(on[t, h * hd:(h + 1) * hd]), R[("O", l, t, h)])
            for h in range(Hkv):
                assert np.array_equal(qrow(kqn[t, h], ksn[t, h, 0]), R[("KQ", l, t, h)])
                assert np.array_equal(qrow(vqn[t, h], vsn[t, h, 0]), R[("VQ", l, t, h)])
        # QA2 from O
        q2, s2 = detgpu.quant_act(o, min(Bs, (H * hd) & -(H * hd)))
        q2n, s2n = q2.cpu().numpy(), s2.cpu().numpy()
        # R1 = x + OP (fp32 OP rows)
        op = np.stack([f32(R[("OP", l, t, -1)]) for t in range(T)])
        r1 = detgpu.dequant_residual(_t(op, dev), None, None, _t(x, dev))
        q3, s3 = detgpu.rmsnorm_quant(r1, nw["post_norm"], eps, min(Bs, D & -D))
        r1n, q3n, s3n = r1.cpu().numpy(), q3.cpu().numpy(), s3.cpu().numpy()
        # SM / QA4 from the fp32 GU rows; R2 = R1 + DN
        gu = np.stack([f32(R[("GU", l, t, -1)]) for t in range(T)])
        q4, s4 = detgpu.swiglu_quant(_t(gu, dev), None, None, min(Bs, I & -I))
        dn = np.stack([f32(R[("DN", l, t, -1)]) for t in range(T)])
        r2 = detgpu.dequant_residual(_t(dn, dev), None, None, r1).cpu().numpy()
        q4n, s4n = q4.cpu().numpy(), s4.cpu().numpy()
        for t in range(T):
            assert np.array_equal(qrow(q2n[t], s2n[t]), R[("QA2", l, t, -1)])
            assert np.array_equal(_u32(r1n[t]), R[("R1", l, t, -1)])
            assert np.array_equal(qrow(q3n[t], s3n[t]), R[("QA3", l, t, -1)])
            assert np.array_equal(qrow(q4n[t], s4n[t]), R[("QA4", l, t, -1)])
            assert np.array_equal(_u32(r2[t]), R[("R2", l, t, -1)])


def test_sha_row_roots_and_trace_roots(dev):
    from uwc_amd import detgpu
    rng = np.random.default_rng(11)
    # row roots for lengths around the 1 KiB block and message-padding boundaries
    # (up to 64 blocks per row: a quad per row, 16 rows per workgroup; 65 and more: a thread per
    # row), with row counts that leave a workgroup partly empty
    for w, nr in ((1, 5), (13, 5), (14, 5), (15, 5), (16, 5), (17, 5), (255, 5), (256, 5), (257, 5), (300, 5),
                  (512, 5), (2048, 37), (2049, 5), (6144, 17), (16384, 3), (16385, 3), (40000, 2)):
        rows = rng.integers(-2**31, 2**31 - 1, (nr, w), dtype=np.int64).astype(np.int32)
        got = detgpu.digest_bytes(detgpu.row_roots(_t(rows, dev)))
        for i in range(nr):
            assert bytes(got[i]) == S.row_root(rows[i]), (w, i)
    # stage-output roots for several tree sizes
    for T in (1, 2, 3, 5, 8, 12, 33, 512, 513, 700, 1100, 2048):  # > 512: the two-phase tree
        out = rng.standard_normal((2, T, 40)).astype(np.float32)
        roots = detgpu.stage_output_roots(_t(out, dev))
        assert roots == [S.stage_output_root(out[b]) for b in range(2)], T
    # the committed trace roots of the tiny fixtures, hashed on the GPU from the committed rows
    for name in ("stage_tiny_qwen3", "stage_tiny_llama", "stage_qwen3_1p7b"):
        d = np.load(os.path.join(GOLDEN, name + ".npz"))
        for si in (0, 1):
            rows = [_t(r.view(np.int32), dev) for r in S.fixture_rows(d, si)]
            assert detgpu.trace_root(rows) == bytes(d[f"s{si}_root"]), (name, si)
