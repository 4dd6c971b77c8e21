"""The decoder-layer / stage-commitment oracle (oracle/detrt_stage.py) against the reference's
Go-referee fixtures (tests/golden/stage_*.npz, extracted by tests/golden/make_stage_fixtures.py).

  * tiny Qwen3 and tiny Llama (D 128, 4 q / 2 kv heads x hd 32, I 256, Hadamard block 64, 12
    tokens): every leaf row of both one-layer stages (all 26 op kinds, including the GEMM rows)
    and the three committed stage trace roots (SHA-256 over every row in program order);
  * real Qwen3-1.7B rows (hd 128, 8 tokens, both fixture layers): each non-GEMM op recomputed
    from the fixture's own inputs (QKV -> QN KN QR KR KQ VQ QQ -> S P O; x + OP -> R1 -> N2;
    GU -> SM; R1 + DN -> R2; the four quant_act rows), and the GEMM rows at the 24 committed
    weight rows per linear.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle import detrt_stage as S

from conftest import GOLDEN


def _load(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"))


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a)).view(np.uint32)


@pytest.mark.parametrize("name", ["stage_tiny_qwen3", "stage_tiny_llama"])
def test_tiny_stages_rows_and_roots(name):
    d = _load(name)
    m = S.model_from_fixture(d)
    for si in range(3):
        T, l0, l1 = (int(v) for v in d[f"s{si}_meta"])
        tokens = d[f"s{si}_tokens"] if f"s{si}_tokens" in d else None
        xin = d[f"s{si}_input"] if f"s{si}_input" in d else None
        rows, out = S.run_stage(m, tokens, xin, l0, l1)
        if f"s{si}_words" in d:
            fr = S.fixture_rows(d, si)
            assert len(fr) == len(rows)
            leaves = S.program(m.cfg["H"], m.cfg["Hkv"], m.cfg["hd"], T, l0, l1)
            bad = [leaves[i] for i, (a, b) in enumerate(zip(rows, fr)) if not np.array_equal(_u32(a), b)]
            assert not bad, f"{name} stage {si}: {len(bad)} rows differ, first {bad[:4]}"
        assert S.trace_root(rows) == bytes(d[f"s{si}_root"]), f"{name} stage {si}: trace root differs"
        np.testing.assert_array_equal(_u32(out), _u32(rows[-T:]))  # the output is the last layer's R2 rows


def test_trace_root_detects_one_flipped_bit():
    d = _load("stage_tiny_qwen3")
    rows = [np.asarray(r) for r in S.fixture_rows(d, 0)]
    rows = [r.view(np.int32) for r in rows]
    assert S.trace_root(rows) == bytes(d["s0_root"])
    rows[300] = rows[300].copy()
    rows[300][0] ^= 1
    assert S.trace_root(rows) != bytes(d["s0_root"])


def test_merkle_shapes():
    """RFC 6962 shapes: one leaf is its own root; n leaves split at the largest power of two < n."""
    lv = [bytes([i]) * 32 for i in range(5)]
    assert S.merkle_root(lv[:1]) == lv[0]
    n2 = S._node(lv[0], lv[1])
    assert S.merkle_root(lv[:2]) == n2
    assert S.merkle_root(lv[:3]) == S._node(n2, lv[2])
    assert S.merkle_root(lv[:5]) == S._node(S._node(n2, S._node(lv[2], lv[3])), lv[4])
    # an empty row still has one (empty) block
    assert S.row_root(np.zeros(0, np.float32)) == S._leaf(b"")


def _rows_by_leaf(d, si, cfg):
    T, l0, l1 = (int(v) for v in d[f"s{si}_meta"])
    leaves = S.program(cfg["H"], cfg["Hkv"], cfg["hd"], T, l0, l1)
    return T, l0, dict(zip(leaves, S.fixture_rows(d, si)))


def test_qwen3_1p7b_nongemm_ops():
    d = _load("stage_qwen3_1p7b")
    D, H, Hkv, hd, I, L, V, eps_bits, Bs, max_pos, arch = (int(v) for v in d["cfg"])
    cfg = dict(H=H, Hkv=Hkv, hd=hd)
    eps = np.array([eps_bits], np.uint32).view(np.float32)[0]
    cos, sin = d["w_rope_cos"], d["w_rope_sin"]
    assert list(d["w_rope_cos_rows"]) == list(range(len(cos)))
    f32 = lambda r: np.asarray(r).view(np.float32)
    i32 = lambda r: np.asarray(r).view(np.int32)
    checked = 0
    for si in (0, 1):
        T, l0, R = _rows_by_leaf(d, si, cfg)
        l = l0
        get = lambda op, t, h=-1: R[(op, l, t, h)]
        x = np.stack([f32(R[("EMBED", 0, t, -1)]) for t in range(T)]) if si == 0 else d[f"s{si}_input"]
        if si == 0:  # embedding rows of the stage's tokens
            emb = dict(zip(d["w_embed_rows"].tolist(), d["w_embed"]))
            np.testing.assert_array_equal(_u32(np.stack([emb[int(t)] for t in d["s0_tokens"]])), _u32(x))
        nw = {nm: d[f"w_{nm}_{l}"] for nm in ("in_norm", "post_norm", "q_norm", "k_norm")}
        # N1, QA1
        h1 = S.det_rmsnorm(x, nw["in_norm"], eps)
        np.testing.assert_array_equal(_u32(h1), np.stack([get("N1", t) for t in range(T)]))
        q1, s1 = S.quant_act(h1, S.lin_bs(Bs, D))
        np.testing.assert_array_equal(np.stack([S._qrow(q1[t], s1[t]).view(np.uint32) for t in range(T)]),
                                      np.stack([get("QA1", t) for t in range(T)]))
        # QKV -> QN KN QR KR KQ VQ QQ
        qkv = np.stack([f32(get("QKV", t)) for t in range(T)])
        q, k, v = qkv[:, :H * hd], qkv[:, H * hd:(H + Hkv) * hd], qkv[:, (H + Hkv) * hd:]
        qn = S.det_rmsnorm(q.reshape(T, H, hd), nw["q_norm"], eps)
        kn = S.det_rmsnorm(k.reshape(T, Hkv, hd), nw["k_norm"], eps)
        qr, kr = S.rope(qn, cos[:T, None], sin[:T, None]), S.rope(kn, cos[:T, None], sin[:T, None])
        kq, ks = S.quant_sym(kr, 127)
        vq, vs = S.quant_sym(v.reshape(T, Hkv, hd), 127)
        qq, qs = S.quant_sym(qr, 127)
        for t in range(T):
            for hh in range(H):
                assert np.array_equal(_u32(qn[t, hh]), get("QN", t, hh))
                assert np.array_equal(_u32(qr[t, hh]), get("QR", t, hh))
                assert np.array_equal(S._qrow(qq[t, hh], qs[t, hh, 0]).view(np.uint32), get("QQ", t, hh))
            for hh in range(Hkv):
                assert np.array_equal(_u32(kn[t, hh]), get("KN", t, hh))
                assert np.array_equal(_u32(kr[t, hh]), get("KR", t, hh))
                assert np.array_equal(S._qrow(kq[t, hh], ks[t, hh, 0]).view(np.uint32), get("KQ", t, hh))
                assert np.array_equal(S._qrow(vq[t, hh], vs[t, hh, 0]).view(np.uint32), get("VQ", t, hh))
        # S P O from the quantized heads
        sc, pi, sp, o = S.attention(qq, qs, kq, ks, vq, vs, S.inv_sqrt_hd(hd))
        for t in range(T):
            for hh in range(H):
                assert np.array_equal(_u32(sc[hh, t, :t + 1]), get("S", t, hh))
                assert np.array_equal(S._qrow(pi[hh, t, :t + 1], sp[hh, t, 0]).view(np.uint32), get("P", t, hh))
                assert np.array_equal(_u32(o[hh, t]), get("O", t, hh))
        # QA2 from O; R1 = x + OP; N2; QA3; SM; QA4; R2 = R1 + DN
        oc = o.transpose(1, 0, 2).reshape(T, H * hd)
        q2, s2 = S.quant_act(oc, S.lin_bs(Bs, H * hd))
        op = np.stack([f32(get("OP", t)) for t in range(T)])
        r1 = x + op
        h2 = S.det_rmsnorm(r1, nw["post_norm"], eps)
        q3, s3 = S.quant_act(h2, S.lin_bs(Bs, D))
        gu = np.stack([f32(get("GU", t)) for t in range(T)])
        sm = S.det_silu(gu[:, :I]) * gu[:, I:]
        q4, s4 = S.quant_act(sm, S.lin_bs(Bs, I))
        dn = np.stack([f32(get("DN", t)) for t in range(T)])
        r2 = r1 + dn
        for t in range(T):
            assert np.array_equal(S._qrow(q2[t], s2[t]).view(np.uint32), get("QA2", t))
            assert np.array_equal(_u32(r1[t]), get("R1", t))
            assert np.array_equal(_u32(h2[t]), get("N2", t))
            assert np.array_equal(S._qrow(q3[t], s3[t]).view(np.uint32), get("QA3", t))
            assert np.array_equal(_u32(sm[t]), get("SM", t))
            assert np.array_equal(S._qrow(q4[t], s4[t]).view(np.uint32), get("QA4", t))
            assert np.array_equal(_u32(r2[t]), get("R2", t))
        # the GEMM rows at the committed weight rows
        for lin, qa, out in (("qkv", (q1, s1), qkv), ("o", (q2, s2), op), ("gu", (q3, s3), gu), ("down", (q4, s4), dn)):
            p = f"w_{lin}_{l}"
            rows = d[p + "_rows"]
            y = S.dequant(S.int_gemm(qa[0], d[p + "_q"]), qa[1], d[p + "_s"])
            np.testing.assert_array_equal(_u32(y), _u32(out[:, rows]))
        # VT / VS
        for hh in range(Hkv):
            for dd in range(hd):
                assert np.array_equal(vq[:, hh, dd].astype(np.int32).view(np.uint32), get("VT", dd, hh))
            assert np.array_equal(_u32(vs[:, hh, 0]), get("VS", -1, hh))
        checked += 1
    assert checked == 2


def test_exact_rowsum_shift_for_softmax_rows():
    """The attention's exp rows have max exactly 1 (det_exp(0) == 1) and every term < 2, so their
    exact_rowsum scale is fixed: shift = 62 - 20 - 1 = 41 (the GPU kernel relies on this)."""
    rng = np.random.default_rng(5)
    z = -np.abs(rng.standard_normal((64, 300)).astype(np.float32)) * np.float32(30)
    z[:, 7] = 0
    z[:, 8] = -np.float32(1e-45)  # a denormal just below zero
    e = S.det_exp(z)
    assert e.max() == np.float32(1.0) and (e < 2).all() and (e >= 0).all()
    _, ex = np.frexp(e.max(axis=-1))
    assert (ex == 1).all()
    assert S.det_exp(np.float32(0.0)) == np.float32(1.0)
    assert S.det_exp(np.float32(-np.inf)) == np.float32(0.0)


def test_attention_rows_equals_full_attention():
    """The row-subset attention (used to check T = 8192 rows) is the full attention's rows, bit for
    bit, at sizes where the full (H, T, T) form runs, with GQA and the first and last positions."""
    rng = np.random.default_rng(23)
    T, H, Hkv, hd = 200, 4, 2, 64
    qq = rng.integers(-127, 128, (T, H, hd)).astype(np.int64)
    kq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int64)
    vq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int64)
    qs = rng.uniform(1e-3, 3e-2, (T, H, 1)).astype(np.float32)
    ks = rng.uniform(1e-3, 3e-2, (T, Hkv, 1)).astype(np.float32)
    vs = rng.uniform(1e-3, 3e-2, (T, Hkv, 1)).astype(np.float32)
    inv = S.inv_sqrt_hd(hd)
    full = S.attention(qq, qs, kq, ks, vq, vs, inv)
    rows = [0, 1, 63, 64, 127, 199, 150]
    part = S.attention_rows(qq, qs, kq, ks, vq, vs, inv, rows)
    for f, p in zip(full, part):
        np.testing.assert_array_equal(f[:, rows].view(np.uint32) if f.dtype == np.float32 else f[:, rows],
                                      p.view(np.uint32) if p.dtype == np.float32 else p)


@pytest.mark.parametrize("name", ["stage_tiny_qwen3", "stage_tiny_llama"])
def test_layer_rows_equals_full_layer(name):
    """layer_rows (the sampled-row form used to check every layer of the T = 8192 forward) is the
    full layer's rows, bit for bit, on the referee fixtures' models (Qwen3 with q/k norms, Llama
    without), first and last positions included; the full layer is pinned by the fixtures."""
    d = _load(name)
    m = S.model_from_fixture(d)
    rng = np.random.default_rng(5)
    T, D = 48, m.cfg["D"]
    x = rng.standard_normal((T, D)).astype(np.float32)
    rows = [0, 1, 17, 30, 47]
    for l in range(len(m.lins)):
        full = S.layer(m, l, x)
        part = S.layer_rows(m, l, x, rows)
        np.testing.assert_array_equal(_u32(full[rows]), _u32(part))
        x = full
