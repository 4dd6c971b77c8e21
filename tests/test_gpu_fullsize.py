"""GPU parity at the BASELINE configurations' full sizes, against the CPU oracle (the reference's own
checks are miner/ampere/tests/test_kernels.py:94-125 and the cross-device known answers of
miner/ampere/bench/crosscheck.py:62-76):

  configs[2]  4096^3, r = 64: eight nonces through MinedWeight.forward_many, i.e. the batched
              split-role GEMM launch the bench times; nonces 0 and 7 against the oracle's full
              mined forward (exact output, all 131,072 tile messages and digests, ~2000 winners),
              every nonce's output and winners against the single-nonce path;
  configs[1]  the four linears of a Qwen3-1.7B layer at M = 2048 through DetLinear;
  configs[3]  the four Llama-3.1-8B linears at M = 8192 as int32 GEMMs, and qkv / down through
              DetLinear with the 128-wide Hadamard block (sampled rows: rows are independent);
  configs[4]  exact attention at T = 8192 (16 / 8 heads, hd 128) on sampled query rows, one whole
              decoder layer at T = 2048 with its stage-output root, and the pinned rope table (the
              28-layer forward at T = 8192 is checked layer by layer in test_gpu_e2e.py);
plus DetLinear's mined path and a sweep after a new block template.

The oracle work is bounded to tens of seconds per test on the GPU box's host cores."""
from __future__ import annotations

import hashlib
import sys

import numpy as np
import pytest
import torch

import oracle as O
from oracle import detrt_stage as S

pytestmark = pytest.mark.gpu

QWEN3 = dict(D=2048, H=16, Hkv=8, hd=128, I=6144, L=1, V=1024, eps=1e-6, Bs=512, max_pos=8192, theta=1e6, arch=0)


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _u32(a) -> np.ndarray:
    if isinstance(a, torch.Tensor):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a).view(np.uint32)


def _winset(buf, max_wins):
    from uwc_amd import ops
    return set(ops.win_records(buf, max_wins))


def test_split_sweep_4096_matches_oracle(dev):
    """the timed kernel (noisy_gemm256 SPLIT, 8 nonces per launch) at 4096^3, r = 64."""
    from uwc_amd import ops
    m = n = k = 4096
    r, count = 64, 8
    rng = np.random.default_rng(4096)
    Bt = rng.integers(-64, 64, size=(n, k), dtype=np.int8)
    As = [rng.integers(-64, 64, size=(m, k), dtype=np.int8) for _ in range(count)]
    job_key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 2000)  # ~2000 winning tiles per nonce: the digests checked through the records
    w = ops.MinedWeight(Bt=torch.from_numpy(Bt).to(dev), b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(job_key, target)
    Ad = [torch.from_numpy(a).to(dev) for a in As]
    ones = torch.ones(m, device=dev)
    dumps = [torch.zeros((m // 64) * 8 * (n // 64) * 4 * ops.DUMP_WORDS, dtype=torch.int32, device=dev)
             for _ in range(count)]
    say("split sweep: forward_many of 8 nonces at 4096^3")
    outs = w.forward_many(Ad, ones, out_mode=ops.OUT_I32, group=8, gemm_group=8, dumps=dumps)
    torch.cuda.synchronize()
    sweep_wins = [set(x) for x in w.sweep_winners()]
    blk = O.block_side(job_key, Bt, r)
    for i in (0, count - 1):
        say(f"split sweep: oracle mined forward of nonce {i}")
        ref = O.mined_forward(As[i], Bt, job_key, target, r, blk=blk)
        assert np.array_equal(outs[i].cpu().numpy(), ref["out"]), i
        d = _u32(dumps[i]).reshape(m // 64, 8, n // 64, 4, ops.DUMP_WORDS)
        assert np.array_equal(d[..., :16], ref["msgs"]), (i, "tile messages")
        assert np.array_equal(d[..., 16:], ref["digests"]), (i, "tile digests")
        assert 1000 < len(ref["winners"]) < 4096 and sweep_wins[i] == ref["winners"], i
    say("split sweep: every nonce against the single-nonce path")
    for i in range(count):
        one = w.forward(Ad[i], ones, out_mode=ops.OUT_I32)
        torch.cuda.synchronize()
        assert torch.equal(one, outs[i]), i
        assert set(w.winners(m)) == sweep_wins[i], i


def test_sweep_after_new_block_template(dev):
    """forward_many, setup_block with another job key, forward_many again: every item still equals
    forward() and the oracle (the per-slot copies of corrB carry the new block's E_B)."""
    from uwc_amd import ops
    m, n, k, r = 256, 256, 1024, 64
    rng = np.random.default_rng(99)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    As = [rng.integers(-64, 65, size=(m, k), dtype=np.int8) for _ in range(5)]
    w = ops.MinedWeight(Bt=torch.from_numpy(Bt).to(dev), b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    Ad = [torch.from_numpy(a).to(dev) for a in As]
    ones = torch.ones(m, device=dev)
    for key in (b"\x01" * 32, b"\x02" * 32):
        target = O.bound_for_wins(m, n, 8)
        w.setup_block(key, target)
        outs = w.forward_many(Ad, ones, out_mode=ops.OUT_I32, group=2, gemm_group=2)
        torch.cuda.synchronize()
        got = [set(x) for x in w.sweep_winners()]
        for i, A in enumerate(Ad):
            one = w.forward(A, ones, out_mode=ops.OUT_I32)
            torch.cuda.synchronize()
            assert torch.equal(one, outs[i]), (key[:1], i)
            assert set(w.winners(m)) == got[i], (key[:1], i)
        ref = O.mined_forward(As[3], Bt, key, target, r)
        assert np.array_equal(outs[3].cpu().numpy(), ref["out"]) and got[3] == ref["winners"]


def _det_linears(dev, shapes, seed):
    from uwc_amd import detrt
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return {nm: detrt.DetLinear(torch.randn((nn_, kk), device=dev, generator=g) * 0.02, dev, 512)
            for nm, (nn_, kk) in shapes.items()}


def test_qwen3_layer_linears_2048(dev):
    """qkv, o, gate_up, down of a Qwen3-1.7B layer at M = 2048 (quant_act, exact GEMM,
    fused dequant) against the oracle's detrt linear, bit for bit."""
    M = 2048
    shapes = {"qkv": (4096, 2048), "o": (2048, 2048), "gu": (12288, 2048), "down": (2048, 6144)}
    lins = _det_linears(dev, shapes, 11)
    rng = np.random.default_rng(12)
    for nm, (nn_, kk) in shapes.items():
        x = rng.standard_normal((M, kk)).astype(np.float32)
        lin = lins[nm]
        y = lin(torch.from_numpy(x).to(dev)).cpu().numpy()
        say(f"layer linears: {nm} {M}x{kk} -> {nn_} on the oracle")
        want = O.det_linear(x, lin.Wq.cpu().numpy(), lin.sw.cpu().numpy(), lin.bs)
        want = want[-1] if isinstance(want, tuple) else want
        assert np.array_equal(_u32(y), _u32(want)), nm


def test_llama_prefill_8192_sampled_rows(dev):
    """configs[3] prefill: the four Llama-3.1-8B linears at M = 8192, qkv (4096 -> 6144), o
    (4096 -> 4096), gate_up (4096 -> 28672) and down (14336 -> 4096); the whole product runs on the
    GPU, sampled rows (first, last, random) are checked."""
    from uwc_amd import ops
    M = 8192
    rng = np.random.default_rng(8192)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(M - 64, M), rng.integers(0, M, 128)]))
    for nm, n, k in (("qkv", 6144, 4096), ("o", 4096, 4096), ("gu", 28672, 4096), ("down", 4096, 14336)):
        X = rng.integers(-64, 65, size=(M, k), dtype=np.int8)
        W = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
        C = ops.igemm_i32(torch.from_numpy(X).to(dev), torch.from_numpy(W).to(dev))
        sampled = C[torch.from_numpy(rows).to(dev)].cpu().numpy()
        del C
        torch.cuda.empty_cache()
        say(f"llama prefill: {nm} {M}x{k} -> {n}, {len(rows)} rows on the oracle")
        assert np.array_equal(sampled, O.igemm(X[rows], W)), nm


@pytest.mark.parametrize("nm,n,k", [("qkv", 6144, 4096), ("down", 4096, 14336)])
def test_llama_prefill_8192_detlinear(dev, nm, n, k):
    """configs[3] prefill through DetLinear (quant_act with Llama's 128-wide Hadamard block, exact
    GEMM, fused dequant; results/rules4/arch-llama3.1-8b-5090.json:4) at M = 8192: fp32 outputs of
    sampled rows bit for bit against the oracle's detrt linear (rows are independent)."""
    from uwc_amd import detrt
    M = 8192
    g = torch.Generator(device=dev)
    g.manual_seed(n + k)
    lin = detrt.DetLinear(torch.randn((n, k), device=dev, generator=g) * 0.02, dev, 128)
    assert lin.bs == 128
    x = torch.randn((M, k), device=dev, generator=g)
    y = lin(x)
    rng = np.random.default_rng(k)
    rows = np.unique(np.concatenate([np.arange(16), np.arange(M - 16, M), rng.integers(0, M, 64)]))
    rd = torch.from_numpy(rows).to(dev)
    got = y[rd].cpu().numpy()
    xs = x[rd].cpu().numpy()
    say(f"llama prefill detlinear: {nm} {M}x{k} -> {n}, {len(rows)} rows on the oracle")
    want = O.det_linear(xs, lin.Wq.cpu().numpy(), lin.sw.cpu().numpy(), lin.bs)[-1]
    assert np.array_equal(_u32(got), _u32(want)), nm


def test_attention_8192_sampled_rows(dev):
    """exact causal attention over 8192 keys, 16 query / 8 kv heads of 128, every query
    row on the GPU; the first and last rows, both sides of every 1024 boundary and random rows
    against the oracle."""
    from uwc_amd import detgpu
    T, H, Hkv, hd = 8192, 16, 8, 128
    rng = np.random.default_rng(81)
    qq = rng.integers(-127, 128, (T, H, hd)).astype(np.int8)
    kq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int8)
    vq = rng.integers(-127, 128, (T, Hkv, hd)).astype(np.int8)
    qs = rng.uniform(1e-3, 3e-2, (T, H, 1)).astype(np.float32)
    ks = rng.uniform(1e-3, 3e-2, (T, Hkv, 1)).astype(np.float32)
    vs = rng.uniform(1e-3, 3e-2, (T, Hkv, 1)).astype(np.float32)
    inv = S.inv_sqrt_hd(hd)
    t = lambda a: torch.from_numpy(a).to(dev)  # noqa: E731
    o = detgpu.attention(t(qq), t(qs), t(kq), t(ks), t(vq), t(vs), 1, T, H, Hkv, float(inv)).cpu().numpy()
    rows = sorted({0, 1, T - 1} | {b + d for b in range(1024, T, 1024) for d in (-1, 0)}
                  | set(rng.integers(0, T, 6).tolist()))
    say(f"attention 8192: {len(rows)} rows on the oracle")
    *_, ref = S.attention_rows(qq.astype(np.int64), qs, kq.astype(np.int64), ks, vq.astype(np.int64), vs, inv, rows)
    want = ref.transpose(1, 0, 2).reshape(len(rows), H * hd)
    np.testing.assert_array_equal(_u32(o[rows]), _u32(want))


def _oracle_of(m, cfg):
    """The oracle's Model for layer 0 of a GPU DetModel built from cfg."""
    c = lambda a: a.detach().cpu().numpy()  # noqa: E731
    cfg = dict(cfg, eps_bits=int(np.float32(cfg["eps"]).view(np.uint32)))
    L = m.layers[0]
    norms = [{nm: c(L[nm]) for nm in ("in_norm", "post_norm", "q_norm", "k_norm")}]
    lins = [{nm: (c(L[nm].Wq), c(L[nm].sw)) for nm in ("qkv", "o", "gu", "down")}]
    return S.Model(cfg, c(m.embed[:16]), norms, lins, c(m.cos), c(m.sin))


def test_decoder_layer_2048_and_pinned_rope(dev):
    """one Qwen3-1.7B-shaped decoder layer over 2048 tokens through the fused GPU layer
    equals the oracle's layer bit for bit, and so do its stage-output root; the rope tables the
    GPU model uses hash to detrt's pinned value (results/step2/xdev_cpu.json:4)."""
    from uwc_amd import detgpu
    m = detgpu.DetModel.random(QWEN3, seed=3, device=dev, with_lm_head=False)
    rope_sha = hashlib.sha256(m.cos.cpu().numpy().tobytes() + m.sin.cpu().numpy().tobytes()).hexdigest()
    assert rope_sha == "8ee66518240c0e045455c4ff8fb6cf1d959e22872c1e0dbba4bbc18985d3df26"
    T, D = 2048, QWEN3["D"]
    rng = np.random.default_rng(2048)
    x = rng.standard_normal((T, D)).astype(np.float32)
    y = detgpu.layer_fused(m, m.layers[0], torch.from_numpy(x).to(dev), 1, T)
    root = detgpu.stage_output_roots(y.reshape(1, T, D))[0]
    y = y.cpu().numpy()
    say("decoder layer 2048: oracle layer")
    want = S.layer(_oracle_of(m, QWEN3), 0, x)
    assert np.array_equal(_u32(y), _u32(want))
    assert root == S.stage_output_root(want)


def test_detlinear_mined_path(dev):
    """DetLinear(mine=True) (qwen3.py:94-116): a layer with k >= 2048 mines (hashed GEMM, exact
    denoise) and its int_gemm equals the plain exact GEMM, with the oracle's winners on the padded
    rows; a layer with k < 2048 is not mined (setup_block turns mine off)."""
    from uwc_amd import detrt, ops
    g = torch.Generator(device=dev)
    g.manual_seed(21)
    job_key = bytes(range(32))
    lin = detrt.DetLinear(torch.randn((6144, 2048), device=dev, generator=g) * 0.02, dev, 512, mine=True)
    target = O.bound_for_wins(128, 6144, 12)
    lin.setup_block(lambda kk: job_key, lambda kk: target)
    assert lin.mine and lin.mw is not None
    rng = np.random.default_rng(22)
    q = rng.integers(-64, 65, size=(64, 2048), dtype=np.int8)
    acc = lin.int_gemm(torch.from_numpy(q).to(dev))
    torch.cuda.synchronize()
    wins = set(lin.mw.winners(128))
    Wq = lin.Wq.cpu().numpy()
    assert np.array_equal(acc.cpu().numpy(), O.igemm(q, Wq))
    qp = np.zeros((128, 2048), np.int8)
    qp[:64] = q
    ref = O.mined_forward(qp, Wq, job_key, target, 128)
    assert ref["winners"] and wins == ref["winners"]
    small = detrt.DetLinear(torch.randn((2048, 1024), device=dev, generator=g) * 0.02, dev, 512, mine=True)
    small.setup_block(lambda kk: job_key, lambda kk: target)
    assert not small.mine and small.mw is None
