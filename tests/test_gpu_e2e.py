"""configs[4] at its full size: the 28-layer Qwen3-1.7B-shaped deterministic forward over 8192 tokens
(vocab 151936, seeded random weights quantized per detrt), run once on the GPU exactly as the bench
runs it (detgpu.forward_stage_roots, then final_logits), and then checked layer by layer against the
CPU oracle: every layer l's output rows are recomputed by the oracle's layer l from the GPU's layer
l - 1 output (rows 0, 1, 8191, both sides of each 1024 boundary and random rows; the keys and values
of all 8192 positions), bit for bit, and every layer's stage-output root equals hashlib's SHA-256
Merkle root over the GPU's rows; the lm_head's int32 and fp32 logits on the same rows equal the
oracle's, and the logits' Merkle root is rebuilt with hashlib (runtime/detrt/qwen3.py:286-312,
runtime/bench/xdevice.py:52-56, spec/stage-program.md:82-88)."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import detrt_stage as S

pytestmark = pytest.mark.gpu

CFG = dict(D=2048, H=16, Hkv=8, hd=128, I=6144, L=28, V=151936, eps=1e-6, Bs=512, max_pos=8192, theta=1e6, arch=0)
T = 8192


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a)).view(np.uint32)


@pytest.fixture(scope="module")
def e2e(dev):
    """The GPU forward, its per-layer outputs and roots, the logits on the sampled rows and the
    oracle's model, all on the host; the GPU's copies are freed."""
    from uwc_amd import detgpu
    say("e2e 8192: building the 28-layer model on the GPU")
    m = detgpu.DetModel.random(CFG, seed=5, device=dev)
    rng = np.random.default_rng(2026)
    toks = rng.integers(0, CFG["V"], size=T)
    rows = np.array(sorted({0, 1, T - 1} | {b + d for b in range(1024, T, 1024) for d in (-1, 0)}
                           | set(rng.integers(0, T, 6).tolist())))
    louts = torch.empty((CFG["L"], T, CFG["D"]), dtype=torch.float32, device=dev)
    say("e2e 8192: forward_stage_roots + final_logits")
    x, roots = detgpu.forward_stage_roots(m, torch.from_numpy(toks[None]).to(dev), outs=louts)
    acc, logits = detgpu.final_logits(m, x)
    lroot = detgpu.merkle_roots(detgpu._row_leaf_words(acc, detgpu.TAG_SOUT, 0, 0), 1)
    acc_row_roots = detgpu.row_roots(acc)
    torch.cuda.synchronize()
    rd = torch.from_numpy(rows).to(dev)
    c = lambda t: t.detach().cpu().numpy()  # noqa: E731
    res = dict(rows=rows, louts=c(louts), roots=detgpu.digest_bytes(roots),
               acc_rows=c(acc[rd]), logits_rows=c(logits[rd]), lroot=bytes(detgpu.digest_bytes(lroot)[0]),
               acc_row_roots=detgpu.digest_bytes(acc_row_roots), x0=c(m.embed[torch.from_numpy(toks).to(dev)]))
    del x, roots, acc, logits, lroot, acc_row_roots, louts
    cfg = dict(CFG, eps_bits=int(np.float32(CFG["eps"]).view(np.uint32)))
    norms = [{nm: c(L[nm]) for nm in ("in_norm", "post_norm", "q_norm", "k_norm")} for L in m.layers]
    lins = [{nm: (c(L[nm].Wq), c(L[nm].sw)) for nm in ("qkv", "o", "gu", "down")} for L in m.layers]
    res["om"] = S.Model(cfg, None, norms, lins, c(m.cos), c(m.sin), lm_head=(c(m.lm_head.Wq), c(m.lm_head.sw)),
                        final_norm=c(m.norm))
    del m
    torch.cuda.empty_cache()
    return res


@pytest.mark.parametrize("l0,l1", [(0, 7), (7, 14), (14, 21), (21, 28)])
def test_every_layer_rows_and_stage_roots(e2e, l0, l1):
    om, rows, louts = e2e["om"], e2e["rows"], e2e["louts"]
    for l in range(l0, l1):
        x_in = e2e["x0"] if l == 0 else louts[l - 1]
        say(f"e2e 8192: layer {l} on the oracle ({len(rows)} rows, keys and values of all {T})")
        want = S.layer_rows(om, l, x_in, rows)
        assert np.array_equal(_u32(louts[l][rows]), _u32(want)), f"layer {l} rows differ"
        assert bytes(e2e["roots"][l]) == S.stage_output_root(louts[l]), f"layer {l} stage root differs"


def test_lm_head_logits_rows_and_root(e2e):
    om, rows = e2e["om"], e2e["rows"]
    say(f"e2e 8192: lm_head on the oracle ({len(rows)} rows x {CFG['V']})")
    acc_o, logits_o = S.final_logits(om, e2e["louts"][-1][rows])
    assert np.array_equal(e2e["acc_rows"], acc_o)
    assert np.array_equal(_u32(e2e["logits_rows"]), _u32(logits_o))
    # row roots of the sampled rows from hashlib, and the logits root from hashlib over every row's
    # tagged leaf (the GPU's row roots)
    for i, t in enumerate(rows):
        assert bytes(e2e["acc_row_roots"][t]) == S.row_root(e2e["acc_rows"][i]), t
    leaves = [S.tagged_leaf(b"sout", t, bytes(r)) for t, r in enumerate(e2e["acc_row_roots"])]
    assert S.merkle_root(leaves) == e2e["lroot"]
