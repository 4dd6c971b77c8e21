"""GPU parity of the exact denoise at every limb count (kernels.cu:598-673): L = 1, 2, 3 and 4 from
the runtime maxabs, through the single hashed GEMM on both tilings, through the batched split-role
launch (one batch mixing limb counts), and through MinedWeight.forward / forward_many on operands
crafted so that a projection exceeds 8127 (three limbs in a real mined forward).

The 256 x 256 kernel has three denoise forms, each reached here: the corrections loaded into the
ring at once (L * 2r <= 256 bytes of k: L = 1, 2 at r = 64, L = 1 at r = 128), stage by stage in
the split kernel (L * 2r == 256), and streamed through the ring (L * 2r > 256)."""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

# a max |projection| in each limb range (kernels.cu:602-607), given as (maxabs[0], maxabs[1])
MAXABS = {1: (40, 63), 2: (64, 5000), 3: (9000, 8128), 4: (2_000_000, 17)}


def _ops():
    from uwc_amd import ops
    return ops


def _winset(w, max_wins, ops):
    words = w.cpu().numpy().view(np.uint32)
    c = min(int(words[0]), max_wins)
    recs = words[1:1 + c * ops.WIN_WORDS].reshape(c, ops.WIN_WORDS)
    return {(int(x[0]), int(x[1]), x[2:].astype("<u4").tobytes()) for x in recs}


def _case(rng, m, n, k, r):
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    B = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    corrA = rng.integers(-64, 64, size=(4, m, 2 * r), dtype=np.int8)
    corrB = rng.integers(-64, 64, size=(4, n, 2 * r), dtype=np.int8)
    return A, B, corrA, corrB


@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("r", [64, 128])
@pytest.mark.parametrize("cfg,m,n", [("256x256", 512, 256), ("128x128", 384, 256)])
def test_single_gemm_denoise_every_limb_count(dev, L, r, cfg, m, n):
    """uwc_noisy_gemm with FLAG_DENOISE (with and without the transcript): the output equals the
    oracle's noisy - sum_{li < L} 128^li corrA[li] corrB[li]^T, L chosen by maxabs, for L = 1..4;
    the hashed call's winners equal the plain-transcript oracle's."""
    ops = _ops()
    k = 1024
    print(f"case single L={L} r={r} cfg={cfg} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(1000 * L + r + m)
    A, B, corrA, corrB = _case(rng, m, n, k, r)
    mx = np.array(MAXABS[L], np.int32)
    want = O.denoise(O.igemm(A, B), corrA, corrB, mx)
    key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 8)
    msgs = O.transcript(A, B, r)
    want_wins = O.winners(O.tile_hashes(msgs, key), target)
    Ad, Bd = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    cA, cB = torch.from_numpy(corrA).to(dev), torch.from_numpy(corrB).to(dev)
    mxd = torch.from_numpy(mx).to(dev)
    for flags in (ops.FLAG_DENOISE, ops.FLAG_HASH | ops.FLAG_DENOISE):
        out = torch.empty((m, n), dtype=torch.int32, device=dev)
        wins = torch.zeros(1 + 512 * ops.WIN_WORDS, dtype=torch.int32, device=dev)
        hashed = bool(flags & ops.FLAG_HASH)
        ops.gemm(Ad, Bd, r=r, flags=flags, corrA=cA, corrB=cB, maxabs=mxd,
                 key=ops.words(key, dev) if hashed else None,
                 target=torch.from_numpy(target.view(np.int32).copy()).to(dev) if hashed else None,
                 wins=wins if hashed else None, max_wins=512, out=out, out_mode=ops.OUT_I32, cfg=cfg)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want), f"flags={flags}"
        if hashed:
            assert _winset(wins, 512, ops) == want_wins


@pytest.mark.parametrize("r,Ls", [(64, [3, 2, 1, 4, 3]), (128, [1, 2, 3, 1]), (64, [2, 3])])
def test_batched_split_denoise_mixed_limb_counts(dev, r, Ls):
    """uwc_noisy_gemm_many on the split-role kernel with items of different limb counts in one
    launch (each item picks L from its own maxabs): every item's output equals the oracle's, and
    its winner set equals its own single call's."""
    ops = _ops()
    m, n, k = 512, 512, 1024
    count = len(Ls)
    print(f"case batched r={r} Ls={Ls} m={m} n={n} k={k}", flush=True)
    rng = np.random.default_rng(7 * r + count)
    B = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    items = []
    for L in Ls:
        A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
        cA = rng.integers(-64, 64, size=(4, m, 2 * r), dtype=np.int8)
        cB = rng.integers(-64, 64, size=(4, n, 2 * r), dtype=np.int8)
        mx = np.array(MAXABS[L], np.int32)
        items.append(dict(A=A, cA=cA, cB=cB, mx=mx, key=rng.bytes(32),
                          want=O.denoise(O.igemm(A, B), cA, cB, mx)))
    target = O.bound_for_wins(m, n, 6)
    td = torch.from_numpy(target.view(np.int32).copy()).to(dev)
    Bd = torch.from_numpy(B).to(dev)
    As = [torch.from_numpy(it["A"]).to(dev) for it in items]
    cAs = [torch.from_numpy(it["cA"]).to(dev) for it in items]
    cBs = [torch.from_numpy(it["cB"]).to(dev) for it in items]
    mxs = [torch.from_numpy(it["mx"]).to(dev) for it in items]
    keys = [ops.words(it["key"], dev) for it in items]
    nw = 1 + 256 * ops.WIN_WORDS
    outs = [torch.empty((m, n), dtype=torch.int32, device=dev) for _ in items]
    wins = [torch.zeros(nw, dtype=torch.int32, device=dev) for _ in items]
    flags = ops.FLAG_HASH | ops.FLAG_DENOISE
    ops.gemm_many(As, Bd, r=r, flags=flags, corrAs=cAs, corrBs=cBs, maxabss=mxs, keys=keys, target=td, winss=wins,
                  max_wins=256, outs=outs, out_mode=ops.OUT_I32)
    torch.cuda.synchronize()
    for i, it in enumerate(items):
        assert np.array_equal(outs[i].cpu().numpy(), it["want"]), f"item {i} (L={Ls[i]})"
        one = torch.empty((m, n), dtype=torch.int32, device=dev)
        w1 = torch.zeros(nw, dtype=torch.int32, device=dev)
        ops.gemm(As[i], Bd, r=r, flags=flags, corrA=cAs[i], corrB=cBs[i], maxabs=mxs[i], key=keys[i], target=td,
                 wins=w1, max_wins=256, out=one, out_mode=ops.OUT_I32)
        torch.cuda.synchronize()
        assert torch.equal(one, outs[i]), i
        assert _winset(wins[i], 256, ops) == _winset(w1, 256, ops), i


def _three_limb_operand(rng, PB: np.ndarray, m: int, k: int, r: int) -> np.ndarray:
    """A random m x k operand in [-64, 64] with, in every row, +64 at each k position whose B-side
    selection pair starts at column c0 and -64 at each whose pair ends there (c0: the column with
    the most such positions), so that X[:, c0] = A S_B^T[:, c0] = 64 x (that count) > 8127."""
    first = PB.astype(np.uint32) & 0xFFFF
    second = PB.astype(np.uint32) >> 16
    cnt = np.bincount(first, minlength=r) + np.bincount(second, minlength=r)
    c0 = int(np.argmax(cnt))
    assert 64 * cnt[c0] > 8127, "too few selection positions for a three-limb projection"
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    A[:, first == c0] = 64
    A[:, second == c0] = -64
    return A


def test_mined_forward_three_limbs(dev):
    """A real mined forward whose projection X exceeds 8127 (three limbs, kernels.cu:602-607):
    MinedWeight.forward's output is the exact product and its winners equal the oracle's; then a
    forward_many sweep mixing three-limb and two-limb nonces in one batched launch gives every
    nonce's exact product and winner set."""
    ops = _ops()
    m, n, k, r = 256, 256, 4096, 64
    print(f"case mined three limbs m={m} n={n} k={k} r={r}", flush=True)
    rng = np.random.default_rng(8128)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    job_key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 12)
    blk = O.block_side(job_key, Bt, r)
    As = [_three_limb_operand(rng, blk["PB"], m, k, r), rng.integers(-64, 65, size=(m, k), dtype=np.int8),
          _three_limb_operand(rng, blk["PB"], m, k, r)]
    refs = [O.mined_forward(A, Bt, job_key, target, r, blk=blk) for A in As]
    assert [O.limbs_needed(int(x["maxabs"].max())) for x in refs] == [3, 2, 3]

    w = ops.MinedWeight(Bt=torch.from_numpy(Bt).to(dev), b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(job_key, target)
    ones = torch.ones(m, device=dev)
    Ad = [torch.from_numpy(A).to(dev) for A in As]
    out = w.forward(Ad[0], ones, out_mode=ops.OUT_I32)
    torch.cuda.synchronize()
    b = w._buf(m)
    assert np.array_equal(b["maxabs"].cpu().numpy(), refs[0]["maxabs"])
    assert np.array_equal(b["corrA"].cpu().numpy(), refs[0]["corrA"])
    assert np.array_equal(out.cpu().numpy(), refs[0]["out"])
    assert np.array_equal(refs[0]["out"], O.igemm(As[0], Bt))
    assert set(w.winners(m)) == refs[0]["winners"] and refs[0]["winners"]

    wins = [torch.zeros(1 + w.max_wins * ops.WIN_WORDS, dtype=torch.int32, device=dev) for _ in As]
    outs = w.forward_many(Ad, ones, out_mode=ops.OUT_I32, wins=wins)
    torch.cuda.synchronize()
    for i, ref in enumerate(refs):
        assert np.array_equal(outs[i].cpu().numpy(), ref["out"]), i
        assert _winset(wins[i], w.max_wins, ops) == ref["winners"], i
