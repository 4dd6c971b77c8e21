"""Host-side logic of the package, checked on the CPU against independent definitions: the win-record
parser, limb counts, the 32-byte word packing, the HF-model helpers and detrt's pinned rope tables."""
from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest
import torch


def test_win_records_parse_count_cap_and_order():
    from uwc_amd import ops
    recs = [(64 * i, 2 * i, bytes(range(i, i + 32))) for i in range(5)]
    buf = np.zeros(1 + 3 * ops.WIN_WORDS, np.uint32)
    buf[0] = 5  # five winners, three record slots: records stop at the cap, the count keeps growing
    for i, (row, col, dig) in enumerate(recs[:3]):
        buf[1 + i * ops.WIN_WORDS:1 + (i + 1) * ops.WIN_WORDS] = [row, col, *np.frombuffer(dig, "<u4")]
    got = ops.win_records(torch.from_numpy(buf.view(np.int32)), 3)
    assert got == recs[:3]
    assert ops.win_records(torch.zeros(1 + ops.WIN_WORDS, dtype=torch.int32), 1) == []


def test_limb_counts_cover_projections():
    """L limbs of [-64, 63] reach exactly 63 (128^L - 1) / 127, the reference's thresholds
    (kernels.cu:602-607), and limbs_for(k) covers 127 k."""
    from uwc_amd import ops
    assert ops.LIMB_CAPS[:3] == (63, 8127, 1040319)
    for L, cap in enumerate(ops.LIMB_CAPS, 1):
        assert cap == sum(63 * 128 ** i for i in range(L))
        assert ops.limbs_for_max(cap) == L and ops.limbs_for_max(cap + 1) == min(L + 1, 4)
    for k in (1, 64, 65, 2048, 4096, 8191, 8192, 14336):
        L = ops.limbs_for(k)
        assert 127 * k <= ops.LIMB_CAPS[L - 1] and (L == 1 or 127 * k > ops.LIMB_CAPS[L - 2])


def test_words_round_trip_little_endian():
    from uwc_amd import ops
    b = bytes(range(7, 39))
    w = ops.words(b, "cpu")
    assert w.dtype == torch.int32 and w.numel() == 8
    assert int(w[0]) == int.from_bytes(b[:4], "little") and ops.words_to_bytes(w) == b


def test_hadamard_rotate_quant_rows():
    from uwc_amd import model as M
    for n in (1, 2, 4, 64, 512):
        H = M.hadamard(n, "cpu", torch.float64)
        assert torch.allclose(H @ H.T, torch.eye(n, dtype=torch.float64), atol=1e-12)  # orthonormal
        i, j = 3 % n, 5 % n
        assert H[i, j].item() == pytest.approx((-1) ** bin(i & j).count("1") / math.sqrt(n))
    x = torch.randn(2, 3, 1024)
    H = M.hadamard(256, "cpu")
    y = M.rotate(x, H)
    blocks = [x[..., s:s + 256] @ H for s in range(0, 1024, 256)]
    assert torch.allclose(y, torch.cat(blocks, -1))
    q, s = M.quant_rows(torch.tensor([[0.0, 1.0, -2.0, 0.5], [0.0, 0.0, 0.0, 0.0]]))
    assert q.tolist() == [[0, 32, -64, 16], [0, 0, 0, 0]] and s[1].item() == pytest.approx(1e-8 / 64)


def test_mineable_shape_rule():
    """Pearl's rank rule as model.py:93-97 states it: max(1024, 16 r) <= k <= 4 r^2, k % r, k % 64,
    n % tile."""
    from uwc_amd import model as M
    assert M.mineable_shape(4096, 2048, 128, 128)
    assert not M.mineable_shape(4096, 1024, 128, 128)      # k < 16 r
    assert M.mineable_shape(4096, 1024, 64, 128)
    assert not M.mineable_shape(4096, 65536 + 128, 128, 128)  # k > 4 r^2
    assert not M.mineable_shape(4100, 2048, 128, 128)


def test_rope_tables_pinned():
    """detrt's fp32 rope tables as this host computes them hash to the reference's pinned files
    (runtime/artifacts/*.npz; the Qwen3-1.7B one is rope_table_sha in results/step2/xdev_cpu.json:4)."""
    from uwc_amd import detgpu
    for (theta, hd, pos), want in detgpu.PINNED_ROPE_SHA.items():
        cos, sin = detgpu.rope_table(theta, hd, pos)
        assert cos.shape == (pos, hd) and cos.dtype == np.float32
        assert hashlib.sha256(cos.tobytes() + sin.tobytes()).hexdigest() == want
    assert detgpu.PINNED_ROPE_SHA[(1e6, 128, 8192)].startswith("8ee66518240c0e04")


def test_division_by_float64_reciprocal_is_correctly_rounded():
    """The kernels divide many float32 values by one per-row float32 constant d as
    float32(float64(x) * (1 / float64(d))) (uwc_div_rd, the attention's at_div): equal to the
    correctly rounded float32 quotient x / d for every float32 x and normal d > 0. Checked here
    against IEEE float32 division on 4 M random pairs over every exponent, quotients next to
    rounding midpoints (x = fl(q d) for q just off a midpoint), exact quotients and the
    quantizers' ranges."""
    rng = np.random.default_rng(2024)
    n = 1 << 22
    # random bit patterns: finite x of any exponent (incl. subnormal), normal positive d
    xb = rng.integers(0, 2**32, n, dtype=np.uint64).astype(np.uint32)
    x = xb.view(np.float32).copy()
    x[~np.isfinite(x)] = np.float32(1.5)
    db = rng.integers(0x00800000, 0x7F800000, n, dtype=np.uint64).astype(np.uint32)
    d = db.view(np.float32).copy()
    # keep the quotient finite and normal-range so that both sides are ordinary float32 values
    with np.errstate(over="ignore", under="ignore", invalid="ignore", divide="ignore"):
        ok = np.isfinite(x / d) & (np.abs(x / d) < np.float32(1e38)) & (np.abs(x / d) > np.float32(1e-37))
    x, d = x[ok], d[ok]
    # quantizer-like: |x| <= amax, d = amax / 127 (or / 64)
    amax = (rng.random(n // 4) * 100 + 1e-3).astype(np.float32)
    xq = (amax * (rng.random(n // 4) * 2 - 1)).astype(np.float32)
    dq = (amax / np.float32(127)).astype(np.float32)
    # near midpoints: x = fl(q d) with q = (2 k + 1) 2^-25 (1 + tiny), k random
    q = ((2 * rng.integers(2**23, 2**24, n // 4) + 1).astype(np.float64) * 2.0**-25) * (1 + 1e-15)
    dm = (rng.random(n // 4) + 0.5).astype(np.float32)
    xm = (q * dm.astype(np.float64)).astype(np.float32)
    # exact quotients
    de = (rng.random(n // 8) + 0.5).astype(np.float32)
    xe = (de * rng.integers(-127, 128, n // 8).astype(np.float32)).astype(np.float32)
    X = np.concatenate([x, xq, xm, xe])
    D = np.concatenate([d, dq, dm, de])
    with np.errstate(over="ignore", under="ignore"):
        want = X / D  # IEEE float32 division, correctly rounded
        rd = 1.0 / D.astype(np.float64)
        got = (X.astype(np.float64) * rd).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
