"""The CPU oracle pinned before it is trusted: known answers, golden fixtures, independent
restatements and brute force, chosen so that a dropped term, a wrong index or a transposed
operand fails at least one check."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle as O
from oracle.blake3_py import blake3 as py_b3
from conftest import GOLDEN


# ------------------------------------------------------------------ BLAKE3
def test_blake3_published_digests():
    # BLAKE3's published digests of the empty input and of "abc"
    assert O.b3(b"").hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"
    assert O.b3(b"abc").hex() == "6437b3ac38465133ffb63b75273a8db548c558465d79db03fd359c6cd5bd9d85"
    assert py_b3(b"").hex() == "af1349b9f5f9a1a6a0404dea36dcc9499bcb25c9adc112b7cc9a93cae41f3262"


def test_blake3_official_test_vectors():
    """The BLAKE3 team's published vectors (tests/golden/blake3_official_vectors.json): one block
    (len 0, 1), a full 16-block chunk (1024: chunk chaining, CHUNK_START/END), two chunks under a
    parent node (1025, 2048: chunk counter, PARENT, ROOT placement), ragged and deep trees (31744 =
    31 chunks, 102400 = 100 chunks), and keyed mode (KEYED_HASH flag and the key in place of the IV)
    on one block, one chunk and a parent node (2048), for both restatements."""
    v = json.load(open(os.path.join(GOLDEN, "blake3_official_vectors.json")))
    key = v["key"].encode()
    for case in v["cases"]:
        data = bytes(i % 251 for i in range(case["input_len"]))
        assert O.b3(data).hex() == case["hash"], case["input_len"]
        assert py_b3(data).hex() == case["hash"], case["input_len"]
        if "keyed_hash" in case:
            assert O.b3(data, key).hex() == case["keyed_hash"], case["input_len"]
            assert py_b3(data, key).hex() == case["keyed_hash"], case["input_len"]


@pytest.mark.parametrize("nchunks", list(range(1, 40)) + [63, 64, 65, 127, 128, 129])
def test_blake3_tree_shapes_agree(nchunks):
    """Recursive (C) and streaming-stack (Python) trees agree on every shape, keyed and plain."""
    rng = np.random.default_rng(nchunks)
    data = rng.bytes(nchunks * 1024)
    key = rng.bytes(32)
    assert O.b3(data, key) == py_b3(data, key)
    assert O.b3(data) == py_b3(data)


@pytest.mark.parametrize("n", [1, 63, 64, 65, 1023, 1025, 2047, 3000, 5121])
def test_blake3_ragged_lengths(n):
    rng = np.random.default_rng(n)
    data = rng.bytes(n)
    assert O.b3(data) == py_b3(data)
    assert O.b3(data, b"\x07" * 32) == py_b3(data, b"\x07" * 32)


def test_blake3_keyed_differs_and_counter_matters():
    # a dropped key flag or a chunk counter fixed at 0 would make these collide
    d = bytes(2048)
    assert O.b3(d) != O.b3(d, bytes(32))
    a = bytes(1024) + bytes([1]) + bytes(1023)
    b = bytes([1]) + bytes(1023) + bytes(1024)
    assert O.b3(a) != O.b3(b)


def test_seed_constants():
    # Pearl's salts: BLAKE3 of their ASCII names (reference.py:25-26)
    assert O.SEED_SALT_A == py_b3(b"pearl/cert-v3/noise-seed/A")
    assert O.SEED_SALT_B == py_b3(b"pearl/cert-v3/noise-seed/B")


# ------------------------------------------------------------------ noise
def _py_random_hash(index, label, key, prepend):
    msg = bytearray(64)
    msg[prepend * 4:prepend * 4 + 4] = (1 + index).to_bytes(4, "little")
    msg[32:64] = label
    return py_b3(bytes(msg), key)


def test_noise_uniform_matches_python_random_hash():
    key = bytes(range(32))
    E = O.uniform_matrix(O.SEED_LABEL_A, key, 8, 64)
    raw = b"".join(_py_random_hash(b, O.SEED_LABEL_A, key, 0) for b in range(16))
    want = ((np.frombuffer(raw, np.uint8) & 63).astype(np.int16) - 32).astype(np.int8).reshape(8, 64)
    assert np.array_equal(E, want)
    assert E.min() >= -32 and E.max() <= 31


@pytest.mark.parametrize("r", [64, 128])
def test_noise_perm_matches_python_and_invariants(r):
    key = bytes(range(1, 33))
    k = 1000
    P = O.perm_packed(O.SEED_LABEL_B, key, k, r)
    first, second = P & 0xFFFF, P >> 16
    assert (first < r).all() and (second < r).all() and (first != second).all()
    for i in range(0, (k + 7) // 8, 17):
        u = np.frombuffer(_py_random_hash(i, O.SEED_LABEL_B, key, 1), "<u4").astype(np.uint64)
        f = u & (r - 1)
        s = f ^ (1 + ((np.uint64(r - 1) * u) >> np.uint64(32)))
        n = min(8, k - 8 * i)
        assert np.array_equal(first[8 * i:8 * i + n], f[:n]) and np.array_equal(second[8 * i:8 * i + n], s[:n])


def test_noise_distributions():
    """The noise rules' distributions at large counts (reference.py:74-93): E = (byte & 63) - 32 takes
    each of the 64 values in [-32, 31] equally often, and the pair rule gives a uniform first index
    and a uniform nonzero XOR distance first ^ second in [1, r - 1]. A wrong mask, offset or pair
    formula (e.g. byte % 63, or second = first + 1 + ...) fails the chi-square bounds (p < 1e-6)."""
    key = bytes(range(7, 39))
    E = O.uniform_matrix(O.SEED_LABEL_A, key, 4096, 64).ravel()
    cnt = np.bincount(E.astype(np.int64) + 32, minlength=64)
    assert cnt.size == 64 and cnt.min() > 0
    exp = E.size / 64
    assert ((cnt - exp) ** 2 / exp).sum() < 140  # chi-square, 63 dof: p ~ 1e-7 at 140
    for r in (64, 128):
        P = O.perm_packed(O.SEED_LABEL_B, key, 1 << 18, r)
        first, second = (P & 0xFFFF).astype(np.int64), (P >> 16).astype(np.int64)
        cf = np.bincount(first, minlength=r)
        dist = np.bincount(first ^ second, minlength=r)
        assert cf.size == r and dist[0] == 0 and dist.size == r
        e1, e2 = first.size / r, first.size / (r - 1)
        lim = r - 1 + 7 * np.sqrt(2 * (r - 1))  # mean + 7 sd of chi-square with r - 1 dof
        assert ((cf - e1) ** 2 / e1).sum() < lim
        assert ((dist[1:] - e2) ** 2 / e2).sum() < lim


def test_scale_bf16_against_torch_cast():
    """The OUT_BF16 epilogue (kernels.cu:440-445, 687-704): f32(acc) * a_scale * b_scale, each
    product rounded to fp32, then to bf16 by round-to-nearest-even. Pinned by torch's own
    fp32 -> bf16 conversion of the same fp32 products, on random values and on exact ties (low 16
    bits 0x8000) with the kept bit 0 and 1, both signs."""
    import torch
    rng = np.random.default_rng(16)
    m, n = 64, 512
    acc = rng.integers(-2 ** 31, 2 ** 31, size=(m, n), dtype=np.int64).astype(np.int32)
    ties = np.array([2 ** 24 + 2 ** 16, 2 ** 24 + 2 ** 17 + 2 ** 16, 2 ** 23 + 2 ** 15, 2 ** 23 + 2 ** 16 + 2 ** 15,
                     2 ** 30 + 2 ** 22, 2 ** 30 + 2 ** 23 + 2 ** 22], np.int64)
    acc[0, :len(ties)] = ties
    acc[0, len(ties):2 * len(ties)] = -ties
    a_scale = rng.uniform(1e-4, 2.0, m).astype(np.float32)
    b_scale = rng.uniform(1e-4, 2.0, n).astype(np.float32)
    a_scale[0] = 1.0
    b_scale[:2 * len(ties)] = 1.0
    f = (acc.astype(np.float32) * a_scale[:, None]) * b_scale[None, :]
    assert ((f[0, :2 * len(ties)].view(np.uint32) & 0xFFFF) == 0x8000).all()
    want = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.scale_bf16(acc, a_scale, b_scale), want)


def test_noise_apply_and_projection_brute_force():
    rng = np.random.default_rng(3)
    rows, k, r = 16, 256, 64
    A = rng.integers(-128, 128, size=(rows, k), dtype=np.int8)
    E = rng.integers(-32, 32, size=(rows, r), dtype=np.int8)
    P = O.perm_packed(O.SEED_LABEL_A, b"\x01" * 32, k, r)
    f, s = (P & 0xFFFF).astype(np.int64), (P >> 16).astype(np.int64)
    want = (A.astype(np.int64) + E[:, f] - E[:, s]) & 0xFF
    assert np.array_equal(O.noise_apply(A, E, P).view(np.uint8), want.astype(np.uint8))
    S = np.zeros((r, k), np.int64)
    S[f, np.arange(k)] += 1
    S[s, np.arange(k)] -= 1
    assert np.array_equal(O.project(A, P, r), A.astype(np.int64) @ S.T)


def test_limbs_reconstruct_and_limb_count():
    rng = np.random.default_rng(4)
    k = 4096
    L = O.limbs_for(k)
    proj = rng.integers(-127 * k, 127 * k + 1, size=(8, 64)).astype(np.int32)
    proj[0, 0], proj[0, 1] = 127 * k, -127 * k
    corr = np.zeros((L, 8, 128), np.int8)
    O.write_limbs(proj, corr, 64)
    c = corr[:, :, 64:].astype(np.int64)
    assert c.min() >= -64 and c.max() <= 63
    assert np.array_equal(sum(c[i] * 128 ** i for i in range(L)), proj)
    assert not corr[:, :, :64].any()
    for mx, want in ((0, 1), (63, 1), (64, 2), (8127, 2), (8128, 3), (1040319, 3), (1040320, 4)):
        assert O.limbs_needed(mx) == want


# ------------------------------------------------------------------ GEMM and transcript
def test_gemm_known_answer_L1():
    """results/xc_cpu.json:4 (miner/ampere/bench/crosscheck.py:62-76)."""
    rng = np.random.default_rng(2026)
    A = rng.integers(-64, 65, size=(1024, 4096), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(3072, 4096), dtype=np.int8)
    C = O.igemm(A, Bt)
    assert hashlib.sha256(C.tobytes()).hexdigest()[:20] == "bf9394d180bda5b0412c"


def l2_quantizer_input() -> np.ndarray:
    """The L2 quantizer input of miner/ampere/bench/crosscheck.py:62-91: drawn from
    default_rng(2026) after the L1 operands, rounded to bf16 (round to nearest even, as torch's
    fp32 -> bf16 conversion) and widened back to fp32."""
    rng = np.random.default_rng(2026)
    rng.integers(-64, 65, size=(1024, 4096), dtype=np.int8)
    rng.integers(-64, 65, size=(3072, 4096), dtype=np.int8)
    x = rng.standard_normal((1024, 4096)).astype(np.float32) * np.linspace(0.05, 6, 4096, dtype=np.float32)
    x[:, 7] *= 40.0
    u = x.view(np.uint32)
    b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    return (b << 16).view(np.float32)


# sha256[:20] of (int8 q, fp32 scale) of the miner's quantizer on that input: results/xc_cpu.json:5-10,
# the same in results/xc_3080.json and results/xc_5090.json
L2_KAT = {0: ("ce0b9f970855d5565ecc", "c15f21b56e165b4e76b7"),
          128: ("440e431806f833e22989", "b11bb63a72dfee572c80"),
          512: ("c51b454f3687cd02109f", "66c49428583d960017f2")}


@pytest.mark.parametrize("bs", [0, 128, 512])
def test_quantizer_known_answers_L2(bs):
    """quant_rows_had (kernels.cu:717-778) = quant_act with qmax 64 on the widened bf16 rows."""
    q, s = O.quant_act(l2_quantizer_input(), bs, 64)
    assert hashlib.sha256(q.tobytes()).hexdigest()[:20] == L2_KAT[bs][0]
    assert hashlib.sha256(s.tobytes()).hexdigest()[:20] == L2_KAT[bs][1]


def test_gemm_ragged_and_extremes():
    rng = np.random.default_rng(5)
    for m, n, k in ((1, 1, 1), (3, 70, 130), (65, 1, 257)):
        A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
        B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
        assert np.array_equal(O.igemm(A, B), (A.astype(np.int64) @ B.astype(np.int64).T).astype(np.int32))
    A = np.full((2, 4096), -128, np.int8)
    assert O.igemm(A, A)[0, 0] == 128 * 128 * 4096
    # int32 accumulation wraps mod 2^32 like the reference's .astype(np.int32)
    A = np.full((1, 2 ** 18 + 64), -128, np.int8)
    assert O.igemm(A, A)[0, 0] == np.int64(128 * 128 * (2 ** 18 + 64)).astype(np.int32)


def _transcript_brute(Ap, Bp, r):
    """Per tile, straight from the definition: cumulative sums of exactly its 128 elements."""
    m, k = Ap.shape
    n = Bp.shape[0]
    out = np.zeros((m // 64, 8, n // 64, 4, 16), np.uint32)
    for rb in range(m // 64):
        for cb in range(n // 64):
            for g in range(8):
                for t in range(4):
                    rows = [rb * 64 + g + 8 * i for i in range(8)]
                    cols = sorted(cb * 64 + 2 * t + e + 8 * j for j in range(8) for e in (0, 1))
                    a = Ap[rows].astype(np.int64)
                    b = Bp[cols].astype(np.int64)
                    msg = [0] * 16
                    for c in range(k // r):
                        acc = a[:, :(c + 1) * r] @ b[:, :(c + 1) * r].T
                        x = 0
                        for v in (acc & 0xFFFFFFFF).ravel():
                            x ^= int(v)
                        s = c % 16
                        msg[s] = (((msg[s] << 13) | (msg[s] >> 19)) & 0xFFFFFFFF) ^ x
                    out[rb, g, cb, t] = msg
    return out


@pytest.mark.parametrize("k,r", [(128, 64), (1280, 64), (256, 128)])
def test_transcript_brute_force(k, r):
    # k = 1280, r = 64: 20 folds, so slots wrap past 16 and rotate twice
    rng = np.random.default_rng(k + r)
    Ap = rng.integers(-127, 128, size=(128, k), dtype=np.int8)
    Bp = rng.integers(-127, 128, size=(64, k), dtype=np.int8)
    assert np.array_equal(O.transcript(Ap, Bp, r), _transcript_brute(Ap, Bp, r))


def test_tile_hash_and_winner_rule():
    key = bytes(range(32))
    msgs = np.arange(2 * 8 * 1 * 4 * 16, dtype=np.uint32).reshape(2, 8, 1, 4, 16)
    dig = O.tile_hashes(msgs, key)
    for idx in [(0, 0, 0, 0), (1, 7, 0, 3)]:
        want = py_b3(O.to_bytes(msgs[idx]), key)
        assert O.to_bytes(dig[idx]) == want
    # a target at one digest's value: exactly that tile and the smaller ones win
    d = dig.reshape(-1, 8)
    vals = [int.from_bytes(O.to_bytes(x), "little") for x in d]
    tgt = sorted(vals)[5]
    target = np.array([(tgt >> (32 * i)) & 0xFFFFFFFF for i in range(8)], np.uint32)
    assert len(O.winners(dig, target)) == 6


def test_mined_forward_denoise_exact():
    """(A + EAL S_A)(Bt + EBRt S_B)^T minus the limb correction is A @ Bt^T exactly."""
    rng = np.random.default_rng(7)
    m, n, k, r = 128, 128, 1024, 64
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    res = O.mined_forward(A, Bt, rng.bytes(32), O.bound_for_wins(m, n, 12), r)
    assert np.array_equal(res["out"], O.igemm(A, Bt))
    # the correction rebuilt from the limb tensors equals the one from the projections
    L = res["corrA"].shape[0]
    corr = sum((res["corrA"][li].astype(np.int64) @ res["corrB"][li].astype(np.int64).T) * 128 ** li for li in range(L))
    noisy = O.igemm(res["ApEA"], res["BpEBt"]).astype(np.int64)
    assert np.array_equal(((noisy - corr) & 0xFFFFFFFF).astype(np.uint32).view(np.int32), res["out"])
    assert 0 < len(res["winners"]) < 64
    # the composed denoise (limb count from maxabs, Horner over limbs) gives the same exact product
    assert np.array_equal(O.denoise(noisy, res["corrA"], res["corrB"], res["maxabs"]), res["out"])


@pytest.mark.parametrize("L", [1, 2, 3, 4])
def test_denoise_every_limb_count_closed_form(L):
    """O.denoise (kernels.cu:598-673) at each limb count: projections X, Y whose max |value| lands
    in limb range L, written as balanced base-128 limbs beside noise copies E_A, E_B, make the
    denoise equal the closed form noisy - X E_B^T - E_A Y^T exactly. A limb count one too small,
    or Horner shifts of 6 instead of 7, breaks it (a dropped limb or a wrong radix fails here)."""
    rng = np.random.default_rng(40 + L)
    m, n, r = 64, 96, 64
    caps = (63, 8127, 1040319, 127 * 262144)
    lo, hi = (0, *caps[:3])[L - 1], caps[L - 1]
    X = rng.integers(-hi, hi + 1, size=(m, r)).astype(np.int32)
    Y = rng.integers(-hi, hi + 1, size=(n, r)).astype(np.int32)
    X[3, 5] = hi  # max |X| in (lo, hi]: exactly L limbs
    assert lo < np.abs(X).max() <= hi and np.abs(Y).max() <= hi
    EA = rng.integers(-32, 32, size=(m, r), dtype=np.int8)
    EB = rng.integers(-32, 32, size=(n, r), dtype=np.int8)
    corrA = np.zeros((4, m, 2 * r), np.int8)
    corrB = np.zeros((4, n, 2 * r), np.int8)
    O.write_limbs(X, corrA, 0)
    O.write_limbs(Y, corrB, r)
    corrA[:, :, r:] = EA
    corrB[:, :, :r] = EB
    noisy = rng.integers(-2 ** 31, 2 ** 31, size=(m, n)).astype(np.int64)
    mx = np.array([np.abs(X).max(), np.abs(Y).max()], np.int32)
    want = noisy - X.astype(np.int64) @ EB.astype(np.int64).T - EA.astype(np.int64) @ Y.astype(np.int64).T
    want = (want & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    assert O.limbs_needed(int(mx.max())) == L
    assert np.array_equal(O.denoise(noisy, corrA, corrB, mx), want)
    if L > 1:
        assert not np.array_equal(O.denoise(noisy, corrA, corrB, mx, lmax=L - 1), want)
        # a wrong radix in the Horner step
        bad = np.zeros((m, n), np.int64)
        for li in range(L - 1, -1, -1):
            bad = (bad << 6) + corrA[li].astype(np.int64) @ corrB[li].astype(np.int64).T
        assert not np.array_equal(((noisy - bad) & 0xFFFFFFFF).astype(np.uint32).view(np.int32), want)


# ------------------------------------------------------------------ detrt golden fixtures
FIXTURES = ["detrt_tiny_qwen3", "detrt_tiny_llama", "detrt_qwen3_1p7b"]


@pytest.mark.parametrize("name", FIXTURES)
def test_quant_act_fixtures(name):
    """Go-referee fixtures (chain/patches/0003, 0021): N1->QA1, O->QA2, N2->QA3, SM->QA4."""
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    Bs = int(z["cfg"][5])
    n = 0
    for l in (0, 1):
        for src, qa in (("N1", "QA1"), ("O", "QA2"), ("N2", "QA3"), ("SM", "QA4")):
            x = z[f"l{l}_{src}"]
            q, s = O.quant_act(x, O.hadamard_bs(Bs, x.shape[1]))
            assert np.array_equal(q, z[f"l{l}_{qa}_q"]), (name, l, qa)
            assert np.array_equal(s.view(np.uint32), z[f"l{l}_{qa}_s"].view(np.uint32)), (name, l, qa)
            n += x.shape[0]
    assert n >= 64


@pytest.mark.parametrize("name", FIXTURES)
def test_linear_element_rule_fixtures(name):
    """QA x W -> (f32(acc) * s_x) * s_w equals the referee's linearElem bit for bit."""
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    for l in (0, 1):
        for lin, qa, op in (("qkv", "QA1", "QKV"), ("o", "QA2", "OP"), ("gu", "QA3", "GU"), ("down", "QA4", "DN")):
            acc = O.igemm(z[f"l{l}_{qa}_q"], z[f"l{l}_W_{lin}_q"])
            y = O.dequant(acc, z[f"l{l}_{qa}_s"], z[f"l{l}_W_{lin}_s"])
            assert np.array_equal(y.view(np.uint32), z[f"l{l}_{op}"].view(np.uint32)), (name, l, lin)


def test_dequant_order_matters():
    # (acc * sx) * sw and acc * (sx * sw) differ for some inputs: the fixture test above would
    # catch a reassociated product; show that such inputs exist
    rng = np.random.default_rng(9)
    acc = rng.integers(-2 ** 20, 2 ** 20, size=(64, 64)).astype(np.int32)
    sx = rng.random(64).astype(np.float32)
    sw = rng.random(64).astype(np.float32)
    y = O.dequant(acc, sx, sw)
    alt = (acc.astype(np.float32) * (sx[:, None] * sw[None, :]).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(y, alt)
