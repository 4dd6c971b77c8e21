"""GPU parity of the cuPOW miner path (libuwc_hip.so through uwc_amd.ops) against the CPU oracle:
bit-exact commitment, noise, noising/projections, every tile's message and digest, the winner
set, and the exact denoised output. Mirrors miner/ampere/tests/test_kernels.py,
test_gemm_cfgs.py and test_proj_gemm.py."""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def _ops():
    from uwc_amd import ops
    return ops


def _u32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("nchunks", [1, 2, 3, 63, 64, 65, 130, 1000, 4097, 65536, 65537, 300_001])
def test_tree_hash_matches_oracle(dev, nchunks):
    ops = _ops()
    rng = np.random.default_rng(nchunks)
    data = rng.integers(0, 256, size=nchunks * 1024, dtype=np.uint8)
    key = rng.bytes(32)
    root = torch.zeros(8, dtype=torch.int32, device=dev)
    ops.b3_root_and_seed(torch.from_numpy(data).to(dev), ops.words(key), root_out=root)
    assert ops.words_to_bytes(root) == O.b3(data.tobytes(), key)


def test_seed_derivation_matches_oracle(dev):
    ops = _ops()
    rng = np.random.default_rng(1)
    m, n, k = 256, 512, 2048
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    job_key = rng.bytes(32)
    a_seed, b_seed, _, _ = O.commitment(job_key, A, Bt)
    jk = ops.words(job_key)
    bs = torch.zeros(8, dtype=torch.int32, device=dev)
    ops.b3_root_and_seed(torch.from_numpy(Bt).to(dev).view(-1), jk, prefix=jk, salt=ops.SALT_B.to(dev), dim=n, seed_out=bs)
    assert ops.words_to_bytes(bs) == b_seed
    as_ = torch.zeros(8, dtype=torch.int32, device=dev)
    ops.b3_root_and_seed(torch.from_numpy(A).to(dev).view(-1), jk, prefix=bs, salt=ops.SALT_A.to(dev), dim=m, seed_out=as_)
    assert ops.words_to_bytes(as_) == a_seed


@pytest.mark.parametrize("count,nchunks", [(1, 65), (3, 1), (5, 130), (16, 64), (4, 4097), (2, 65537), (32, 2049),
                                           (4, 16384), (8, 8193)])
def test_batched_commitment_matches_oracle(dev, count, nchunks):
    """b3_root_and_seed_many: every item's root and salted seed equal the oracle's (and the
    single-input entry point's), whatever the batch size and tree shape; from 65536 chunks per
    launch on (the last three cases and (2, 65537)) the chunks go one per lane, 256 per workgroup,
    with a partial last workgroup in all but (4, 16384)."""
    ops = _ops()
    rng = np.random.default_rng(count * 1000 + nchunks)
    datas = [rng.integers(0, 256, size=nchunks * 1024, dtype=np.uint8) for _ in range(count)]
    key, prefix = rng.bytes(32), rng.bytes(32)
    salt = ops.SALT_A.to(dev)
    roots = [torch.zeros(8, dtype=torch.int32, device=dev) for _ in range(count)]
    seeds = [torch.zeros(8, dtype=torch.int32, device=dev) for _ in range(count)]
    ops.b3_root_and_seed_many([torch.from_numpy(d).to(dev) for d in datas], ops.words(key), prefix=ops.words(prefix),
                              salt=salt, dim=nchunks, root_outs=roots, seed_outs=seeds)
    for d, root, seed in zip(datas, roots, seeds):
        want = O.b3(d.tobytes(), key)
        assert ops.words_to_bytes(root) == want
        one = torch.zeros(8, dtype=torch.int32, device=dev)
        ops.b3_root_and_seed(torch.from_numpy(d).to(dev), ops.words(key), prefix=ops.words(prefix), salt=salt,
                             dim=nchunks, seed_out=one)
        assert ops.words_to_bytes(seed) == ops.words_to_bytes(one)
    # the seed itself against the oracle's derivation: BLAKE3(prefix || keyed(salt, root || dim || 0^28))
    assert ops.words_to_bytes(seeds[-1]) == O.b3(prefix + O.bind_root(want, nchunks, O.SEED_SALT_A))


@pytest.mark.parametrize("count,rows,k,r", [(4, 256, 4096, 64), (3, 128, 1000, 128), (16, 32, 8, 64)])
def test_batched_nonce_noise_matches_single(dev, count, rows, k, r):
    """nonce_noise_many: item i equals nonce_noise with key i (E, P, St, SpT, zeroed counters)."""
    ops = _ops()
    rng = np.random.default_rng(count + rows + k + r)
    keys = [ops.words(rng.bytes(32)) for _ in range(count)]
    lab = ops.LABEL_A.to(dev)

    def bufs():
        return dict(E=torch.empty((rows, r), dtype=torch.int8, device=dev), P=torch.empty(k, dtype=torch.int32, device=dev),
                    St=torch.full((r, k), 5, dtype=torch.int8, device=dev),
                    SpT=torch.full((k, 64), 5, dtype=torch.int8, device=dev) if r <= 64 else None,
                    z0=torch.full((2,), 9, dtype=torch.int32, device=dev),
                    z1=torch.full((3,), 9, dtype=torch.int32, device=dev))
    many = [bufs() for _ in range(count)]
    ops.nonce_noise_many([b["E"] for b in many], [b["P"] for b in many], k, r, lab, keys, Sts=[b["St"] for b in many],
                         zero0s=[b["z0"] for b in many], zero1s=[b["z1"][:1] for b in many],
                         SpTs=[b["SpT"] for b in many] if r <= 64 else None)
    for key, b in zip(keys, many):
        one = bufs()
        ops.nonce_noise(one["E"], one["P"], k, r, lab, key, St=one["St"], zero0=one["z0"], zero1=one["z1"][:1],
                        SpT=one["SpT"])
        for name in ("E", "P", "St", "SpT", "z0", "z1"):
            if one[name] is not None:
                assert torch.equal(b[name], one[name]), name
        assert b["z0"].cpu().tolist() == [0, 0] and b["z1"].cpu().tolist() == [0, 9, 9]
    assert np.array_equal(many[0]["E"].cpu().numpy(), O.uniform_matrix(O.SEED_LABEL_A, ops.words_to_bytes(keys[0]), rows, r))


@pytest.mark.parametrize("r", [64, 128])
def test_noise_generation_matches_oracle(dev, r):
    ops = _ops()
    rng = np.random.default_rng(2)
    key = rng.bytes(32)
    rows, k = 256, 3072 + 5
    E = torch.empty((rows, r), dtype=torch.int8, device=dev)
    zero = torch.full((3,), 7, dtype=torch.int32, device=dev)
    ops.noise_uniform(E, ops.LABEL_A.to(dev), ops.words(key), zero_me=zero, zero_n=2)
    assert np.array_equal(E.cpu().numpy(), O.uniform_matrix(O.SEED_LABEL_A, key, rows, r))
    assert zero.cpu().tolist() == [0, 0, 7]
    P = torch.empty(k, dtype=torch.int32, device=dev)
    ops.noise_perm(P, k, r, ops.LABEL_B.to(dev), ops.words(key))
    assert np.array_equal(_u32(P), O.perm_packed(O.SEED_LABEL_B, key, k, r))


@pytest.mark.parametrize("rows,k,r", [(128, 2048, 128), (8, 4, 64), (24, 1000, 64), (16, 4100, 128), (64, 4096, 16)])
def test_noise_rows_noising_and_projection(dev, rows, k, r):
    """The general-shape operand pass (rows % 8, k % 4): noised rows, projection limbs, the E copy
    and max |projection| against the oracle; a second call with only the projection and maxabs
    (the B side of the LDS-atomic path) gives the same limbs."""
    ops = _ops()
    rng = np.random.default_rng(3 + rows + k + r)
    A = rng.integers(-64, 65, size=(rows, k), dtype=np.int8)
    E = rng.integers(-32, 32, size=(rows, r), dtype=np.int8)
    Pn = O.perm_packed(O.SEED_LABEL_A, b"\x01" * 32, k, r)
    Pp = O.perm_packed(O.SEED_LABEL_B, b"\x02" * 32, k, r)
    pack = lambda P: torch.from_numpy(P.view(np.int32).copy()).to(dev)
    dst = torch.empty((rows, k), dtype=torch.int8, device=dev)
    L = ops.limbs_for(k)
    corr = torch.zeros((L, rows, 2 * r), dtype=torch.int8, device=dev)
    mx = torch.zeros(1, dtype=torch.int32, device=dev)
    Ad = torch.from_numpy(A).to(dev)
    ops.noise_rows(Ad, rows, k, r, E=torch.from_numpy(E).to(dev), Pn=pack(Pn), dst=dst, Pp=pack(Pp), corr=corr,
                   corr_off=0, ecopy_off=r, maxabs=mx)
    assert np.array_equal(dst.cpu().numpy(), O.noise_apply(A, E, Pn))
    proj = O.project(A, Pp, r)
    want = np.zeros((L, rows, 2 * r), np.int8)
    O.write_limbs(proj, want, 0)
    for li in range(L):
        want[li, :, r:] = E
    assert np.array_equal(corr.cpu().numpy(), want)
    assert int(mx.item()) == int(np.abs(proj).max())
    corr2 = torch.zeros_like(corr)
    mx2 = torch.full((1,), 3, dtype=torch.int32, device=dev)
    ops.noise_rows(Ad, rows, k, r, Pp=pack(Pp), corr=corr2, corr_off=r, maxabs=mx2)
    want2 = np.zeros((L, rows, 2 * r), np.int8)
    O.write_limbs(proj, want2, r)
    assert np.array_equal(corr2.cpu().numpy(), want2)
    assert int(mx2.item()) == max(3, int(np.abs(proj).max()))


@pytest.mark.parametrize("m,n,k,r", [(128, 128, 1024, 64), (256, 256, 2048, 64), (256, 384, 2048, 128),
                                     (128, 256, 1280, 64)])
def test_mined_forward_exact_and_every_tile_matches(dev, m, n, k, r):
    """Full per-call path: output == A @ Bt^T exactly; every tile's 16-word message and digest
    and the winner set equal the oracle's (miner/ampere/tests/test_kernels.py:94-125)."""
    ops = _ops()
    rng = np.random.default_rng(m + n + k + r)
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    job_key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 12)
    ref = O.mined_forward(A, Bt, job_key, target, r)

    w = ops.MinedWeight(Bt=torch.from_numpy(Bt).to(dev), b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(job_key, target)
    dump = torch.zeros((m // 64) * 8 * (n // 64) * 4 * ops.DUMP_WORDS, dtype=torch.int32, device=dev)
    out = w._forward(torch.from_numpy(A).to(dev), torch.ones(m, device=dev), None, ops.OUT_I32, True, dump=dump)
    b = w._buf(m)
    assert ops.words_to_bytes(w.b_seed) == ref["b_seed"]
    assert ops.words_to_bytes(b["a_seed"]) == ref["a_seed"]
    assert np.array_equal(w.EBRt.cpu().numpy(), ref["EBRt"]) and np.array_equal(_u32(w.PB), ref["PB"])
    assert np.array_equal(w.BpEBt.cpu().numpy(), ref["BpEBt"])
    assert np.array_equal(b["EAL"].cpu().numpy(), ref["EAL"]) and np.array_equal(_u32(b["PA"]), ref["PA"])
    assert np.array_equal(b["ApEA"].cpu().numpy(), ref["ApEA"])
    assert np.array_equal(b["corrA"].cpu().numpy(), ref["corrA"])
    assert np.array_equal(w.corrB.cpu().numpy(), ref["corrB"])
    assert np.array_equal(b["maxabs"].cpu().numpy(), ref["maxabs"])
    d = _u32(dump).reshape(m // 64, 8, n // 64, 4, ops.DUMP_WORDS)
    assert np.array_equal(d[..., :16], ref["msgs"]), "tile messages differ"
    assert np.array_equal(d[..., 16:], ref["digests"]), "tile digests differ"
    assert np.array_equal(out.cpu().numpy(), ref["out"]), "denoised output is not the exact product"
    got = set(w.winners(m))
    assert ref["winners"] and got == ref["winners"]


def test_noise_mine_matches_and_out_modes(dev):
    """noise_mine (hash only) gives the same winners; bf16 / fp32 epilogues match the oracle."""
    ops = _ops()
    rng = np.random.default_rng(11)
    m, n, k, r = 256, 256, 1024, 64
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    job_key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 12)
    ref = O.mined_forward(A, Bt, job_key, target, r)
    w = ops.MinedWeight(Bt=torch.from_numpy(Bt).to(dev), b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(job_key, target)
    Ad = torch.from_numpy(A).to(dev)
    w.noise_mine(Ad)
    assert set(w.winners(m)) == ref["winners"]
    a_scale = torch.from_numpy(rng.random(m).astype(np.float32) * 0.01).to(dev)
    w.b_scale = torch.from_numpy(rng.random(n).astype(np.float32) * 0.01).to(dev)
    yb = w.forward(Ad, a_scale, out_mode=ops.OUT_BF16)
    assert set(w.winners(m)) == ref["winners"]
    want = O.scale_bf16(ref["out"], a_scale.cpu().numpy(), w.b_scale.cpu().numpy())
    assert np.array_equal(yb.view(torch.int16).cpu().numpy().view(np.uint16), want)
    yf = w.forward(Ad, a_scale, out_mode=ops.OUT_F32)
    wf = O.dequant(ref["out"], a_scale.cpu().numpy(), w.b_scale.cpu().numpy())
    assert np.array_equal(yf.cpu().numpy().view(np.uint32), wf.view(np.uint32))


def test_graphed_forward_matches_eager_every_replay(dev):
    ops = _ops()
    rng = np.random.default_rng(5)
    m, n, k = 256, 512, 2048
    Bt = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8)).to(dev)
    w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=128, max_wins=4096)
    w.setup_block(rng.bytes(32), O.bound_for_wins(m, n, 20))
    gf = ops.GraphedForward(w, m, out_mode=ops.OUT_I32)
    for rep in range(3):
        A = torch.from_numpy(rng.integers(-64, 65, size=(m, k), dtype=np.int8)).to(dev)
        gf.A.copy_(A)
        got = gf().clone()
        torch.cuda.synchronize()
        wins_graph = sorted(w.winners(m))
        eager = w.forward(A, torch.ones(m, device=dev), out_mode=ops.OUT_I32)
        torch.cuda.synchronize()
        assert torch.equal(got, eager), rep
        assert torch.equal(got.cpu(), torch.from_numpy(O.igemm(A.cpu().numpy(), Bt.cpu().numpy()))), rep
        assert wins_graph == sorted(w.winners(m)), rep


def test_win_records_capped(dev):
    """More winners than max_wins: the count keeps growing, records stop at the cap."""
    ops = _ops()
    rng = np.random.default_rng(12)
    m, n, k, r = 128, 128, 512, 64
    A = torch.from_numpy(rng.integers(-64, 65, size=(m, k), dtype=np.int8)).to(dev)
    B = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8)).to(dev)
    key = ops.words(rng.bytes(32))
    target = torch.full((8,), -1, dtype=torch.int32, device=dev)  # every tile wins
    wins = torch.zeros(1 + 5 * ops.WIN_WORDS, dtype=torch.int32, device=dev)
    ops.gemm(A, B, r=r, flags=ops.FLAG_HASH, key=key, target=target, wins=wins, max_wins=5)
    w = _u32(wins)
    assert w[0] == (m // 8) * (n // 16)
    recs = w[1:].reshape(5, ops.WIN_WORDS)
    assert all(rr[0] % 64 < 8 and rr[1] % 2 == 0 for rr in recs)


@pytest.mark.parametrize("r", [64, 128])
def test_proj_matrix_project_and_noise_project(dev, r):
    """The matrix-core projection path (proj_matrix + project / noise_project) against the oracle."""
    ops = _ops()
    rng = np.random.default_rng(31 + r)
    rows, k = 96, 1536
    A = rng.integers(-64, 65, size=(rows, k), dtype=np.int8)
    E = rng.integers(-32, 32, size=(rows, r), dtype=np.int8)
    Pn = O.perm_packed(O.SEED_LABEL_A, b"\x05" * 32, k, r)
    Pp = O.perm_packed(O.SEED_LABEL_B, b"\x06" * 32, k, r)
    pack = lambda P: torch.from_numpy(P.view(np.int32).copy()).to(dev)
    St = ops.proj_matrix(pack(Pp), k, r)
    S = np.zeros((r, k), np.int64)
    S[(Pp & 0xFFFF).astype(np.int64), np.arange(k)] += 1
    S[(Pp >> 16).astype(np.int64), np.arange(k)] -= 1
    assert np.array_equal(St.cpu().numpy().astype(np.int64), S)
    L = ops.limbs_for(k)
    proj = O.project(A, Pp, r)
    Ad = torch.from_numpy(A).to(dev)
    corr = torch.zeros((L, rows, 2 * r), dtype=torch.int8, device=dev)
    mx = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.project(Ad, St, corr, r, mx)
    want = np.zeros((L, rows, 2 * r), np.int8)
    O.write_limbs(proj, want, r)
    assert np.array_equal(corr.cpu().numpy(), want)
    assert int(mx.item()) == int(np.abs(proj).max())
    # fused noising + projection + E copy
    dst = torch.empty_like(Ad)
    corr2 = torch.zeros_like(corr)
    mx2 = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.noise_project(Ad, rows, k, r, E=torch.from_numpy(E).to(dev), Pn=pack(Pn), dst=dst, St=St, corr=corr2, corr_off=0,
                      ecopy_off=r, maxabs=mx2)
    assert np.array_equal(dst.cpu().numpy(), O.noise_apply(A, E, Pn))
    want2 = np.zeros((L, rows, 2 * r), np.int8)
    O.write_limbs(proj, want2, 0)
    for li in range(L):
        want2[li, :, r:] = E
    assert np.array_equal(corr2.cpu().numpy(), want2)
    assert int(mx2.item()) == int(np.abs(proj).max())


@pytest.mark.parametrize("m,n,k,r", [(128, 192, 1536, 64), (64, 32, 4096, 64), (256, 128, 768, 16),
                                     (96, 64, 256, 32)])
def test_side_project_matches_oracle(dev, m, n, k, r):
    """One launch for the operand side: ApEA (noise on the matrix cores from SpA), X limbs + EAL
    copy (corrA), Y limbs (corrB) and both maxima equal the oracle (1 to 16 chunks of 256
    columns); maxabs is an atomic max into what the buffer held; a second call gives the same
    bytes."""
    ops = _ops()
    rng = np.random.default_rng(m * 7 + n + k + r)
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    Bp = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    E = rng.integers(-32, 32, size=(m, r), dtype=np.int8)
    PA = O.perm_packed(O.SEED_LABEL_A, rng.bytes(32), k, r)
    PB = O.perm_packed(O.SEED_LABEL_B, rng.bytes(32), k, r)
    pack = lambda P: torch.from_numpy(P.view(np.int32).copy()).to(dev)
    L = ops.limbs_for(k)
    StA, StB = ops.proj_matrix(pack(PA), k, r), ops.proj_matrix(pack(PB), k, r)
    SpA = torch.zeros((k, 64), dtype=torch.int8, device=dev)
    SpA[:, :r] = StA.t()
    X, Y = O.project(A, PB, r), O.project(Bp, PA, r)
    wantA = np.zeros((L, m, 2 * r), np.int8)
    O.write_limbs(X, wantA, 0)
    for li in range(L):
        wantA[li, :, r:] = E
    wantB = np.full((L, n, 2 * r), 7, np.int8)
    O.write_limbs(Y, wantB, r)
    Ad, Bd = torch.from_numpy(A).to(dev), torch.from_numpy(Bp).to(dev)
    for call in range(2):
        ApEA = torch.empty_like(Ad)
        corrA = torch.zeros((L, m, 2 * r), dtype=torch.int8, device=dev)
        corrB = torch.full((L, n, 2 * r), 7, dtype=torch.int8, device=dev)
        mx = torch.tensor([0, 3], dtype=torch.int32, device=dev)
        ops.side_project(Ad, torch.from_numpy(E).to(dev), SpA, ApEA, StB, corrA, Bd, StA, corrB, maxabs=mx,
                         corr_a_off=0, ecopy_off=r, corr_b_off=r)
        assert np.array_equal(ApEA.cpu().numpy(), O.noise_apply(A, E, PA)), call
        assert np.array_equal(corrA.cpu().numpy(), wantA), call
        assert np.array_equal(corrB.cpu().numpy(), wantB), call
        assert mx.cpu().tolist() == [int(np.abs(X).max()), max(3, int(np.abs(Y).max()))], call


def test_projection_paths_identical(dev):
    """The matrix-core projections leave the mined forward bit-identical to the LDS-atomic path:
    output, both correction tensors, maxabs and winning tiles (miner/ampere/tests/test_proj_gemm.py)."""
    ops = _ops()
    torch.manual_seed(0)
    for (n, k, m) in ((512, 2048, 128), (256, 1024, 384)):
        Bt = torch.randint(-64, 65, (n, k), dtype=torch.int8, device=dev)
        A = torch.randint(-64, 65, (m, k), dtype=torch.int8, device=dev)
        ones = torch.ones(m, dtype=torch.float32, device=dev)
        res = {}
        for mode in (False, True):
            w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=128, max_wins=4096)
            w.setup_block(bytes(range(32)), O.bound_for_wins(m, n, 12))
            out = w._forward(A, ones, None, ops.OUT_I32, True, None, mode)
            b = w._buf(m)
            res[mode] = (out.clone(), b["corrA"].clone(), w.corrB.clone(), b["maxabs"].clone(), sorted(w.winners(m)))
            assert torch.equal(out.cpu(), (A.cpu().long() @ Bt.cpu().long().t()).int())
        for name, x, y in zip(("out", "corrA", "corrB", "maxabs"), res[False][:4], res[True][:4]):
            assert torch.equal(x, y), (n, k, m, name)
        assert res[False][4] == res[True][4] and 0 < len(res[True][4])


@pytest.mark.parametrize("rows,k,r", [(256, 4096, 64), (128, 1000, 128), (32, 8, 64)])
def test_nonce_noise_fused_matches_oracle(dev, rows, k, r):
    """One launch: E as uniform_matrix, P as perm_matrix, St as the dense selection matrix,
    and both counter ranges zeroed."""
    ops = _ops()
    rng = np.random.default_rng(rows + k + r)
    key = rng.bytes(32)
    E = torch.empty((rows, r), dtype=torch.int8, device=dev)
    P = torch.empty(k, dtype=torch.int32, device=dev)
    St = torch.full((r, k), 5, dtype=torch.int8, device=dev)
    SpT = torch.full((k, 64), 5, dtype=torch.int8, device=dev) if r <= 64 else None
    z0 = torch.full((2,), 9, dtype=torch.int32, device=dev)
    z1 = torch.full((3,), 9, dtype=torch.int32, device=dev)
    ops.nonce_noise(E, P, k, r, ops.LABEL_A.to(dev), ops.words(key), St=St, zero0=z0, zero1=z1[:1], SpT=SpT)
    assert np.array_equal(E.cpu().numpy(), O.uniform_matrix(O.SEED_LABEL_A, key, rows, r))
    Pw = O.perm_packed(O.SEED_LABEL_A, key, k, r)
    assert np.array_equal(_u32(P), Pw)
    S = np.zeros((r, k), np.int64)
    S[(Pw & 0xFFFF).astype(np.int64), np.arange(k)] += 1
    S[(Pw >> 16).astype(np.int64), np.arange(k)] -= 1
    assert np.array_equal(St.cpu().numpy().astype(np.int64), S)
    if SpT is not None:  # the transpose as 64-byte rows, zero past r
        want = np.zeros((k, 64), np.int64)
        want[:, :r] = S.T
        assert np.array_equal(SpT.cpu().numpy().astype(np.int64), want)
    assert z0.cpu().tolist() == [0, 0] and z1.cpu().tolist() == [0, 9, 9]


@pytest.mark.parametrize("m,n,k,r", [(256, 256, 1024, 64), (512, 768, 2048, 128), (256, 512, 1280, 64)])
def test_tile_configs_identical(dev, m, n, k, r):
    """Every GEMM tiling gives the same mined result: exact output, the same tile messages and
    digests, the same winners (miner/ampere/tests/test_gemm_cfgs.py)."""
    ops = _ops()
    rng = np.random.default_rng(m * 3 + n + k + r)
    A = torch.from_numpy(rng.integers(-64, 65, size=(m, k), dtype=np.int8)).to(dev)
    Bt = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8)).to(dev)
    w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(rng.bytes(32), O.bound_for_wins(m, n, 12))
    ones = torch.ones(m, dtype=torch.float32, device=dev)
    ref = torch.from_numpy(O.igemm(A.cpu().numpy(), Bt.cpu().numpy()))
    got = {}
    for cfg in ops.CONFIGS:
        dump = torch.zeros((m // 64) * 8 * (n // 64) * 4 * ops.DUMP_WORDS, dtype=torch.int32, device=dev)
        out = w._forward(A, ones, None, ops.OUT_I32, True, cfg, True, dump=dump)
        assert torch.equal(out.cpu(), ref), (cfg, "output")
        got[cfg] = (sorted(w.winners(m)), dump.cpu())
    base = got["128x128"]
    assert 0 < len(base[0]) < w.max_wins
    for cfg, (wins, dump) in got.items():
        assert wins == base[0] and torch.equal(dump, base[1]), cfg


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (512, 256, 4096), (2048, 4096, 2048)])
def test_large_tile_plain_gemm(dev, m, n, k):
    ops, = (_ops(),)
    rng = np.random.default_rng(m + 7 * n + k)
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    C = ops.igemm_i32(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev))
    assert np.array_equal(C.cpu().numpy(), O.igemm(A, B))


@pytest.mark.parametrize("group,n_items", [(8, 5), (2, 5), (1, 3), (16, 17)])
def test_forward_many_grouped_equals_forward(dev, group, n_items):
    """forward_many (batched commitments and noise per group of nonces, then each nonce's
    projections and hashed GEMM) gives every nonce's output and winner set exactly as a
    sequential forward does; without per-item win buffers winners() reports the last item."""
    ops = _ops()
    rng = np.random.default_rng(77 + group)
    m, n, k, r = 256, 256, 1024, 64
    Bt = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8)).to(dev)
    job_key = rng.bytes(32)
    target = O.bound_for_wins(m, n, 8)
    w = ops.MinedWeight(Bt=Bt, b_scale=torch.ones(n, device=dev), r=r, max_wins=4096)
    w.setup_block(job_key, target)
    As = [torch.from_numpy(rng.integers(-64, 65, size=(m, k), dtype=np.int8)).to(dev) for _ in range(n_items)]
    ones = torch.ones(m, device=dev)
    ref = []
    for A in As:
        out = w.forward(A, ones, out_mode=ops.OUT_I32)
        torch.cuda.synchronize()
        ref.append((out.clone(), set(w.winners(m))))
    wins = [torch.zeros(1 + w.max_wins * ops.WIN_WORDS, dtype=torch.int32, device=dev) for _ in As]
    outs = w.forward_many(As, ones, out_mode=ops.OUT_I32, wins=wins, group=group)
    torch.cuda.synchronize()
    for i, (o, wb) in enumerate(zip(outs, wins)):
        assert torch.equal(o, ref[i][0]), i
        words = wb.cpu().numpy().view(np.uint32)
        cnt = min(int(words[0]), w.max_wins)
        recs = words[1:1 + cnt * ops.WIN_WORDS].reshape(cnt, ops.WIN_WORDS)
        got = {(int(x[0]), int(x[1]), x[2:].astype("<u4").tobytes()) for x in recs}
        assert got == ref[i][1], i
    assert any(len(x[1]) for x in ref)
    outs = w.forward_many(As, ones, out_mode=ops.OUT_I32, group=group)
    torch.cuda.synchronize()
    assert all(torch.equal(o, x[0]) for o, x in zip(outs, ref))
    assert set(w.winners(m)) == ref[-1][1]


@pytest.mark.parametrize("count,m,n,k,out_mode", [(3, 512, 512, 1024, 1), (17, 256, 512, 512, 1), (33, 256, 256, 512, 1),
                                                   (2, 256, 256, 1024, 2)])
def test_gemm_many_equals_single_calls(dev, count, m, n, k, out_mode):
    """gemm_many (hashed, denoised GEMMs sharing B: the split-role batched kernel for int32 outputs,
    one launch per item otherwise) gives every item's output and winner set exactly as its own
    gemm() call does, including batches longer than one launch."""
    ops = _ops()
    rng = np.random.default_rng(count * 7 + m + out_mode)
    r, L = 64, 2
    B = torch.from_numpy(rng.integers(-64, 65, size=(n, k), dtype=np.int8)).to(dev)
    As = [torch.from_numpy(rng.integers(-64, 65, size=(m, k), dtype=np.int8)).to(dev) for _ in range(count)]
    cAs = [torch.from_numpy(rng.integers(-64, 64, size=(L, m, 2 * r), dtype=np.int8)).to(dev) for _ in range(count)]
    cBs = [torch.from_numpy(rng.integers(-64, 64, size=(L, n, 2 * r), dtype=np.int8)).to(dev) for _ in range(count)]
    mxs = [torch.tensor([100 + i, 50], dtype=torch.int32, device=dev) for i in range(count)]
    keys = [ops.words(rng.bytes(32)) for _ in range(count)]
    target = torch.from_numpy(O.bound_for_wins(m, n, 6).astype(np.uint32).view(np.int32).copy()).to(dev)
    a_scale = torch.from_numpy(rng.random(m, dtype=np.float32)).to(dev)
    b_scale = torch.from_numpy(rng.random(n, dtype=np.float32)).to(dev)
    dt = {1: torch.int32, 2: torch.bfloat16}[out_mode]
    flags = ops.FLAG_HASH | ops.FLAG_DENOISE
    nw = 1 + 256 * ops.WIN_WORDS

    def winset(w):
        words = w.cpu().numpy().view(np.uint32)
        c = min(int(words[0]), 256)
        recs = words[1:1 + c * ops.WIN_WORDS].reshape(c, ops.WIN_WORDS)
        return {(int(x[0]), int(x[1]), x[2:].astype("<u4").tobytes()) for x in recs}

    outs = [torch.empty((m, n), dtype=dt, device=dev) for _ in range(count)]
    wins = [torch.zeros(nw, dtype=torch.int32, device=dev) for _ in range(count)]
    ops.gemm_many(As, B, r=r, flags=flags, corrAs=cAs, corrBs=cBs, maxabss=mxs, keys=keys, target=target, winss=wins,
                  max_wins=256, a_scale=a_scale, b_scale=b_scale, outs=outs, out_mode=out_mode)
    torch.cuda.synchronize()
    any_win = False
    for i in range(count):
        one = torch.empty((m, n), dtype=dt, device=dev)
        w1 = torch.zeros(nw, dtype=torch.int32, device=dev)
        ops.gemm(As[i], B, r=r, flags=flags, corrA=cAs[i], corrB=cBs[i], maxabs=mxs[i], key=keys[i], target=target,
                 wins=w1, max_wins=256, a_scale=a_scale, b_scale=b_scale, out=one, out_mode=out_mode)
        torch.cuda.synchronize()
        assert torch.equal(outs[i].view(torch.int16) if out_mode == 2 else outs[i],
                           one.view(torch.int16) if out_mode == 2 else one), i
        assert winset(wins[i]) == winset(w1), i
        any_win = any_win or bool(winset(w1))
    assert any_win


@pytest.mark.parametrize("count,m,n,k,r", [(3, 128, 256, 512, 64), (2, 256, 128, 384, 16), (5, 128, 128, 1152, 32),
                                           (8, 512, 384, 4096, 64)])
def test_side_project_many_matches_oracle(dev, count, m, n, k, r):
    """The batched operand side (one launch for a group of nonces sharing B'): every item's noised
    operand, X limbs + E copy, Y limbs and both maxima equal the oracle; maxabs is an atomic max
    into what each buffer held."""
    ops = _ops()
    rng = np.random.default_rng(count * 11 + m + n + k + r)
    Bp = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    PB = O.perm_packed(O.SEED_LABEL_B, rng.bytes(32), k, r)
    pack = lambda P: torch.from_numpy(P.view(np.int32).copy()).to(dev)
    StB = ops.proj_matrix(pack(PB), k, r)
    L = ops.limbs_for(k)
    items = []
    for i in range(count):
        A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
        E = rng.integers(-32, 32, size=(m, r), dtype=np.int8)
        PA = O.perm_packed(O.SEED_LABEL_A, rng.bytes(32), k, r)
        StA = ops.proj_matrix(pack(PA), k, r)
        SpA = torch.zeros((k, 64), dtype=torch.int8, device=dev)
        SpA[:, :r] = StA.t()
        items.append(dict(A=A, E=E, PA=PA, Ad=torch.from_numpy(A).to(dev), Ed=torch.from_numpy(E).to(dev), StA=StA,
                          SpA=SpA, ApEA=torch.empty((m, k), dtype=torch.int8, device=dev),
                          corrA=torch.zeros((L, m, 2 * r), dtype=torch.int8, device=dev),
                          corrB=torch.full((L, n, 2 * r), 7, dtype=torch.int8, device=dev),
                          mx=torch.tensor([0, 3], dtype=torch.int32, device=dev)))
    Bd = torch.from_numpy(Bp).to(dev)
    ops.side_project_many([it["Ad"] for it in items], [it["Ed"] for it in items], [it["SpA"] for it in items],
                          [it["ApEA"] for it in items], StB, [it["corrA"] for it in items], Bd,
                          [it["StA"] for it in items], [it["corrB"] for it in items],
                          maxabss=[it["mx"] for it in items], corr_a_off=0, ecopy_off=r, corr_b_off=r)
    torch.cuda.synchronize()
    for i, it in enumerate(items):
        X, Y = O.project(it["A"], PB, r), O.project(Bp, it["PA"], r)
        wantA = np.zeros((L, m, 2 * r), np.int8)
        O.write_limbs(X, wantA, 0)
        for li in range(L):
            wantA[li, :, r:] = it["E"]
        wantB = np.full((L, n, 2 * r), 7, np.int8)
        O.write_limbs(Y, wantB, r)
        assert np.array_equal(it["ApEA"].cpu().numpy(), O.noise_apply(it["A"], it["E"], it["PA"])), i
        assert np.array_equal(it["corrA"].cpu().numpy(), wantA), i
        assert np.array_equal(it["corrB"].cpu().numpy(), wantB), i
        assert it["mx"].cpu().tolist() == [int(np.abs(X).max()), max(3, int(np.abs(Y).max()))], i
