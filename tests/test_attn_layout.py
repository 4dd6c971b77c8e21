"""CPU emulation of the attention kernel's data movement (useful-work-coin_amd/csrc/uwc_attn.hip,
uwc_layer.hip's vt_pos): which key and query every lane and MFMA slot touches, and every load and
store address against its buffer. No GPU needed.

v_mfma_i32_16x16x64_i8 (gfx950): A is 16 rows x 64 k with lane l holding row l & 15 and k bytes
16 (l >> 4) .. + 16; B likewise with column l & 15; C lane l register i is row 4 (l >> 4) + i,
column l & 15. The kernel relies only on A and B using the same (lane group, slot) -> k map,
so the emulation below applies the product exactly that way."""
from __future__ import annotations

import numpy as np
import pytest

from oracle import detrt_stage as S


def vt_pos(j: int) -> int:
    return (j & ~63) | (((j >> 2) & 3) << 4) | (((j >> 4) & 3) << 2) | (j & 3)


def mfma_16x16x64(a_frag, b_frag):
    """a_frag, b_frag: (64 lanes, 16 slots) int. Returns C (64 lanes, 4 regs)."""
    A = np.zeros((16, 64), np.int64)
    Bm = np.zeros((64, 16), np.int64)
    for l in range(64):
        for s in range(16):
            A[l & 15, 16 * (l >> 4) + s] = a_frag[l, s]
            Bm[16 * (l >> 4) + s, l & 15] = b_frag[l, s]
    C = A @ Bm
    out = np.zeros((64, 4), np.int64)
    for l in range(64):
        for i in range(4):
            out[l, i] = C[4 * (l >> 4) + i, l & 15]
    return out


def test_vt_pos_is_a_block_permutation():
    for base in (0, 64, 128):
        got = sorted(vt_pos(base + j) for j in range(64))
        assert got == list(range(base, base + 64))
    # the C register order of a 64-key tile equals the k slot order of the P x V MFMA
    for g in range(4):
        for s in range(16):
            key = 16 * (s >> 2) + 4 * g + (s & 3)   # C: block b = s >> 2, register i = s & 3
            assert vt_pos(key) == 16 * g + s        # where the A operand's lane group g reads slot s


def emulate(qq, qs, kq, ks, vq, vs, B, T, H, Hkv, hd, inv):
    """The kernel's index arithmetic with exact integer products; returns o (N, H * hd) and the
    largest address touched per buffer."""
    NC, ND = (hd + 63) // 64, hd // 16
    Tp = -(-T // 64) * 64
    N = B * T
    vt = np.zeros(B * Hkv * hd * Tp, np.int64)
    for n in range(N):  # v_transpose / qkv_post's vt store
        bseq, pos = divmod(n, T)
        for hk in range(Hkv):
            for d in range(hd):
                vt[((bseq * Hkv + hk) * hd + d) * Tp + vt_pos(pos)] = vq[n, hk, d]
    maxaddr = dict(qq=0, kq=0, vt=0, ks=0, vs=0, o=0, qs=0)
    o = np.zeros((N, H * hd), np.float32)
    lanes = np.arange(64)
    ql, g = lanes & 15, lanes >> 4
    for bseq in range(B):
        nb = bseq * T
        for h in range(H):
            hk = h // (H // Hkv)
            for q0 in range(0, T, 16):  # one wave per 16 queries
                qi = q0 + ql
                qc = np.minimum(qi, T - 1)
                maxaddr["qs"] = max(maxaddr["qs"], int(((nb + qc) * H + h).max()))
                my_qs = qs[nb + qc, h, 0]
                qf = np.zeros((NC, 64, 16), np.int64)
                for c in range(NC):
                    for l in range(64):
                        d0 = 64 * c + 16 * g[l]
                        if d0 < hd:
                            addr = ((nb + qc[l]) * H + h) * hd + d0
                            maxaddr["qq"] = max(maxaddr["qq"], addr + 15)
                            qf[c, l] = qq[nb + qc[l], h, d0:d0 + 16]
                kmax = min(T, q0 + 16)
                nkt = (kmax + 63) // 64
                tiles = []
                for kt in range(nkt):
                    Sv = np.full((64, 4, 4), -np.inf, np.float32)
                    for b in range(4):
                        kr = np.minimum(kt * 64 + 16 * b + ql, T - 1)
                        acc = np.zeros((64, 4), np.int64)
                        for c in range(NC):
                            kf = np.zeros((64, 16), np.int64)
                            for l in range(64):
                                d0 = 64 * c + 16 * g[l]
                                if d0 < hd:
                                    addr = ((nb + kr[l]) * Hkv + hk) * hd + d0
                                    maxaddr["kq"] = max(maxaddr["kq"], addr + 15)
                                    kf[l] = kq[nb + kr[l], hk, d0:d0 + 16]
                            acc += mfma_16x16x64(kf, qf[c])
                        for i in range(4):
                            j = kt * 64 + 16 * b + 4 * g + i
                            ok = (j <= qi) & (j < T)
                            jc = np.minimum(j, T - 1)
                            sc = ((acc[:, i].astype(np.float32) * my_qs) * ks[nb + jc, hk, 0]) * inv
                            Sv[:, b, i] = np.where(ok, sc, -np.inf)
                            if ok.any():
                                maxaddr["ks"] = max(maxaddr["ks"], int(((nb + j[ok]) * Hkv + hk).max()))
                    tiles.append(Sv)
                # row statistics per query (lanes with equal ql), as the oracle defines them
                allS = np.concatenate([t.reshape(64, 16) for t in tiles], axis=1)  # (64, 16 * nkt)
                keys = np.concatenate([[kt * 64 + 16 * (s >> 2) + 4 * g + (s & 3) for s in range(16)]
                                       for kt in range(nkt)], axis=0).T            # (64, 16 * nkt)
                ohi = np.zeros((ND, 64, 4), np.int64)
                olo = np.zeros((ND, 64, 4), np.int64)
                pis = np.zeros((64, allS.shape[1]), np.int64)
                sps = np.zeros(64, np.float32)
                for qv in range(16):
                    ls = np.nonzero(ql == qv)[0]
                    row = allS[ls].ravel()
                    kk = keys[ls].ravel()
                    valid = row != -np.inf
                    if not valid.any():
                        continue
                    mx = row[valid].max()
                    e = np.zeros_like(row)
                    e[valid] = S.det_exp(row[valid] - mx)
                    den = S.exact_rowsum(e[None, :], S.MAX_KEYS)[0]
                    pv = np.zeros_like(row)
                    pv[valid] = (e[valid] / den) * vs[nb + kk[valid], hk, 0]
                    sp = np.maximum(pv.max(), np.float32(1e-30)) / np.float32(S.P_LEVELS)
                    pi = np.where(valid, np.clip(np.rint(pv / sp), 0, S.P_LEVELS), 0).astype(np.int64)
                    pis[ls] = pi.reshape(len(ls), -1)
                    sps[ls] = sp
                for kt in range(nkt):
                    p = pis[:, 16 * kt:16 * kt + 16]
                    bhi, blo = p >> 7, p & 127
                    for d in range(ND):
                        vf = np.zeros((64, 16), np.int64)
                        for l in range(64):
                            addr = ((bseq * Hkv + hk) * hd + 16 * d + ql[l]) * Tp + kt * 64 + 16 * g[l]
                            maxaddr["vt"] = max(maxaddr["vt"], addr + 15)
                            vf[l] = vt[addr:addr + 16]
                        ohi[d] += mfma_16x16x64(vf, bhi)
                        olo[d] += mfma_16x16x64(vf, blo)
                for l in range(64):
                    if qi[l] >= T:
                        continue
                    for d in range(ND):
                        for i in range(4):
                            a = (int(ohi[d, l, i]) << 7) + int(olo[d, l, i])
                            col = 16 * d + 4 * g[l] + i
                            addr = ((nb + qi[l]) * H + h) * hd + col
                            maxaddr["o"] = max(maxaddr["o"], addr)
                            o[nb + qi[l], h * hd + col] = np.float32(a) * sps[l]
    return o, maxaddr


@pytest.mark.parametrize("B,T,H,Hkv,hd", [(1, 12, 4, 2, 32), (2, 5, 2, 1, 64), (1, 70, 2, 2, 128), (1, 1, 1, 1, 32)])
def test_attention_layout_matches_oracle(B, T, H, Hkv, hd):
    rng = np.random.default_rng(T * 31 + hd)
    N = B * T
    qq = rng.integers(-127, 128, (N, H, hd))
    kq = rng.integers(-127, 128, (N, Hkv, hd))
    vq = rng.integers(-127, 128, (N, Hkv, hd))
    qs = rng.uniform(1e-3, 1e-2, (N, H, 1)).astype(np.float32)
    ks = rng.uniform(1e-3, 1e-2, (N, Hkv, 1)).astype(np.float32)
    vs = rng.uniform(1e-3, 1e-2, (N, Hkv, 1)).astype(np.float32)
    inv = S.inv_sqrt_hd(hd)
    o, maxaddr = emulate(qq, qs, kq, ks, vq, vs, B, T, H, Hkv, hd, inv)
    for bseq in range(B):
        sl = slice(bseq * T, (bseq + 1) * T)
        _, _, _, ref = S.attention(qq[sl], qs[sl], kq[sl], ks[sl], vq[sl], vs[sl], inv)
        np.testing.assert_array_equal(o[sl].view(np.uint32), ref.transpose(1, 0, 2).reshape(T, H * hd).view(np.uint32))
    Tp = -(-T // 64) * 64
    assert maxaddr["qq"] < N * H * hd and maxaddr["kq"] < N * Hkv * hd
    assert maxaddr["vt"] < B * Hkv * hd * Tp and maxaddr["o"] < N * H * hd
    assert maxaddr["ks"] < N * Hkv and maxaddr["qs"] < N * H


def _at_block(i, ntiles, H, Hkv, B):
    """uwc_attn.hip at_block: block id -> (q tile, head, sequence)."""
    G, units = H // Hkv, B * Hkv
    if units % 8 == 0:
        x, j = i & 7, i >> 3
        per_tile = units // 8 * G
        qt = ntiles - 1 - j // per_tile
        r = j % per_tile
        u = x + 8 * (r // G)
        return qt, (u % Hkv) * G + r % G, u // Hkv
    return ntiles - 1 - i % ntiles, (i // ntiles) % H, i // (ntiles * H)


@pytest.mark.parametrize("ntiles,H,Hkv,B", [(128, 16, 8, 1), (64, 32, 8, 1), (5, 8, 8, 2), (3, 4, 2, 4),
                                            (7, 6, 3, 1), (16, 16, 16, 1), (2, 8, 1, 3)])
def test_block_mapping_is_a_bijection_and_xcd_local(ntiles, H, Hkv, B):
    """Every (q tile, head, sequence) gets exactly one block; when the kv units split over the 8
    XCDs (id % 8), each XCD's blocks read the keys of its own units only, and within an XCD the
    q tiles come longest first."""
    total = ntiles * H * B
    got = [_at_block(i, ntiles, H, Hkv, B) for i in range(total)]
    assert sorted(got) == sorted((qt, h, b) for qt in range(ntiles) for h in range(H) for b in range(B))
    if B * Hkv % 8 == 0:
        G = H // Hkv
        for x in range(8):
            mine = [got[i] for i in range(x, total, 8)]
            assert {(b, h // G) for _, h, b in mine} == {((u // Hkv), u % Hkv) for u in range(x, B * Hkv, 8)}
            qts = [qt for qt, _, _ in mine]
            assert qts == sorted(qts, reverse=True)


def _rowmax_tile_maps(hd: int, W: int = 4):
    """attn_rowmax_kernel's ring tile of 64 key rows x hd bytes in 16-byte slots, DMA'd by the W
    waves of a workgroup: the DMA map (wave, DMA u, lane) -> (key row m, piece p) at slot s, and
    the read map (lane, block b, chunk c) -> slot. swz(m) = (m / (16 / PR)) & (PR - 1), PR = hd / 16
    pieces per row."""
    PR = hd // 16
    TILE = 64 * hd
    KS = TILE // 16 // W
    KD = KS // 64 if KS >= 64 else 1
    KL = 64 if KS >= 64 else KS
    assert KD * KL * W * 16 == TILE
    swz = lambda m: (m // (16 // PR)) & (PR - 1)
    written = {}
    for wave in range(W):
        for u in range(KD):
            for lane in range(KL):
                s = (wave * KD + u) * KL + lane
                m = s // PR
                p = (s % PR) ^ swz(m)
                assert s not in written
                written[s] = (m, p)
    reads = {}
    NC = (hd + 63) // 64
    for lane in range(64):
        ql, g = lane & 15, lane >> 4
        for b in range(4):
            for c in range(NC):
                p = 4 * c + g
                if p < PR:
                    m = 16 * b + ql
                    reads[(lane, b, c)] = m * PR + (p ^ swz(m))
    return PR, written, reads


@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("W", [4, 8, 16])
def test_rowmax_ring_dma_and_reads(hd, W):
    """Every 16-byte piece of the 64 key rows is DMA'd exactly once by the W waves (4 per head of
    the workgroup), the slots of one DMA instruction are contiguous (lane l at slot base + l, as
    global_load_lds writes them), eight (hd 128) consecutive lanes read one whole key row, the
    lane that reads (block b, chunk c) finds key row 16 b + (lane & 15) at dims 64 c + 16 (lane >> 4),
    and the 16 lanes of one lane group hit 16 distinct 16-byte bank groups (no LDS bank
    conflict). The key scales: 64 / W lanes of each wave, every key once."""
    PR, written, reads = _rowmax_tile_maps(hd, W)
    assert sorted(written) == list(range(64 * PR))
    assert sorted(written.values()) == [(m, p) for m in range(64) for p in range(PR)]
    if hd == 128:
        for s0 in range(0, 64 * PR, 8):
            assert {written[s][0] for s in range(s0, s0 + 8)} == {s0 // 8}
    for (lane, b, c), s in reads.items():
        assert written[s] == (16 * b + (lane & 15), 4 * c + (lane >> 4))
    for b in range(4):
        for c in range((hd + 63) // 64):
            for g in range(4):
                slots = [reads[(g * 16 + ql, b, c)] for ql in range(16) if (g * 16 + ql, b, c) in reads]
                if slots:
                    assert len({s % 16 for s in slots}) == len(slots)
    SL = 64 // W
    assert sorted(w * SL + l for w in range(W) for l in range(SL)) == list(range(64))


def _ring_schedule(nkt: int, NS: int, per_tile: int):
    """One wave's DMA ring of NS stages as the attention kernels run it: tiles 0 .. NS - 2 issued
    up front, tile kt + NS - 1 issued after the barrier of iteration kt into tile kt - 1's stage;
    the wait before iteration kt leaves at most (NS - 2) per_tile of the wave's DMAs pending, or
    none when no later tile is in flight. Checks that the tile a wait covers has landed and that
    a stage is overwritten only after the iteration that read it (every wave passed the barrier
    of the next one)."""
    NW = (NS - 2) * per_tile
    issued = []        # tile per DMA, in issue order
    stage_of = {}
    last_read = {}     # stage -> last tile read from it
    for t in range(NS - 1):
        if t < nkt:
            issued += [t] * per_tile
            stage_of[t] = t % NS
    done = 0           # DMAs known complete
    for kt in range(nkt):
        allowed = NW if kt + NS - 2 < nkt else 0
        done = max(done, len(issued) - allowed)
        assert all(x != kt for x in issued[done:]), "tile read before its DMA completed"
        if kt + NS - 1 < nkt:
            st = (kt + NS - 1) % NS
            assert last_read.get(st, -1) <= kt - 1 and st == (kt - 1) % NS
            issued += [kt + NS - 1] * per_tile
            stage_of[kt + NS - 1] = st
        assert stage_of[kt] == kt % NS
        last_read[kt % NS] = kt


@pytest.mark.parametrize("T,hd", [(1, 128), (100, 64), (300, 32), (2048, 128)])
def test_rowmax_ring_schedule(T, hd):
    """attn_rowmax_kernel's ring: NS = 4 stages, KD + 1 DMAs per wave and tile (key rows, key
    scales)."""
    TILE = 64 * hd
    KS = TILE // 16 // 4
    KD = KS // 64 if KS >= 64 else 1
    for qt in range((T + 63) // 64):
        _ring_schedule(qt + 1, 4, KD + 1)


def _vchunk(r: int) -> int:
    """Chunk (four 16-byte slots) of row r of a 16-row block in the P x V ring."""
    return 4 * ((r >> 1) & 3) + 2 * (r & 1) + (r >> 3)


def _pv_maps(hd: int):
    """The P x V sweep's (attention_kernel MODES 3 and 4) V ring tile: hd / 16 blocks of 16 V^T
    rows x 64 key bytes, row r of block d in chunk _vchunk(r) (slots 64 d + 4 chunk .. + 3), its
    piece p at slot p ^ ((r >> 1) & 3) of the chunk; the four waves DMA the tile in VD
    instructions of VL lanes each, lane l of an instruction writing slot base + l. Returns the
    DMAs per wave and tile, the DMA map slot -> (row, piece, instruction) and the read map
    (lane, fragment d) -> slot."""
    VT = hd * 64
    VS = VT // 16 // 4
    VD = VS // 64 if VS >= 64 else 1
    VL = 64 if VS >= 64 else VS
    assert VD * VL * 4 * 16 == VT
    inv = {_vchunk(r): r for r in range(16)}
    written = {}
    for wave in range(4):
        for u in range(VD):
            base = (wave * VD + u) * VL
            for lane in range(VL):
                s16 = base + lane
                r = inv[(s16 >> 2) & 15]
                row = 16 * (s16 >> 6) + r
                p = (s16 & 3) ^ ((r >> 1) & 3)
                assert s16 not in written
                written[s16] = (row, p, (wave, u))
    reads = {}
    for lane in range(64):
        ql, g = lane & 15, lane >> 4
        for d in range(hd // 16):
            reads[(lane, d)] = 64 * d + 4 * _vchunk(ql) + (g ^ ((ql >> 1) & 3))
    return VD + 5, written, reads


@pytest.mark.parametrize("hd", [32, 64, 128])
def test_pv_ring_dma_and_reads(hd):
    """Every 16-byte piece of the tile's hd V^T rows is DMA'd exactly once by the four waves;
    four consecutive lanes of one DMA read one row's 64 contiguous bytes; the lane that reads
    fragment d finds dim 16 d + (lane & 15) at keys 16 (lane >> 4) .. + 15 (the MFMA B operand).
    Banks: every lane's slot residue mod 16 equals the one attn_rowmax_kernel's ring read gives
    the same lane (chunk c = 0, whose pattern rocprofv3 counts free of bank conflicts), so the
    two reads spread over the banks alike; the 16 lanes of a lane group hit 16 distinct 16-byte
    bank groups. The V scales: lanes 0-15 of wave w DMA keys 16 w .. + 15."""
    _, written, reads = _pv_maps(hd)
    assert sorted(written) == list(range(hd * 4))
    assert sorted((r, p) for r, p, _ in written.values()) == [(r, p) for r in range(hd) for p in range(4)]
    for s0 in range(0, hd * 4, 4):
        rows = {written[s][0] for s in range(s0, s0 + 4)}
        assert len(rows) == 1 and {written[s][1] for s in range(s0, s0 + 4)} == {0, 1, 2, 3}
        assert len({written[s][2] for s in range(s0, s0 + 4)}) == 1
    for (lane, d), s in reads.items():
        assert written[s][:2] == (16 * d + (lane & 15), lane >> 4)
    _, _, rm_reads = _rowmax_tile_maps(128)
    for (lane, d), s in reads.items():
        assert s % 16 == rm_reads[(lane, 0, 0)] % 16, (lane, d)
    for d in range(hd // 16):
        for g in range(4):
            assert len({reads[(g * 16 + ql, d)] % 16 for ql in range(16)}) == 16
    assert sorted(w * 16 + l for w in range(4) for l in range(16)) == list(range(64))


@pytest.mark.parametrize("T,hd", [(1, 128), (100, 64), (300, 32), (2048, 128)])
def test_pv_ring_schedule(T, hd):
    """The P x V ring (after the sums, in the same kernel): NS = 2 stages, 4 + VD + 1 DMAs per wave
    and tile (exponentials, V, V scales); tile kt + 1 is issued after the barrier of iteration kt
    and the kernel waits for vmcnt(0) before each iteration, so no other tile is in flight."""
    per, _, _ = _pv_maps(hd)
    for qt in range((T + 63) // 64):
        _ring_schedule(qt + 1, 2, per)
