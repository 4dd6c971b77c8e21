"""CPU check of the large-tile GEMM's data movement (useful-work-coin_amd/csrc/uwc_gemm256.hip):
with the tile constants read from the source, the direct-to-LDS segments cover each stage
exactly once, every DMA source row lies inside the workgroup's tile rows, and every MFMA
fragment read finds the tile row and k bytes it expects under the LDS swizzle. A segment count
that overshoots the tile (reads past the last operand row) fails here, not on a GPU."""
import itertools
import os
import re

import pytest

from conftest import PKG

SRC = os.path.join(PKG, "csrc", "uwc_gemm256.hip")


def consts(bk: int) -> dict:
    src = open(SRC).read()
    d = {"W_BK": bk}
    for name in ("W_BM", "W_BN", "W_THREADS"):
        d[name] = int(re.search(rf"#define {name} (\d+)", src).group(1))
    # the expressions the kernel uses, evaluated with the same definitions
    for name in ("W_WAVES", "W_TILE", "W_SEGS_PER_WAVE", "W_RPS", "W_CH", "W_KP"):
        expr = re.search(rf"#define {name} \(([^)]*)\)", src).group(1)
        d[name] = int(eval(expr.replace("/", "//"), {}, dict(d)))
    d["W_STAGES"] = 4 if bk == 64 else 2
    return d


@pytest.mark.parametrize("bk", [64, 128])
def test_dma_and_fragment_layout(bk):
    c = consts(bk)
    BK, TILE, SPW, RPS, CH, KP, WAVES = c["W_BK"], c["W_TILE"], c["W_SEGS_PER_WAVE"], c["W_RPS"], c["W_CH"], c["W_KP"], c["W_WAVES"]
    assert SPW * WAVES * 1024 == TILE, "DMA segments must cover one operand tile exactly"
    assert 2 * TILE * c["W_STAGES"] <= 160 * 1024
    swz = (lambda r: ((r >> 1) ^ (r >> 2)) & 3) if BK == 64 else (lambda r: (r ^ (r >> 3)) & 7)
    img = {}
    for wave, lane in itertools.product(range(WAVES), range(64)):
        rin, phys = lane // CH, lane % CH
        for t in range(SPW):
            s = SPW * wave + t
            row = RPS * s + rin
            col = (phys ^ swz(row)) * 16
            assert row < c["W_BM"] and col + 16 <= BK, "DMA source outside the tile"
            for op in (0, 1):
                off = op * TILE + s * 1024 + lane * 16
                assert off not in img
                img[off] = (op, row, col)
    assert len(img) == 2 * TILE // 16
    for wave, lane in itertools.product(range(WAVES), range(64)):
        wm, wn, r, h = wave >> 2, wave & 3, lane & 31, lane >> 5
        for kp in range(KP):
            ci = 2 * kp + h
            for mb in range(4):
                off = (wm * 128 + mb * 32) * BK + r * BK + ((ci ^ swz(r + 32 * (mb & 1))) << 4)
                assert img[off] == (0, wm * 128 + mb * 32 + r, ci * 16)
            for nb in range(2):
                off = TILE + (wn * 64 + nb * 32) * BK + r * BK + ((ci ^ swz(r + 32 * (nb & 1))) << 4)
                assert img[off] == (1, wn * 64 + nb * 32 + r, ci * 16)


def test_bank_groups_conflict_free():
    """16 consecutive rows at one logical chunk fall in 16 distinct 16-byte bank groups (64
    banks), and any 8 consecutive rows in 8 distinct ones (32 banks)."""
    for BK, swz in ((64, lambda r: ((r >> 1) ^ (r >> 2)) & 3), (128, lambda r: (r ^ (r >> 3)) & 7)):
        CH = BK // 16
        for base in range(0, 64, 16):
            for ci in range(CH):
                g64 = {((base + i) * BK + ((ci ^ swz(base + i)) << 4)) // 16 % 16 for i in range(16)}
                assert len(g64) == 16, (BK, base, ci)
                for b8 in (base, base + 8):
                    g32 = {((b8 + i) * BK + ((ci ^ swz(b8 + i)) << 4)) // 16 % 8 for i in range(8)}
                    assert len(g32) == 8, (BK, b8, ci)
