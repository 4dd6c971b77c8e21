"""GPU parity of the DMA-streamed skinny GEMM form (m <= 64, k % 1024 == 0: W through an LDS
ring by DMA, X of a token group resident in LDS or streamed with W) through the C-ABI. Shapes are
picked to reach every branch of its plan: one and two token groups, X resident or streamed (8 or
16 X rows per entry), one and two partials buffers, ring depths 4..6, ragged n (a partial last
16-row block), n as small as one block, many blocks per workgroup (a weight-scale table of several
DMAs), 1, 2, 3, 4, 14 and 30 chunks of 1 KB per row, and the odd m that must fall back to the
other forms. Each result is compared with the 128 x 128 tiled kernel
(UWC_FLAG_TILE128) and, where it is cheap, with the CPU oracle; the fp32 / bf16 epilogues bit for
bit with the oracle's dequant (runtime/detrt/qwen3.py:106-126)."""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def _gemm(A, B, out_mode, flags=0, sx=None, sw=None):
    from uwc_amd import _lib, ops
    m, k = A.shape
    n = B.shape[0]
    dt = {ops.OUT_I32: torch.int32, ops.OUT_F32: torch.float32, ops.OUT_BF16: torch.bfloat16}[out_mode]
    out = torch.empty((m, n), dtype=dt, device=A.device)
    _lib.call("uwc_noisy_gemm", A.data_ptr(), B.data_ptr(), m, n, k, 0, None, None, None, 0, None, None, None, 0,
              None if sx is None else sx.data_ptr(), None if sw is None else sw.data_ptr(), out.data_ptr(), out_mode,
              flags, None, torch.cuda.current_stream().cuda_stream)
    return out


# (m, n, k): token groups / partials buffers / ring depth the plan gives on a 256-CU part
SHAPES = [
    (1, 4, 1024),        # one block, one workgroup busy
    (3, 20, 1024),       # partial second block
    (16, 1000, 2048),    # 63 blocks, the last one partial
    (19, 1000, 1024),    # two token tiles in one group
    (34, 300, 4096),     # two token groups of 17, one partials buffer
    (48, 96, 2048),      # two groups of 24
    (64, 96, 2048),      # two groups of 32, one partials buffer
    (64, 1000, 1024),    # two groups, ring depth 5
    (8, 4096, 14336),    # 14 chunks per row, two groups of 4
    (8, 64, 3072),       # 3 chunks per row
    (1, 28672, 4096),    # 7 blocks per workgroup
    (64, 6144, 2048),
    (32, 6144, 4096),    # Llama-3.1-8B qkv at M = 32
    (33, 300, 4096),     # odd m whose X does not fit one group: the other forms
    # X streamed through the ring with W (too large to stay resident)
    (32, 4096, 14336),   # Llama-3.1-8B down at M = 32: two groups of 16, 16 X rows per entry
    (9, 1000, 14336),    # odd m, one group of 9 (rows 9..15 of the entry repeat row 8)
    (24, 2000, 14336),   # two groups of 12
    (6, 256, 30720),     # 8 X rows per entry, 30 chunks per row
]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_skinny_dma_int32(dev, m, n, k):
    from uwc_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(7 * m + n + k)
    A = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    B = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    C = _gemm(A, B, ops.OUT_I32)
    T = _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128)
    assert torch.equal(C, T)
    if m * n * k <= 64 * 6144 * 2048:
        assert np.array_equal(C.cpu().numpy(), O.igemm(A.cpu().numpy(), B.cpu().numpy()))


def test_skinny_dma_many_blocks_per_workgroup(dev):
    """38 blocks per workgroup: the weight-scale table takes three DMAs; int32 and fp32 out."""
    from uwc_amd import ops
    m, n, k = 2, 151936, 1024
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    A = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    B = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    sx = torch.rand(m, device=dev) + 0.5
    sw = torch.rand(n, device=dev) * 1e-3
    C = _gemm(A, B, ops.OUT_I32)
    assert torch.equal(C, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))
    Y = _gemm(A, B, ops.OUT_F32, sx=sx, sw=sw)
    assert torch.equal(Y, _gemm(A, B, ops.OUT_F32, flags=ops.FLAG_TILE128, sx=sx, sw=sw))


@pytest.mark.parametrize("m,n,k", [(1, 6144, 2048), (19, 1000, 1024), (64, 6144, 2048), (34, 300, 4096),
                                   (8, 4096, 14336), (32, 4096, 14336), (9, 1000, 14336)])
def test_skinny_dma_dequant_epilogues(dev, m, n, k):
    """OUT_F32 = fmul(fmul(f32(acc), sx), sw) and OUT_BF16 = its RNE bf16, bit-exact vs the oracle."""
    from uwc_amd import ops
    rng = np.random.default_rng(m + n + k)
    A = rng.integers(-64, 65, size=(m, k), dtype=np.int8)
    B = rng.integers(-64, 65, size=(n, k), dtype=np.int8)
    sx = (rng.random(m, dtype=np.float32) * 1e-2 + 1e-4).astype(np.float32)
    sw = (rng.random(n, dtype=np.float32) * 1e-3 + 1e-5).astype(np.float32)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    sxt, swt = torch.from_numpy(sx).to(dev), torch.from_numpy(sw).to(dev)
    acc = O.igemm(A, B)
    Y = _gemm(At, Bt, ops.OUT_F32, sx=sxt, sw=swt)
    assert np.array_equal(Y.cpu().numpy().view(np.uint32), O.dequant(acc, sx, sw).view(np.uint32))
    Yb = _gemm(At, Bt, ops.OUT_BF16, sx=sxt, sw=swt)
    assert np.array_equal(Yb.cpu().view(torch.int16).numpy().view(np.uint16), O.scale_bf16(acc, sx, sw))


def test_skinny_dma_repeated_calls_and_rotation(dev):
    """Back-to-back calls over distinct weights (no state carried between launches) give the same
    products as one call each."""
    from uwc_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    A = torch.randint(-128, 128, (64, 2048), dtype=torch.int8, device=dev, generator=g)
    Bs = [torch.randint(-128, 128, (6144, 2048), dtype=torch.int8, device=dev, generator=g) for _ in range(3)]
    first = [_gemm(A, B, ops.OUT_I32) for B in Bs]
    again = [_gemm(A, B, ops.OUT_I32) for B in reversed(Bs)][::-1]
    for a, b, B in zip(first, again, Bs):
        assert torch.equal(a, b)
        assert torch.equal(a, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))
