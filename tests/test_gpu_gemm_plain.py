"""GPU parity of the DMA-pipelined plain GEMM (128 x 128 and 128 x 256 tiles, ring depths 2-4,
DMA issued per step or spread over the next step's passes)
through the C-ABI: every configuration at shapes reaching fewer k steps than ring stages, k steps
not a multiple of the ring depth, one and several tiles, and the configs[1] linears at M = 2048,
against the generic 128 x 128 kernel (UWC_FLAG_TILE128) and the CPU oracle; the fp32 / bf16
dequant epilogues bit for bit with the oracle (runtime/detrt/qwen3.py:106-126)."""
import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

# (bm, bn) of configurations 0..7 (c and c + 4 share a tiling)
CFG_TILES = [(128, 128), (128, 256), (128, 128), (128, 256)] * 2


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


def _rand(dev, seed, *shape):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    return torch.randint(-128, 128, shape, dtype=torch.int8, device=dev, generator=g)


SHAPES = [
    (128, 256, 128),     # one tile, one k step (fewer than any ring)
    (256, 512, 256),     # two k steps
    (384, 768, 384),     # three k steps: not a multiple of ring depths 2 and 4
    (256, 1024, 640),    # five k steps
    (1024, 1536, 1152),  # nine k steps, 48-96 tiles
]


@pytest.mark.parametrize("cfg", range(8))
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_plain_cfg_int32(dev, cfg, m, n, k):
    from uwc_amd import ops
    A, B = _rand(dev, m + k + cfg, m, k), _rand(dev, n + 7 * k, n, k)
    C = _gemm(A, B, ops.OUT_I32, flags=ops.plain_cfg(cfg))
    assert torch.equal(C, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))
    if m * n * k <= 256 * 1024 * 640:
        assert np.array_equal(C.cpu().numpy(), O.igemm(A.cpu().numpy(), B.cpu().numpy()))


@pytest.mark.parametrize("cfg", range(8))
def test_plain_cfg_dequant(dev, cfg):
    """OUT_F32 = fmul(fmul(f32(acc), sx), sw) and OUT_BF16 = its RNE bf16, bit-exact vs the oracle."""
    from uwc_amd import ops
    m, n, k = 256, 512, 384
    rng = np.random.default_rng(cfg)
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    sx = (rng.random(m, dtype=np.float32) * 1e-2 + 1e-4).astype(np.float32)
    sw = (rng.random(n, dtype=np.float32) * 1e-3 + 1e-5).astype(np.float32)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    sxt, swt = torch.from_numpy(sx).to(dev), torch.from_numpy(sw).to(dev)
    acc = O.igemm(A, B)
    Y = _gemm(At, Bt, ops.OUT_F32, flags=ops.plain_cfg(cfg), sx=sxt, sw=swt)
    assert np.array_equal(Y.cpu().numpy().view(np.uint32), O.dequant(acc, sx, sw).view(np.uint32))
    Yb = _gemm(At, Bt, ops.OUT_BF16, flags=ops.plain_cfg(cfg), sx=sxt, sw=swt)
    assert np.array_equal(Yb.cpu().view(torch.int16).numpy().view(np.uint16), O.scale_bf16(acc, sx, sw))


# the Qwen3-1.7B layer linears at M = 2048 (qkv, o, gate_up, down), through the
# automatic choice (no flags) and every configuration that takes the shape
@pytest.mark.parametrize("n,k", [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144)])
def test_plain_config1_linears(dev, n, k):
    from uwc_amd import ops
    m = 2048
    A, B = _rand(dev, n + 1, m, k), _rand(dev, k + 2, n, k)
    ref = _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128)
    assert torch.equal(_gemm(A, B, ops.OUT_I32), ref)
    for cfg, (bm, bn) in enumerate(CFG_TILES):
        if m % bm == 0 and n % bn == 0:
            assert torch.equal(_gemm(A, B, ops.OUT_I32, flags=ops.plain_cfg(cfg)), ref), cfg
    # rows sampled against the oracle: the first, the last and a random tile row's worth
    rows = np.r_[0:8, m - 8:m, 1000:1016]
    Ac = A.cpu().numpy()[rows]
    assert np.array_equal(ref.cpu().numpy()[rows], O.igemm(Ac, B.cpu().numpy()))


def test_plain_repeated_calls_distinct_weights(dev):
    """Back-to-back launches over distinct weights carry no state between calls."""
    from uwc_amd import ops
    A = _rand(dev, 5, 512, 1024)
    Bs = [_rand(dev, 6 + i, 1024, 1024) for i in range(3)]
    for cfg in range(8):
        first = [_gemm(A, B, ops.OUT_I32, flags=ops.plain_cfg(cfg)) for B in Bs]
        again = [_gemm(A, B, ops.OUT_I32, flags=ops.plain_cfg(cfg)) for B in reversed(Bs)][::-1]
        for a, b, B in zip(first, again, Bs):
            assert torch.equal(a, b)
            assert torch.equal(a, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))


@pytest.mark.parametrize("k", [384, 1152])
def test_large_tile_plain_odd_k_steps(dev, k):
    """The 256 x 256 kernel's plain form (4096 x 4096: one tile per CU) with an odd number of
    128-wide k steps, so its last step runs outside the two-stage main loop; int32, fp32 and bf16
    outputs against the generic 128 x 128 kernel, the int32 rows sampled against the oracle."""
    from uwc_amd import ops
    m = n = 4096
    A, B = _rand(dev, k, m, k), _rand(dev, k + 1, n, k)
    sx = torch.rand(m, device=dev) * 1e-2 + 1e-4
    sw = torch.rand(n, device=dev) * 1e-3 + 1e-5
    C = _gemm(A, B, ops.OUT_I32)
    assert torch.equal(C, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))
    rows = np.r_[0:4, 2047:2051, m - 4:m]
    assert np.array_equal(C.cpu().numpy()[rows], O.igemm(A.cpu().numpy()[rows], B.cpu().numpy()))
    for mode in (ops.OUT_F32, ops.OUT_BF16):
        Y = _gemm(A, B, mode, sx=sx, sw=sw)
        Yr = _gemm(A, B, mode, flags=ops.FLAG_TILE128, sx=sx, sw=sw)
        assert torch.equal(Y.view(torch.int16) if mode == ops.OUT_BF16 else Y.view(torch.int32),
                           Yr.view(torch.int16) if mode == ops.OUT_BF16 else Yr.view(torch.int32))


@pytest.mark.parametrize("m,n,k", [(2048, 32768, 256), (2560, 30720, 384), (4096, 16384, 128), (8192, 4096, 2048),
                                   (2560, 16384, 128), (4096, 8192, 640)])
def test_plain_multi_tile(dev, m, n, k):
    """Plain int32 GEMMs of at least two 256 x 256 tiles per CU run on the persistent split-role
    kernel (each workgroup takes tiles b, b + grid, ...; 1024, 1200, 1024, 512, 640 and 512 tiles
    here, so at some shapes some workgroups take one more tile than others; 2, 3, 1, 16, 1 and 5 k
    steps): the output equals the generic 128 x 128 kernel's, and a sample of rows equals the
    oracle's exact product."""
    from uwc_amd import ops
    A, B = _rand(dev, m + k, m, k), _rand(dev, n + 3 * k, n, k)
    C = _gemm(A, B, ops.OUT_I32)
    assert torch.equal(C, _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128))
    rows = np.r_[0:3, m // 2, m - 1]
    assert np.array_equal(C[rows].cpu().numpy(), O.igemm(A[rows].cpu().numpy(), B.cpu().numpy()))
