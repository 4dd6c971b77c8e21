"""GPU parity of the skinny GEMM path (m <= 64: decode and small batches, BASELINE configs 1 and 4)
through the C-ABI: exact int32 products against the CPU oracle and against the 128 x 128
tiled kernel (UWC_FLAG_TILE128), every token count 1..64 boundary, ragged n and k, and the
fp32 / bf16 dequant epilogues bit for bit (runtime/detrt/qwen3.py:106-126). Both skinny forms
run: the X-stationary one (X staged in LDS, m * (k + 16) bytes up to ~150 KB) and the streaming
one for larger X (e.g. 40 x 14336, 64 x 4096)."""
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


@pytest.mark.parametrize("m", [1, 2, 5, 15, 16, 17, 31, 32, 33, 48, 49, 63, 64])
@pytest.mark.parametrize("n,k", [(96, 2048), (250, 576), (4100, 64)])
def test_skinny_int32_matches_oracle(dev, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    from uwc_amd import ops
    C = _gemm(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev), ops.OUT_I32)
    assert np.array_equal(C.cpu().numpy(), O.igemm(A, B))


@pytest.mark.parametrize("m,n,k", [(1, 28672, 4096), (8, 4096, 14336), (32, 6144, 4096), (64, 6144, 2048),
                                   (4, 32768, 1024), (3, 16, 192), (40, 4096, 14336), (64, 300, 4096),
                                   (17, 50000, 128), (64, 1, 2048)])
def test_skinny_equals_tiled_kernel(dev, m, n, k):
    """The split-k skinny path and the 128 x 128 tiled kernel give the same int32 product (exact
    sums: the k split and the reduction order cannot change the result)."""
    from uwc_amd import ops
    g = torch.Generator(device=dev)
    g.manual_seed(m + n + k)
    A = torch.randint(-128, 128, (m, k), dtype=torch.int8, device=dev, generator=g)
    B = torch.randint(-128, 128, (n, k), dtype=torch.int8, device=dev, generator=g)
    C = _gemm(A, B, ops.OUT_I32)
    T = _gemm(A, B, ops.OUT_I32, flags=ops.FLAG_TILE128)
    assert torch.equal(C, T)
    if m * n * k <= 64 * 6144 * 2048:
        assert np.array_equal(C.cpu().numpy(), O.igemm(A.cpu().numpy(), B.cpu().numpy()))


@pytest.mark.parametrize("m,n,k", [(1, 6144, 2048), (19, 1000, 1024), (64, 6144, 2048)])
def test_skinny_dequant_epilogues(dev, m, n, k):
    """OUT_F32 = fmul(fmul(f32(acc), sx), sw) and OUT_BF16 = its RNE bf16, bit-exact vs the oracle."""
    from uwc_amd import ops
    rng = np.random.default_rng(m + n)
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


def test_skinny_det_linear_decode(dev):
    """DetLinear.__call__ at a decode batch (m = 4, Llama-3.1-8B o shape) equals the oracle's
    quant_act -> exact GEMM -> dequant chain bit for bit."""
    from uwc_amd import detrt
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((4096, 4096)) * 0.02).astype(np.float32)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    lay = detrt.DetLinear(torch.from_numpy(W), dev, 128, mine=False)
    Wq, sw, bs = O.quant_weight(W, 128)
    y = lay(torch.from_numpy(x).to(dev))
    _, _, _, want = O.det_linear(x, Wq, sw, bs)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
