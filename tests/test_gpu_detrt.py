"""GPU parity of the detrt integer linear (libuwc_hip.so through uwc_amd): exact int32 GEMMs at
the BASELINE shapes and ragged edges, quant_act and the fused dequant bit-exact against the
Go-referee golden fixtures and the CPU oracle (runtime/tests/test_detrt.py,
runtime/tests/test_fp32_native.py)."""
import hashlib
import os

import numpy as np
import pytest
import torch

import oracle as O
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

FIXTURES = ["detrt_tiny_qwen3", "detrt_tiny_llama", "detrt_qwen3_1p7b"]


def _mods():
    from uwc_amd import detrt, ops
    return ops, detrt


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (256, 384, 1024), (1, 128, 2048), (65, 200, 576), (7, 1, 64),
                                   (64, 6144, 2048), (300, 257, 4096)])
def test_igemm_matches_oracle(dev, m, n, k):
    ops, _ = _mods()
    rng = np.random.default_rng(m * 7 + n + k)
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    C = ops.igemm_i32(torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev))
    assert np.array_equal(C.cpu().numpy(), O.igemm(A, B))


def test_igemm_known_answer_L1(dev):
    """results/xc_cpu.json:4: the same int32 product on every device."""
    ops, _ = _mods()
    rng = np.random.default_rng(2026)
    A = rng.integers(-64, 65, size=(1024, 4096), dtype=np.int8)
    Bt = rng.integers(-64, 65, size=(3072, 4096), dtype=np.int8)
    C = ops.igemm_i32(torch.from_numpy(A).to(dev), torch.from_numpy(Bt).to(dev))
    assert hashlib.sha256(C.cpu().numpy().tobytes()).hexdigest()[:20] == "bf9394d180bda5b0412c"


def test_igemm_extremes(dev):
    ops, _ = _mods()
    A = torch.full((128, 4096), -128, dtype=torch.int8, device=dev)
    B = torch.full((128, 4096), -128, dtype=torch.int8, device=dev)
    assert int(ops.igemm_i32(A, B)[5, 7].item()) == 128 * 128 * 4096
    B = torch.full((128, 4096), 127, dtype=torch.int8, device=dev)
    assert int(ops.igemm_i32(A, B)[127, 127].item()) == -128 * 127 * 4096


@pytest.mark.parametrize("name", FIXTURES)
def test_quant_act_fixtures(dev, name):
    _, detrt = _mods()
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    Bs = int(z["cfg"][5])
    for l in (0, 1):
        for src, qa in (("N1", "QA1"), ("O", "QA2"), ("N2", "QA3"), ("SM", "QA4")):
            x = z[f"l{l}_{src}"]
            q, s = detrt.quant_act(torch.from_numpy(x).to(dev), detrt.hadamard_bs(Bs, x.shape[1]))
            assert np.array_equal(q.cpu().numpy(), z[f"l{l}_{qa}_q"]), (name, l, qa)
            assert np.array_equal(s.cpu().numpy().view(np.uint32), z[f"l{l}_{qa}_s"].view(np.uint32)), (name, l, qa)


@pytest.mark.parametrize("name", FIXTURES)
def test_linear_fixtures(dev, name):
    """QA x W through the fused GEMM + dequant epilogue equals the referee's linearElem."""
    _, detrt = _mods()
    z = np.load(os.path.join(GOLDEN, name + ".npz"))
    for l in (0, 1):
        for lin, qa, op in (("qkv", "QA1", "QKV"), ("o", "QA2", "OP"), ("gu", "QA3", "GU"), ("down", "QA4", "DN")):
            lay = detrt.DetLinear.from_quantized(torch.from_numpy(z[f"l{l}_W_{lin}_q"]).to(dev),
                                                 torch.from_numpy(z[f"l{l}_W_{lin}_s"]).to(dev), 0)
            q = torch.from_numpy(z[f"l{l}_{qa}_q"]).to(dev)
            sx = torch.from_numpy(z[f"l{l}_{qa}_s"]).to(dev)
            acc = lay.int_gemm(q)
            y = detrt.dequant(acc, sx, lay.sw)
            assert np.array_equal(y.cpu().numpy().view(np.uint32), z[f"l{l}_{op}"].view(np.uint32)), (name, l, lin)
            y2 = torch.empty_like(y)
            from uwc_amd import _lib
            _lib.call("uwc_igemm_dequant_f32", q.data_ptr(), lay.Wq.data_ptr(), q.shape[0], lay.n, lay.k, sx.data_ptr(),
                      lay.sw.data_ptr(), y2.data_ptr(), torch.cuda.current_stream().cuda_stream)
            assert torch.equal(y, y2)


@pytest.mark.parametrize("rows,k", [(2048, 1024), (1024, 1536)])
@pytest.mark.parametrize("bs", [0, 2, 16, 32, 64, 128, 256, 512])
def test_quant_act_double_group_kernel(dev, rows, k, bs):
    """The one-wave-per-1024-elements quantizer (taken from 2048 double groups on): every Hadamard
    block size, so that every count of cross-lane stages (and with it every sign the lanes end with)
    runs; k = 1536 leaves the second wave of a row half empty. Tiny, huge, zero and subnormal rows,
    against the oracle bit for bit."""
    _, detrt = _mods()
    rng = np.random.default_rng(rows + k + bs)
    x = rng.standard_normal((rows, k)).astype(np.float32) * np.exp(rng.uniform(-30, 30, size=(rows, 1))).astype(np.float32)
    x[0] = 0.0
    x[1] *= np.float32(1e-38)
    x[2, 7] = 3.0e38
    x[3, :] = np.float32(-2.5)  # equal values: the transform concentrates them in few lanes
    q, s = detrt.quant_act(torch.from_numpy(x).to(dev), bs)
    wq, ws = O.quant_act(x, bs)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))


@pytest.mark.parametrize("k,bs", [(2048, 512), (6144, 512), (4096, 128), (14336, 128), (2048, 0), (128, 64),
                                  (4096, 512), (4608, 512), (1536, 1), (512, 8), (640, 128), (4096, 1024)])
def test_quant_act_random_rows(dev, k, bs):
    """fp32 sweep: IEEE adds, max, divide, rint and sqrt on gfx950 equal x86 SSE bit for bit,
    including tiny, huge and all-zero rows (runtime/tests/test_fp32_native.py)."""
    _, detrt = _mods()
    rng = np.random.default_rng(k + bs)
    rows = 96
    x = rng.standard_normal((rows, k)).astype(np.float32) * np.exp(rng.uniform(-30, 30, size=(rows, 1))).astype(np.float32)
    x[0] = 0.0
    x[1] *= np.float32(1e-38)  # subnormal inputs
    x[2, 7] = 3.0e38
    q, s = detrt.quant_act(torch.from_numpy(x).to(dev), bs)
    wq, ws = O.quant_act(x, bs)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))


def test_det_linear_call_matches_oracle(dev):
    """DetLinear(W) quantizes W on the GPU exactly as detrt does on the CPU, and __call__ is
    quant_act -> exact GEMM -> dequant (qwen3.py:71-126), at the Qwen3-1.7B MLP-up shape."""
    _, detrt = _mods()
    rng = np.random.default_rng(21)
    W = (rng.standard_normal((6144, 2048)) * 0.02).astype(np.float32)
    x = rng.standard_normal((64, 2048)).astype(np.float32)
    lay = detrt.DetLinear(torch.from_numpy(W), dev, 512, mine=False)
    Wq, sw, bs = O.quant_weight(W, 512)
    assert lay.bs == bs
    assert np.array_equal(lay.Wq.cpu().numpy(), Wq)
    assert np.array_equal(lay.sw.cpu().numpy().view(np.uint32), sw.view(np.uint32))
    y = lay(torch.from_numpy(x).to(dev))
    _, _, _, want = O.det_linear(x, Wq, sw, bs)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("m,n,k", [(4096, 4096 + 128, 1024), (4096, 4096 + 384, 256)])
def test_column_split_gemm_all_out_modes(dev, m, n, k):
    """n not a multiple of 256 with enough 256 x 256 tiles to fill the CUs (a vocabulary-sized
    lm_head): the column split (256 x 256 tiles, then a 128 x 128 tail writing into the same rows)
    gives the exact product and the exact fused epilogues."""
    ops, _ = _mods()
    from uwc_amd import _lib
    rng = np.random.default_rng(n + k)
    A = rng.integers(-128, 128, size=(m, k), dtype=np.int8)
    B = rng.integers(-128, 128, size=(n, k), dtype=np.int8)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    ref = O.igemm(A, B)
    assert np.array_equal(ops.igemm_i32(At, Bt).cpu().numpy(), ref)
    sx = rng.uniform(1e-3, 1.0, m).astype(np.float32)
    sw = rng.uniform(1e-3, 1.0, n).astype(np.float32)
    Y = torch.empty((m, n), dtype=torch.float32, device=dev)
    sxt, swt = torch.from_numpy(sx).to(dev), torch.from_numpy(sw).to(dev)  # held until the launch has run
    _lib.call("uwc_igemm_dequant_f32", At.data_ptr(), Bt.data_ptr(), m, n, k, sxt.data_ptr(), swt.data_ptr(),
              Y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(Y.cpu().numpy().view(np.uint32), O.dequant(ref, sx, sw).view(np.uint32))


@pytest.mark.parametrize("m,n", [(1, 1), (3, 4), (7, 6), (5, 151936), (70000, 8), (65537, 12)])
def test_dequant_every_layout(dev, m, n):
    """uwc_dequant_f32 equals the oracle's (f32(acc) * sx[row]) * sw[col] bit for bit: the
    four-column form (n % 4 == 0, rows on grid y, more rows than the grid's 65535 taking the row
    loop) and the element form (n % 4 != 0)."""
    _, detrt = _mods()
    rng = np.random.default_rng(m * 7 + n)
    acc = rng.integers(-2**31, 2**31 - 1, size=(m, n), dtype=np.int64).astype(np.int32)
    sx = rng.uniform(1e-6, 1e-2, m).astype(np.float32)
    sw = rng.uniform(1e-6, 1e-2, n).astype(np.float32)
    y = detrt.dequant(torch.from_numpy(acc).to(dev), torch.from_numpy(sx).to(dev), torch.from_numpy(sw).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), O.dequant(acc, sx, sw).view(np.uint32))
