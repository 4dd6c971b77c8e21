"""GPU parity of the miner's activation quantizer and the HF-model caller (uwc_amd.model):
quant_rows_had against the reference's published L2 known answers and the CPU oracle, and
MinedLinear in "mined" / "plain" mode bit-identical to "int" and to the oracle's integer math
(miner/ampere/tests/test_model.py, results/xc_cpu.json:5-10)."""
import hashlib

import numpy as np
import pytest
import torch

import oracle as O
from test_oracle import L2_KAT, l2_quantizer_input

pytestmark = pytest.mark.gpu


def _bf16(x: np.ndarray, dev) -> torch.Tensor:
    """fp32 rows whose values are already bf16-exact, as a bf16 device tensor."""
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev).to(torch.bfloat16)


@pytest.mark.parametrize("bs", [0, 128, 512])
def test_quant_rows_had_known_answers_L2(dev, bs):
    from uwc_amd import ops
    x = _bf16(l2_quantizer_input(), dev)
    q, s = ops.quant_rows_had(x, bs)
    assert hashlib.sha256(q.cpu().numpy().tobytes()).hexdigest()[:20] == L2_KAT[bs][0]
    assert hashlib.sha256(s.cpu().numpy().tobytes()).hexdigest()[:20] == L2_KAT[bs][1]


@pytest.mark.parametrize("m,k,bs", [(64, 17408, 512), (33, 2560, 128), (7, 1000, 8), (300, 2560, 0), (5, 24, 8)])
def test_quant_rows_had_matches_oracle(dev, m, k, bs):
    """Wide rows (Qwen3-14B down_proj input, the register path with a reload pass), rows that are
    not a multiple of 512 (the LDS path), tiny and unrotated rows."""
    from uwc_amd import ops
    rng = np.random.default_rng(m + k + bs)
    x = (rng.standard_normal((m, k)) * np.linspace(0.1, 8, k)).astype(np.float32)
    xb = torch.from_numpy(x).to(dev).to(torch.bfloat16)
    q, s = ops.quant_rows_had(xb, bs)
    wq, ws = O.quant_act(xb.float().cpu().numpy(), bs, 64)
    assert np.array_equal(q.cpu().numpy(), wq)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ws.view(np.uint32))


def test_fused_quantizer_matches_torch_rotation(dev):
    """The FWHT quantizer agrees with the torch matmul rotation up to float rounding ties
    (miner/ampere/tests/test_model.py:26-36)."""
    from uwc_amd import model as M
    from uwc_amd import ops
    torch.manual_seed(1)
    x = (torch.randn(300, 2560, device=dev) * torch.linspace(0.1, 8, 2560, device=dev)).to(torch.bfloat16)
    for bs in (0, 128, 512):
        q, s = ops.quant_rows_had(x, bs)
        H = M.hadamard(bs, dev) if bs else None
        qr, sr = M.quant_rows(M.rotate(x.float(), H))
        assert torch.allclose(s, sr, rtol=1e-5)
        assert (q.int() - qr.int()).abs().max().item() <= 1
        assert (q != qr).float().mean().item() < 1e-3


def test_mined_equals_int_and_plain(dev):
    """MinedLinear in "mined" mode (commit + noise + hashed GEMM + exact denoise, bf16 out) is
    bit-identical to "int" and "plain"; "int" equals the oracle's quantizer -> exact GEMM ->
    bf16((f32(acc) * sx) * sw) (miner/ampere/tests/test_model.py:9-22)."""
    import torch.nn as nn
    from uwc_amd import model as M
    torch.manual_seed(0)
    lins = [nn.Linear(2560, 4096, bias=False), nn.Linear(2560, 1024, bias=False)]
    a = M.MinedLinear(lins, dev, mode="int")
    b = M.MinedLinear(lins, dev, mode="mined")
    c = M.MinedLinear(lins, dev, mode="plain")
    assert b.mineable and torch.equal(a.Wq, b.Wq) and torch.equal(a.sw, b.sw)
    b.setup_block(lambda k: bytes(32), lambda k: np.zeros(8, np.uint32))
    x = torch.randn(3, 333, 2560, device=dev, dtype=torch.bfloat16)  # m = 999 -> padded to 1024
    ya, yb, yc = a(x), b(x), c(x)
    assert ya.shape == yb.shape == (3, 333, 5120)
    assert torch.equal(ya, yb) and torch.equal(ya, yc)
    ref = x.float() @ torch.cat([l.weight for l in lins]).to(dev).t()
    rel = ((ya.float() - ref).norm() / ref.norm()).item()
    assert rel < 0.03, rel
    # the integer math itself, on the CPU oracle
    xq, sx = O.quant_act(x.reshape(-1, 2560).float().cpu().numpy(), 512, 64)
    acc = O.igemm(xq, a.Wq.cpu().numpy())
    want = O.scale_bf16(acc, sx, a.sw.cpu().numpy())
    assert np.array_equal(ya.reshape(-1, 5120).cpu().view(torch.int16).numpy().view(np.uint16), want)
    assert b.hashed_macs == 1024 * 5120 * 2560 and b.useful_macs == 999 * 5120 * 2560


def test_decode_rows_and_bias(dev):
    """Small m (decode) through the int path, with a bias: y = bf16 product + bias."""
    import torch.nn as nn
    from uwc_amd import model as M
    torch.manual_seed(3)
    lin = nn.Linear(2048, 384, bias=True)
    a = M.MinedLinear([lin], dev, mode="int")
    x = torch.randn(5, 2048, device=dev, dtype=torch.bfloat16)
    y = a(x)
    xq, sx = O.quant_act(x.float().cpu().numpy(), 512, 64)
    want = O.scale_bf16(O.igemm(xq, a.Wq.cpu().numpy()), sx, a.sw.cpu().numpy())
    prod = torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).to(dev)
    assert torch.equal(y, prod + lin.bias.detach().to(dev, torch.bfloat16))


def test_convert_qwen3_mined_forward_equals_int(dev):
    """convert_qwen3 on a small random Qwen3 (2 layers, hidden 2048, every linear mineable): the
    mined model's logits equal the int model's bit for bit, and track the float model. The model
    runs in fp32 with eager attention (the rest of the model is plain torch)."""
    transformers = pytest.importorskip("transformers")
    from uwc_amd import model as M
    cfg = transformers.Qwen3Config(vocab_size=2048, hidden_size=2048, intermediate_size=2048, num_hidden_layers=2,
                                   num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                                   max_position_embeddings=256, tie_word_embeddings=False)
    cfg._attn_implementation = "eager"
    torch.manual_seed(4)
    base = transformers.Qwen3ForCausalLM(cfg).eval()
    sd = base.state_dict()
    ids = torch.randint(0, 2048, (2, 64), device=dev)

    def build(mode):
        mdl = transformers.Qwen3ForCausalLM(cfg).eval()
        mdl.load_state_dict(sd)
        mls = M.convert_qwen3(mdl, dev, mode=mode, hadamard_block=512)
        for ml in mls:  # the model runs in fp32: hand the bf16 linear outputs on as fp32 (exact)
            ml.register_forward_hook(lambda mod, inp, out: out.float())
        mdl.to(dev)
        return mdl, mls

    ref_model = base.to(dev)
    with torch.no_grad():
        ref = ref_model(input_ids=ids).logits.float()
    m_int, _ = build("int")
    m_mined, mls = build("mined")
    assert all(ml.mineable for ml in mls)
    for ml in mls:
        ml.setup_block(lambda k: bytes(range(32)), lambda k: np.full(8, 0xFFFFFFFF, np.uint32))
    with torch.no_grad():
        li = m_int(input_ids=ids).logits
        lm = m_mined(input_ids=ids).logits
    assert torch.equal(li, lm)
    assert sum(ml.hashed_macs for ml in mls) > 0
    cos = torch.nn.functional.cosine_similarity(li.float().flatten(), ref.flatten(), dim=0).item()
    assert cos > 0.95, cos
