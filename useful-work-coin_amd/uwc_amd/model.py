"""Integer-only linear layers for Hugging Face Qwen3 models, mined with cuPOW on MI355X: the call
surface of the reference's miner/ampere/uwc_ampere/model.py (MinedLinear, convert_qwen3) over
this package's HIP kernels.

Quantization (model.py:1-17):
  weights      per-output-channel symmetric, W' = W H, s_w = max|W'_row| / 64
  activations  per-token symmetric (dynamic), x' = x H, s_x = max|x'_row| / 64 (quant_rows_had)
  y = bf16((f32(q(x') q(W')^T) * s_x) * s_w)  (+ bias)
H is an optional block-diagonal Walsh-Hadamard rotation (orthonormal).

Modes per layer (model.py:8-16):
  "bf16"  original weights (baseline, torch)
  "int"   the same integer math, no mining: quant_rows_had -> exact int8 GEMM with the bf16
          scaling epilogue (libuwc_hip's plain GEMM; the reference used cuBLAS int8 here, and an
          fp32 matmul for m < 17 that is exact only while every partial sum stays below 2^24:
          this mirror uses the exact integer GEMM for every m)
  "plain" the same integer math through the mining GEMM kernel with no transcript
  "mined" MinedWeight.forward: commit + noise + hashed GEMM + exact denoise, bit-identical to "int"
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

QMAX = 64


def hadamard(n: int, device, dtype=torch.float32) -> torch.Tensor:
    """Orthonormal Sylvester Hadamard matrix of size n (a power of two) (model.py:30-35)."""
    if n & (n - 1):
        raise AssertionError(f"hadamard: n={n} is not a power of two")
    H = torch.ones(1, 1)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return (H / math.sqrt(n)).to(device=device, dtype=dtype)


def rotate(x: torch.Tensor, H: torch.Tensor | None) -> torch.Tensor:
    """x rotated block-wise by H along the last dim (model.py:38-43)."""
    if H is None:
        return x
    bs = H.shape[0]
    shp = x.shape
    return (x.reshape(*shp[:-1], shp[-1] // bs, bs).to(H.dtype) @ H).reshape(shp)


def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-row quantization to int8 values in [-64, 64] (model.py:46-51)."""
    xf = x.float()
    s = xf.abs().amax(dim=-1, keepdim=True).clamp_min(1e-8) / QMAX
    q = torch.round(xf / s).clamp_(-QMAX, QMAX).to(torch.int8)
    return q, s.squeeze(-1)


class MinedLinear(nn.Module):
    """Replacement for one or more nn.Linear layers that share an input (fused along n)
    (model.py:54-141)."""

    def __init__(self, linears: list[nn.Linear], device, mode: str = "mined", hadamard_block: int = 512,
                 r: int = 128, cfg: str | None = None):
        super().__init__()
        if mode not in ("bf16", "int", "plain", "mined"):
            raise ValueError(f"MinedLinear: unknown mode {mode!r}")
        self.mode = mode
        self.splits = [l.out_features for l in linears]
        W = torch.cat([l.weight.detach() for l in linears], 0)
        bias = [l.bias for l in linears]
        self.bias = None if all(b is None for b in bias) else torch.cat(
            [b.detach() if b is not None else torch.zeros(l.out_features) for b, l in zip(bias, linears)]
        ).to(device, torch.bfloat16)
        self.n, self.k = W.shape
        self.H = None
        if hadamard_block:
            bs = min(hadamard_block, self.k & -self.k)
            self.H = hadamard(bs, device)
        if mode == "bf16":
            self.W = W.to(device=device, dtype=torch.bfloat16)
        else:
            # quantize in row chunks on the GPU so huge layers (lm_head) never need a full fp32 copy
            qs, ss = [], []
            for s0 in range(0, self.n, 16384):
                q, sc = quant_rows(rotate(W[s0:s0 + 16384].to(device=device, dtype=torch.float32), self.H))
                qs.append(q)
                ss.append(sc)
            self.Wq, self.sw = torch.cat(qs).contiguous(), torch.cat(ss).contiguous()
        del W
        self.r = r
        self.cfg = cfg or ops.DEFAULT_CFG
        self.bn = ops.BN
        self.mw: ops.MinedWeight | None = None
        self.hashed_macs = 0  # m_pad * n * k summed over mined calls
        self.useful_macs = 0  # m * n * k summed over calls

    @property
    def mineable(self) -> bool:
        """Shapes the mining path takes (model.py:93-97)."""
        k, n, r = self.k, self.n, self.r
        return k >= max(1024, 16 * r) and k % r == 0 and k % 64 == 0 and k <= 4 * r * r and n % self.bn == 0

    def setup_block(self, job_key_for_k, bound_for_k):
        """job_key_for_k(k) -> 32-byte job key; bound_for_k(k) -> 8 target words."""
        if self.mode != "mined" or not self.mineable:
            return
        if self.mw is None:
            self.mw = ops.MinedWeight(Bt=self.Wq, b_scale=self.sw, r=self.r)
        self.mw.setup_block(job_key_for_k(self.k), bound_for_k(self.k))

    def _int_forward(self, xq: torch.Tensor, sx: torch.Tensor) -> torch.Tensor:
        """bf16((f32(xq @ Wq^T) * sx) * sw) with the exact integer GEMM (any m)."""
        y = torch.empty((xq.shape[0], self.n), dtype=torch.bfloat16, device=xq.device)
        ops.gemm(xq, self.Wq, a_scale=sx, b_scale=self.sw, out=y, out_mode=ops.OUT_BF16)
        return y

    @torch.compiler.disable
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shp = x.shape
        x2 = x.reshape(-1, self.k)
        m = x2.shape[0]
        if self.mode == "bf16":
            y = F.linear(x2.to(torch.bfloat16), self.W)
        else:
            bs = self.H.shape[0] if self.H is not None else 0
            kernel_path = self.mode in ("mined", "plain") and self.mineable
            mp = -(-m // ops.BM) * ops.BM if kernel_path else m
            xb = x2.to(torch.bfloat16)
            if mp != m:
                xb = F.pad(xb, (0, 0, 0, mp - m))
            xq, sx = ops.quant_rows_had(xb.contiguous(), bs)  # fused rotate + quantize
            if self.mode == "mined" and self.mineable:
                if self.mw is None:
                    raise RuntimeError("MinedLinear: call setup_block() before a mined forward")
                y = self.mw.forward(xq.contiguous(), sx.contiguous())[:m]
                self.hashed_macs += mp * self.n * self.k
            elif self.mode == "plain" and self.mineable:
                y = torch.empty((mp, self.n), dtype=torch.bfloat16, device=xq.device)
                ops.gemm(xq, self.Wq, a_scale=sx, b_scale=self.sw, out=y, out_mode=ops.OUT_BF16, cfg=self.cfg)
                y = y[:m]
            else:
                y = self._int_forward(xq.contiguous(), sx)
        self.useful_macs += m * self.n * self.k
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*shp[:-1], self.n)


class _Slice(nn.Module):
    """k_proj / v_proj / up_proj stand-in: returns its slice of the fused output computed by the
    head layer (model.py:144-157)."""

    def __init__(self, head: "_FusedHead", idx: int):
        super().__init__()
        self.head, self.idx = head, idx

    @torch.compiler.disable
    def forward(self, x):
        if self.head.last_input is not x:
            raise AssertionError("fused layers must be called with the same input tensor, in order")
        y = self.head.outputs[self.idx]
        if self.idx == len(self.head.outputs) - 1:  # last consumer: drop the references
            self.head.outputs = self.head.last_input = None
        return y


class _FusedHead(nn.Module):
    """The first of a fused group: runs the MinedLinear and keeps the split outputs (model.py:160-172)."""

    def __init__(self, ml: MinedLinear):
        super().__init__()
        self.ml = ml
        self.last_input = None
        self.outputs = None

    @torch.compiler.disable
    def forward(self, x):
        y = self.ml(x)
        self.last_input = x
        self.outputs = torch.split(y, self.ml.splits, dim=-1)
        return self.outputs[0]


def convert_qwen3(model, device, mode="mined", hadamard_block=512, mine_lm_head=True, cfg=None) -> list[MinedLinear]:
    """Swap every linear in a HF Qwen3 model (q/k/v fused, gate/up fused). Returns the MinedLinears
    (model.py:175-197)."""
    mls = []
    base = model.model if hasattr(model, "model") else model  # CausalLM or bare Qwen3Model (embeddings)
    for layer in base.layers:
        at, mlp = layer.self_attn, layer.mlp
        qkv = MinedLinear([at.q_proj, at.k_proj, at.v_proj], device, mode, hadamard_block, cfg=cfg)
        head = _FusedHead(qkv)
        at.q_proj, at.k_proj, at.v_proj = head, _Slice(head, 1), _Slice(head, 2)
        o = MinedLinear([at.o_proj], device, mode, hadamard_block, cfg=cfg)
        at.o_proj = o
        gu = MinedLinear([mlp.gate_proj, mlp.up_proj], device, mode, hadamard_block, cfg=cfg)
        head2 = _FusedHead(gu)
        mlp.gate_proj, mlp.up_proj = head2, _Slice(head2, 1)
        d = MinedLinear([mlp.down_proj], device, mode, hadamard_block, cfg=cfg)
        mlp.down_proj = d
        mls += [qkv, o, gu, d]
    if mine_lm_head and hasattr(model, "lm_head"):
        lm = MinedLinear([model.lm_head], device, mode, hadamard_block, cfg=cfg)
        model.lm_head = lm
        mls.append(lm)
    return mls
