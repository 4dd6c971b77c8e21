"""Integer linear layers for Hugging Face Qwen3 models, mined with cuPOW on MI355X: the public
surface of the reference's miner/ampere/uwc_ampere/model.py (hadamard, rotate, quant_rows,
MinedLinear, convert_qwen3) over this package's HIP kernels.

The integer math of a layer (model.py:1-17): weights quantized once per output row and activations
per token, both symmetric to [-64, 64] after an optional block-diagonal orthonormal Walsh-Hadamard
rotation of the k axis; the output is bf16((f32(q_x q_W^T) * s_x) * s_w) (+ bias), computed with
the exact int8 GEMM, so every mode below except "bf16" produces the same bits.

  "bf16"   the original weights in bf16 (baseline);
  "int"    the integer math through the plain exact GEMM, any number of rows;
  "plain"  the integer math through the mining GEMM kernel with no transcript (a provider that
           does not mine), for mineable shapes;
  "mined"  MinedWeight.forward: commitment, noise, hashed GEMM and exact denoise, for mineable
           shapes.
A shape that cannot be mined runs the "int" math in every integer mode.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops

QMAX = 64
MODES = ("bf16", "int", "plain", "mined")


def hadamard(n: int, device, dtype=torch.float32) -> torch.Tensor:
    """The orthonormal Sylvester-Hadamard matrix of order n (a power of two): entry (i, j) is
    (-1)^popcount(i & j) / sqrt(n) (model.py:30-35)."""
    if n < 1 or n & (n - 1):
        raise AssertionError(f"hadamard: n={n} is not a power of two")
    idx = torch.arange(n)
    both = idx[:, None] & idx[None, :]
    parity = torch.zeros_like(both)
    while bool(both.any()):
        parity ^= both & 1
        both = both >> 1
    return ((1 - 2 * parity).to(torch.float32) / math.sqrt(n)).to(device=device, dtype=dtype)


def rotate(x: torch.Tensor, H: torch.Tensor | None) -> torch.Tensor:
    """x with every block of H.shape[0] consecutive entries of its last axis multiplied by H
    (model.py:38-43); the identity without H."""
    if H is None:
        return x
    blocks = x.to(H.dtype).unflatten(-1, (-1, H.shape[0]))
    return torch.matmul(blocks, H).flatten(-2)


def quant_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-row quantization (model.py:46-51): s = max(max|x_row|, 1e-8) / 64,
    q = round-half-even(x / s) clamped to [-64, 64]; returns (int8 q, fp32 s per row)."""
    xf = x.to(torch.float32)
    scale = torch.clamp(xf.abs().amax(-1), min=1e-8) / QMAX
    q = torch.clamp(torch.round(xf / scale.unsqueeze(-1)), -QMAX, QMAX)
    return q.to(torch.int8), scale


def mineable_shape(n: int, k: int, r: int, tile_n: int) -> bool:
    """Shapes the mining path takes (model.py:93-97): k at least max(1024, 16 r) and at most 4 r^2
    (Pearl's rank rule), k a multiple of r and of the 64-wide k step, n a multiple of the GEMM
    tile's N."""
    return max(1024, 16 * r) <= k <= 4 * r * r and k % r == 0 and k % 64 == 0 and n % tile_n == 0


class MinedLinear(nn.Module):
    """One nn.Linear, or several that read the same input concatenated along n, as an integer
    linear that can mine (model.py:54-141). `splits` are the fused layers' output widths."""

    def __init__(self, linears: list[nn.Linear], device, mode: str = "mined", hadamard_block: int = 512,
                 r: int = 128, cfg: str | None = None):
        super().__init__()
        if mode not in MODES:
            raise ValueError(f"MinedLinear: unknown mode {mode!r} (one of {MODES})")
        self.mode, self.r = mode, r
        self.cfg = cfg or ops.DEFAULT_CFG
        self.splits = [lin.out_features for lin in linears]
        self.k = linears[0].in_features
        self.n = sum(self.splits)
        self.bias = self._fused_bias(linears, device)
        self.H = hadamard(min(hadamard_block, self.k & -self.k), device) if hadamard_block else None
        self.mw: ops.MinedWeight | None = None
        self.hashed_macs = 0  # padded rows * n * k over mined calls
        self.useful_macs = 0  # rows * n * k over all calls
        if mode == "bf16":
            self.W = torch.cat([lin.weight.detach().to(device, torch.bfloat16) for lin in linears])
        else:
            self.Wq, self.sw = self._quantize_weights(linears, device)
        self._run = {"bf16": self._run_bf16, "int": self._run_int, "plain": self._run_plain,
                     "mined": self._run_mined}[mode]

    @staticmethod
    def _fused_bias(linears, device):
        if all(lin.bias is None for lin in linears):
            return None
        parts = [lin.bias.detach() if lin.bias is not None else lin.weight.new_zeros(lin.out_features)
                 for lin in linears]
        return torch.cat([p.to(device) for p in parts]).to(torch.bfloat16)

    def _quantize_weights(self, linears, device, rows_per_pass: int = 8192):
        """Rotate and quantize the weight rows on the GPU a slab at a time (an lm_head never needs
        a full fp32 copy on the device)."""
        qs, ss = [], []
        for lin in linears:
            W = lin.weight.detach()
            for r0 in range(0, W.shape[0], rows_per_pass):
                slab = W[r0:r0 + rows_per_pass].to(device=device, dtype=torch.float32)
                q, s = quant_rows(rotate(slab, self.H))
                qs.append(q)
                ss.append(s)
        return torch.cat(qs).contiguous(), torch.cat(ss).contiguous()

    @property
    def mineable(self) -> bool:
        return mineable_shape(self.n, self.k, self.r, ops.BN)

    def setup_block(self, job_key_for_k, bound_for_k):
        """Prepare the mined mode for a block template: job_key_for_k(k) -> 32-byte job key,
        bound_for_k(k) -> 8 little-endian target words. No-op for other modes and unmineable
        shapes."""
        if self.mode != "mined" or not self.mineable:
            return
        if self.mw is None:
            self.mw = ops.MinedWeight(Bt=self.Wq, b_scale=self.sw, r=self.r)
        self.mw.setup_block(job_key_for_k(self.k), bound_for_k(self.k))

    # ---- the integer paths: bf16 rows in, bf16 rows out
    def _quantize_acts(self, rows: torch.Tensor, pad_to: int = 1):
        """Rotation and quantization fused in one kernel; rows padded with zeros to a multiple of
        pad_to (zero rows quantize to zero and are cut from the output)."""
        extra = -rows.shape[0] % pad_to
        xb = rows.to(torch.bfloat16)
        if extra:
            xb = F.pad(xb, (0, 0, 0, extra))
        return ops.quant_rows_had(xb.contiguous(), self.H.shape[0] if self.H is not None else 0)

    def _exact_bf16(self, xq: torch.Tensor, sx: torch.Tensor) -> torch.Tensor:
        y = torch.empty((xq.shape[0], self.n), dtype=torch.bfloat16, device=xq.device)
        ops.gemm(xq, self.Wq, a_scale=sx, b_scale=self.sw, out=y, out_mode=ops.OUT_BF16)
        return y

    def _run_bf16(self, rows: torch.Tensor) -> torch.Tensor:
        return F.linear(rows.to(torch.bfloat16), self.W)

    def _run_int(self, rows: torch.Tensor) -> torch.Tensor:
        xq, sx = self._quantize_acts(rows)
        return self._exact_bf16(xq, sx)

    def _run_plain(self, rows: torch.Tensor) -> torch.Tensor:
        if not self.mineable:
            return self._run_int(rows)
        xq, sx = self._quantize_acts(rows, ops.BM)
        y = torch.empty((xq.shape[0], self.n), dtype=torch.bfloat16, device=xq.device)
        ops.gemm(xq, self.Wq, a_scale=sx, b_scale=self.sw, out=y, out_mode=ops.OUT_BF16, cfg=self.cfg)
        return y[:rows.shape[0]]

    def _run_mined(self, rows: torch.Tensor) -> torch.Tensor:
        if not self.mineable:
            return self._run_int(rows)
        if self.mw is None:
            raise RuntimeError("MinedLinear: setup_block() must run before a mined forward")
        xq, sx = self._quantize_acts(rows, ops.BM)
        self.hashed_macs += xq.shape[0] * self.n * self.k
        return self.mw.forward(xq, sx.contiguous(), out_mode=ops.OUT_BF16)[:rows.shape[0]]

    @torch.compiler.disable
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rows = x.reshape(-1, self.k)
        y = self._run(rows)
        self.useful_macs += rows.shape[0] * self.n * self.k
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*x.shape[:-1], self.n)


class _SharedOutput:
    """The fused output of one MinedLinear for the input it was last called with, handed out a
    slice at a time to the modules that stand in for the original linears. A slice is served
    from the cache while the input is the same tensor object at the same version (the cache
    holds the input itself, so a later tensor that reuses its address never matches); once
    every part has taken its slice the cache and the input are dropped, so no activation
    outlives its layer."""

    def __init__(self, ml: MinedLinear):
        self.ml = ml
        self._x = None
        self._version = None
        self._parts = None
        self._pending = 0

    def part(self, x: torch.Tensor, index: int) -> torch.Tensor:
        if self._parts is None or self._x is not x or self._version != x._version:
            self._parts = torch.split(self.ml(x), self.ml.splits, dim=-1)
            self._x, self._version, self._pending = x, x._version, len(self._parts)
        y = self._parts[index]
        self._pending -= 1
        if self._pending == 0:
            self._parts = self._x = self._version = None
        return y


class _Part(nn.Module):
    """Stands in for one of the linears fused into a MinedLinear (q/k/v, gate/up)."""

    def __init__(self, shared: _SharedOutput, index: int):
        super().__init__()
        self.shared, self.index = shared, index
        if index == 0:  # the group's parameters live in the module tree once, under its first part
            self.ml = shared.ml

    @torch.compiler.disable
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.shared.part(x, self.index)


def _fuse(parent: nn.Module, names: list[str], device, mode, hadamard_block, cfg) -> MinedLinear:
    """Replace parent.<name> for every name by one MinedLinear over all of them."""
    ml = MinedLinear([getattr(parent, nm) for nm in names], device, mode, hadamard_block, cfg=cfg)
    if len(names) == 1:
        setattr(parent, names[0], ml)
    else:
        shared = _SharedOutput(ml)
        for i, nm in enumerate(names):
            setattr(parent, nm, _Part(shared, i))
    return ml


def convert_qwen3(model, device, mode="mined", hadamard_block=512, mine_lm_head=True, cfg=None) -> list[MinedLinear]:
    """Replace every linear of a Hugging Face Qwen3 model (a CausalLM or a bare Qwen3Model) by a
    MinedLinear, q/k/v and gate/up fused; returns them per layer (qkv, o, gate_up, down), then
    the lm_head (model.py:175-197)."""
    decoder = getattr(model, "model", model)
    out = []
    for layer in decoder.layers:
        att, mlp = layer.self_attn, layer.mlp
        for parent, group in ((att, ["q_proj", "k_proj", "v_proj"]), (att, ["o_proj"]),
                              (mlp, ["gate_proj", "up_proj"]), (mlp, ["down_proj"])):
            out.append(_fuse(parent, group, device, mode, hadamard_block, cfg))
    if mine_lm_head and hasattr(model, "lm_head"):
        out.append(_fuse(model, ["lm_head"], device, mode, hadamard_block, cfg))
    return out
