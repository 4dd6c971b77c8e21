"""detrt's deterministic integer linear on MI355X: the call surface of runtime/detrt/qwen3.py:71-126
(DetLinear) and runtime/detrt/core.py:162-195 (quant_act), over libuwc_hip.so.

Bit-identical to the reference CPU path (fp64 GEMM of int8 values, emulated fp32 elementwise):
int8 x int8 sums are exact in int32, and every fp32 step of quant_act and the dequant
(f32(acc) * s_x) * s_w is one correctly rounded IEEE op in the reference's order.
"""
from __future__ import annotations

import torch

from . import _lib
from . import ops


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def hadamard_bs(hadamard_block: int, k: int) -> int:
    """DetLinear's block size: min(Bs, k & -k), or 0 without rotation (qwen3.py:76)."""
    return min(hadamard_block, k & -k) if hadamard_block else 0


def quant_act(x: torch.Tensor, bs: int, qmax: int = 64) -> tuple[torch.Tensor, torch.Tensor]:
    """q = round(y / s), s = max|y| / qmax with y = fwht(x, bs); returns (int8 q, fp32 scale s / sqrt(bs))."""
    x = x.contiguous()
    if x.dtype != torch.float32:
        x = x.to(torch.float32)
    rows, k = x.shape
    if bs > 1 and k % bs:
        raise AssertionError(f"quant_act: bs={bs} must divide k={k}")
    q = torch.empty((rows, k), dtype=torch.int8, device=x.device)
    s = torch.empty(rows, dtype=torch.float32, device=x.device)
    _lib.call("uwc_quant_act_f32", x.data_ptr(), rows, k, bs, qmax, q.data_ptr(), s.data_ptr(), _stream())
    return q, s


def quant_sym(x: torch.Tensor, qmax: int) -> tuple[torch.Tensor, torch.Tensor]:
    """core.quant_sym per row of a 2-D tensor (no rotation): (integer-valued q as int8, scale)."""
    return quant_act(x, 0, qmax)


def dequant(acc: torch.Tensor, sx: torch.Tensor, sw: torch.Tensor) -> torch.Tensor:
    """fmul(fmul(f32(acc), s_x), s_w) for an int32 accumulator."""
    m, n = acc.shape
    y = torch.empty((m, n), dtype=torch.float32, device=acc.device)
    _lib.call("uwc_dequant_f32", acc.contiguous().data_ptr(), sx.contiguous().data_ptr(), sw.contiguous().data_ptr(),
              m, n, y.data_ptr(), _stream())
    return y


class DetLinear:
    """int8 W7A7 linear: W -> Wq = quant_sym(fwht(W, bs), 64), s_w folded by 1/sqrt(bs);
    __call__(x) = (f32(quant_act(x) @ Wq^T) * s_x) * s_w.

    With mine=True, setup_block() prepares a MinedWeight (r = 128) for the layers detrt mines, and
    int_gemm() then runs the mined forward (hashed tiles, exact denoise, int32 out) instead of the
    plain GEMM: the same integers either way (qwen3.py:94-116)."""

    def __init__(self, W: torch.Tensor, device, hadamard_block: int, mine: bool = False):
        n, k = W.shape
        self.n, self.k, self.device = n, k, torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("uwc_amd.detrt.DetLinear runs on a GPU; the CPU reference is detrt itself")
        self.bs = hadamard_bs(hadamard_block, k)
        # quant_act applied to each weight row is exactly quant_sym(fwht(W, bs), 64) plus the fold
        Wd = W.detach().to(self.device, torch.float32).contiguous()
        qs, ss = [], []
        for s0 in range(0, n, 8192):
            q, s = quant_act(Wd[s0:s0 + 8192], self.bs)
            qs.append(q)
            ss.append(s)
        self.Wq = torch.cat(qs).contiguous()
        self.sw = torch.cat(ss).contiguous()
        self.mine = bool(mine)
        self.mw = None

    @classmethod
    def from_quantized(cls, Wq: torch.Tensor, sw: torch.Tensor, bs: int) -> "DetLinear":
        """A DetLinear over already quantized rows (e.g. a committed weights table)."""
        self = cls.__new__(cls)
        self.n, self.k = Wq.shape
        self.device = Wq.device
        self.bs = bs
        self.Wq = Wq.contiguous()
        self.sw = sw.to(torch.float32).contiguous()
        self.mine, self.mw = False, None
        return self

    # the layers detrt mines (qwen3.py:96): k >= 2048, k % 128 == 0 and n a multiple of the GEMM
    # tile's N, which is 128 in the reference's default configuration ("128x3", ops.py:35-37) and
    # is the hashed GEMM's requirement here (m, n % 128; 256-multiples take the large tiles)
    MINE_MIN_K = 2048

    def mineable(self) -> bool:
        return self.k >= self.MINE_MIN_K and self.k % 128 == 0 and self.n % ops.BN == 0

    def setup_block(self, job_key_for_k, bound_for_k):
        """Prepare this weight for mining under a block template (qwen3.py:94-104); a layer that
        cannot be mined stops trying (mine becomes False), as the reference does."""
        if not self.mine:
            return
        ok = self.mineable()
        if not ok:
            self.mine = False
            return
        if self.mw is None:
            self.mw = ops.MinedWeight(Bt=self.Wq, b_scale=self.sw, r=128)
        self.mw.setup_block(job_key_for_k(self.k), bound_for_k(self.k))

    def int_gemm(self, q: torch.Tensor) -> torch.Tensor:
        """Exact q @ Wq^T for int8 q (m x k), as int32."""
        m = q.shape[0]
        if self.mine and self.mw is not None:
            mp = -(-m // ops.BM) * ops.BM
            qp = torch.nn.functional.pad(q, (0, 0, 0, mp - m)) if mp != m else q
            ones = torch.ones(mp, dtype=torch.float32, device=q.device)
            return self.mw.forward(qp.contiguous(), ones, out_mode=ops.OUT_I32)[:m]
        return ops.igemm_i32(q.contiguous(), self.Wq)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        shp = x.shape
        q, sx = quant_act(x.reshape(-1, self.k), self.bs)
        if self.mine and self.mw is not None:
            y = dequant(self.int_gemm(q), sx, self.sw)
        else:
            y = torch.empty((q.shape[0], self.n), dtype=torch.float32, device=q.device)
            _lib.call("uwc_igemm_dequant_f32", q.data_ptr(), self.Wq.data_ptr(), q.shape[0], self.n, self.k,
                      sx.data_ptr(), self.sw.data_ptr(), y.data_ptr(), _stream())
        return y.reshape(*shp[:-1], self.n)
