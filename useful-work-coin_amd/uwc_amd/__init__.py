"""uwc_amd: the int8 x int8 -> int32 GEMM hot path of useful-work-coin on MI355X (gfx950).

  uwc_amd.ops     the miner's NoisyGEMM surface (gemm, MinedWeight, b3_root_and_seed, noise_*)
  uwc_amd.detrt   the deterministic runtime's linear (DetLinear, quant_act, dequant)

Both call libuwc_hip.so (include/uwc.h) through ctypes on torch's current stream.
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "detrt"]
