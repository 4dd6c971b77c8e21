"""ctypes binding of libuwc_hip.so (the C-ABI declared in include/uwc.h).

The library is built in-tree by useful-work-coin_amd/csrc/build.sh (or __graft_entry__.build()).
There is no fallback: if the library is missing or a call fails, this module raises.
"""
from __future__ import annotations

import ctypes
import hashlib
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libuwc_hip.so")
HEADER_PATH = os.path.join(_HERE, "..", "..", "include", "uwc.h")

vp = ctypes.c_void_p
i32 = ctypes.c_int
u32 = ctypes.c_uint32
u64 = ctypes.c_uint64
i64 = ctypes.c_int64
f32 = ctypes.c_float

# name -> argument types (every function returns int status unless listed in _RESTYPE)
SIGNATURES = {
    "uwc_version": [],
    "uwc_last_error": [],
    "uwc_header_sha": [],
    "uwc_noisy_gemm": [vp, vp, i32, i32, i32, i32, vp, vp, vp, i32, vp, vp, vp, i32, vp, vp, vp, i32, i32, vp, vp],
    "uwc_noisy_gemm_many": [i32, vp, vp, i32, i32, i32, i32, vp, vp, vp, i32, vp, vp, vp, i32, vp, vp, vp, i32, i32, vp, vp],
    "uwc_igemm_i32": [vp, vp, i32, i32, i32, vp, vp],
    "uwc_igemm_dequant_f32": [vp, vp, i32, i32, i32, vp, vp, vp, vp],
    "uwc_igemm_dequant_residual_f32": [vp, vp, i32, i32, i32, vp, vp, vp, vp, vp],
    "uwc_b3_scratch_words": [u64],
    "uwc_b3_root_and_seed": [vp, u64, vp, vp, vp, u32, vp, vp, vp, u64, vp],
    "uwc_b3_root_and_seed_static": [vp, u64, vp, vp, vp, u32, vp, vp, vp],
    "uwc_b3_root_and_seed_many": [vp, i32, u64, vp, vp, vp, u32, vp, vp, vp, u64, vp],
    "uwc_noise_uniform": [vp, u32, vp, vp, vp, i32, vp],
    "uwc_noise_perm": [vp, u32, u32, vp, vp, vp],
    "uwc_noise_rows": [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp, i32, vp],
    "uwc_nonce_noise": [vp, i32, i32, vp, i32, vp, vp, vp, vp, vp, i32, vp, i32, vp],
    "uwc_nonce_noise_many": [i32, vp, i32, i32, vp, i32, vp, vp, vp, vp, vp, i32, vp, i32, vp],
    "uwc_proj_matrix": [vp, i32, i32, vp, vp],
    "uwc_project": [vp, i32, i32, i32, vp, vp, i32, vp, i32, vp],
    "uwc_noise_project": [vp, i32, i32, i32, vp, vp, vp, vp, vp, i32, i32, vp, i32, vp],
    "uwc_side_project": [vp, i32, vp, vp, vp, vp, vp, i32, i32, vp, i32, vp, vp, i32, i32, i32, vp, i32, vp],
    "uwc_side_project_many": [i32, vp, vp, vp, vp, vp, vp, i32, i32, vp, vp, vp, i32, i32, i32, i32, i32, vp, i32, vp],
    "uwc_quant_act_f32": [vp, i32, i32, i32, i32, vp, vp, vp],
    "uwc_quant_rows_had": [vp, i32, i32, i32, vp, vp, vp],
    "uwc_dequant_f32": [vp, vp, vp, i32, i32, vp, vp],
    "uwc_rmsnorm_quant_f32": [vp, vp, i32, i32, i32, f32, f32, vp, vp, vp],
    "uwc_rmsnorm_f32": [vp, vp, i32, i32, f32, f32, vp, vp],
    "uwc_qkv_post": [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32, vp, vp, vp, vp, vp, vp, vp, vp],
    "uwc_vt_tokens": [i32],
    "uwc_v_transpose": [vp, i32, i32, i32, i32, vp, vp],
    "uwc_attention": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, vp, vp],
    "uwc_attention_scratch_bytes": [i32, i32, i32],
    "uwc_attention_ws": [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, vp, vp, u64, vp],
    "uwc_swiglu_quant": [vp, vp, vp, i32, i32, i32, vp, vp, vp],
    "uwc_dequant_residual": [vp, vp, vp, vp, i32, i32, vp, vp],
    "uwc_embed_rows": [vp, i64, i32, vp, i32, vp, vp, vp],
    "uwc_sha_row_leaves": [vp, i64, i32, vp, i64, u32, u32, u32, vp, vp, vp],
    "uwc_sha_merkle_roots": [vp, i32, i32, vp, i64, vp, vp],
    "uwc_det_elementwise": [i32, vp, vp, vp, i64, vp],
    "uwc_mfma_rate_probe": [i32, i32, vp, i64, vp],
}
_RESTYPE = {"uwc_last_error": ctypes.c_char_p, "uwc_header_sha": ctypes.c_char_p,
            "uwc_attention_scratch_bytes": ctypes.c_uint64}

_LIB = None


class UwcError(RuntimeError):
    """A libuwc_hip call rejected its arguments or failed to launch."""


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built: run useful-work-coin_amd/csrc/build.sh "
                              "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        if os.path.exists(HEADER_PATH):  # the source tree's header: the library must be built from it
            with open(HEADER_PATH, "rb") as f:
                want = hashlib.sha256(f.read()).hexdigest()[:16]
            got = L.uwc_header_sha().decode()
            if got != want:
                raise ImportError(f"{LIB_PATH} was built from another include/uwc.h (stamp {got}, header {want}): "
                                  "rebuild with useful-work-coin_amd/csrc/build.sh (or __graft_entry__.build())")
        _LIB = L
    return _LIB


def call(name: str, *args) -> None:
    """Call an int-status entry point; raise UwcError with uwc_last_error() on failure."""
    st = getattr(lib(), name)(*args)
    if st != 0:
        msg = lib().uwc_last_error().decode(errors="replace")
        raise UwcError(f"{name} failed (status {st}): {msg}")
