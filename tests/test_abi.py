"""The C-ABI library loads and exports every entry point include/uwc.h declares; argument checks
reject bad calls before any GPU work (so these run without a GPU)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "uwc.h")


def declared() -> list[str]:
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(uwc_\w+)\s*\(", src)))


def test_header_declares_expected_surface():
    names = declared()
    for must in ("uwc_noisy_gemm", "uwc_igemm_i32", "uwc_igemm_dequant_f32", "uwc_b3_root_and_seed",
                 "uwc_noise_uniform", "uwc_noise_perm", "uwc_noise_rows", "uwc_quant_act_f32", "uwc_dequant_f32",
                 "uwc_proj_matrix", "uwc_project", "uwc_noise_project", "uwc_nonce_noise", "uwc_last_error", "uwc_version",
                 "uwc_quant_rows_had", "uwc_side_project"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from uwc_amd import _lib
    L = _lib.lib()
    for name in declared():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, name
    assert L.uwc_version() == 1


def test_library_built_from_this_header():
    """The loader refuses a library stamped with another header's hash (argument lists would not
    match); the stamp is the first 16 hex digits of SHA-256 of include/uwc.h."""
    import hashlib
    from uwc_amd import _lib
    want = hashlib.sha256(open(HEADER, "rb").read()).hexdigest()[:16]
    assert _lib.lib().uwc_header_sha().decode() == want


def test_scratch_words_host_only():
    from uwc_amd import _lib
    L = _lib.lib()
    assert L.uwc_b3_scratch_words(1024) == 8
    assert L.uwc_b3_scratch_words(64 * 1024) == 8
    assert L.uwc_b3_scratch_words(65 * 1024) == 16
    # 16 MiB: 256 workgroup values
    assert L.uwc_b3_scratch_words(16 << 20) == 256 * 8
    # 1 GiB: 16384 values, then one level of 16 groups
    assert L.uwc_b3_scratch_words(1 << 30) == 16384 * 8 + 16 * 8


def test_attention_scratch_bytes_host_only():
    """The stored-exp attention's scratch: 4 KiB per (16-query block, 64-key tile) pair of the
    causal triangle, per sequence and head, then one float per query and head (the row max) from
    a 256-byte boundary."""
    from uwc_amd import _lib
    L = _lib.lib()
    rows = lambda B, T, H: (B * T * H * 4 + 255) // 256 * 256
    assert L.uwc_attention_scratch_bytes(0, 8, 1) == 0
    assert L.uwc_attention_scratch_bytes(1, 1, 1) == 4 * 4096 + 256       # 4 blocks of 16 in one 64-key tile
    assert L.uwc_attention_scratch_bytes(1, 65, 1) == 12 * 4096 + 512     # 4 blocks x 1 tile + 4 x 2
    # brute force over the blocks of 16 queries: block wq sees key tiles 0 .. wq / 4
    for T in (64, 100, 1000, 8192):
        Tp = (T + 63) // 64 * 64
        tiles = sum(wq // 4 + 1 for wq in range(Tp // 16))
        assert L.uwc_attention_scratch_bytes(3, T, 5) == 3 * 5 * tiles * 4096 + rows(3, T, 5)
    assert L.uwc_attention_scratch_bytes(1, 8192, 16) == 2164260864 + 8192 * 16 * 4


@pytest.mark.parametrize("kwargs,msg", [
    (dict(k=100), "multiple of 64"),
    (dict(flags=1, m=100), "mining needs"),
    (dict(flags=1, r=96), "power of two"),
    (dict(flags=2, corr=False), "needs corrA"),
    (dict(out_mode=7), "unknown out_mode"),
    (dict(out_mode=3, scales=False), "a_scale and b_scale"),
    (dict(flags=8), "unknown flags"),
    (dict(flags=0x1000), "unknown flags"),                     # a plain configuration without FLAG_PLAIN
    (dict(flags=0x200 | (9 << 12)), "configuration 9 unknown"),
    (dict(flags=0x200 | 1, m=128), "FLAG_PLAIN is for plain"),  # with FLAG_HASH
    (dict(flags=0x300), "FLAG_PLAIN is for plain"),             # with FLAG_TILE128
    (dict(flags=0x200 | (1 << 12), n=128), "does not take"),    # 128 x 256 tiles, n = 128
    (dict(flags=0x200, m=192), "does not take"),                # 128-row tiles, m = 192
])
def test_noisy_gemm_rejects_bad_arguments(kwargs, msg):
    from uwc_amd import _lib
    L = _lib.lib()
    a = dict(m=128, n=128, k=256, r=64, flags=0, out_mode=1, corr=True, scales=True)
    a.update(kwargs)
    fake = ctypes.c_void_p(1 << 20)  # aligned, never dereferenced: validation fails first
    corr = fake if a["corr"] else None
    sc = fake if a["scales"] else None
    st = L.uwc_noisy_gemm(fake, fake, a["m"], a["n"], a["k"], a["r"], corr, corr, corr, 2, fake, fake, None, 0, sc, sc,
                          fake, a["out_mode"], a["flags"], None, None)
    assert st == -1
    assert msg in L.uwc_last_error().decode()


def test_other_entry_points_reject_bad_arguments():
    from uwc_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(1 << 20)
    assert L.uwc_b3_root_and_seed(fake, 1000, fake, None, None, 0, None, None, fake, 100, None) == -1
    assert "multiple of 1024" in L.uwc_last_error().decode()
    assert L.uwc_noise_perm(fake, 64, 96, fake, fake, None) == -1
    assert L.uwc_noise_rows(fake, 12, 64, 64, None, None, None, None, None, -1, -1, None, 0, None) == -1
    # requested limbs or E copy without a corr buffer to write them into
    assert L.uwc_noise_rows(fake, 16, 64, 64, None, None, None, fake, None, 0, -1, None, 3, None) == -1
    assert "need corr" in L.uwc_last_error().decode()
    assert L.uwc_noise_rows(fake, 16, 64, 64, fake, fake, fake, None, None, -1, 0, None, 3, None) == -1
    assert "need corr" in L.uwc_last_error().decode()
    assert L.uwc_quant_act_f32(fake, 4, 96, 64, 64, fake, fake, None) == -1
    assert "power of two" in L.uwc_last_error().decode()
    assert L.uwc_quant_act_f32(fake, 4, 64, 0, 200, fake, fake, None) == -1
    assert L.uwc_quant_rows_had(fake, 4, 100, 0, fake, fake, None) == -1
    assert "multiple of 8" in L.uwc_last_error().decode()
    assert L.uwc_quant_rows_had(fake, 4, 96, 64, fake, fake, None) == -1
    # the fused GEMM + residual: the output may not overlap the residual
    assert L.uwc_igemm_dequant_residual_f32(fake, fake, 256, 256, 128, fake, fake, fake, fake, None) == -1
    assert "overlaps" in L.uwc_last_error().decode()
    assert L.uwc_igemm_dequant_residual_f32(fake, fake, 256, 256, 128, fake, fake, None, fake, None) == -1
    assert "null" in L.uwc_last_error().decode()
    # the stored-exp attention: a scratch one byte short of the exponentials and the row maxima
    # is refused before any launch; so is a missing one
    need = L.uwc_attention_scratch_bytes(1, 300, 4)
    inv = ctypes.c_float(0.125)
    assert L.uwc_attention_ws(fake, fake, fake, fake, fake, fake, 1, 300, 4, 2, 64, inv, fake, fake, need - 1,
                              None) == -1
    assert "escratch holds" in L.uwc_last_error().decode()
    assert L.uwc_attention_ws(fake, fake, fake, fake, fake, fake, 1, 300, 4, 2, 64, inv, fake, None, need, None) == -1
    assert "null escratch" in L.uwc_last_error().decode()
    assert L.uwc_attention(fake, fake, fake, fake, fake, fake, 1, 300, 4, 3, 64, inv, fake, None) == -1
    assert "H % Hkv" in L.uwc_last_error().decode() or "Hkv" in L.uwc_last_error().decode()
    # qkv_post loads and stores whole vectors: a base off a 16-byte boundary is refused
    odd = ctypes.c_void_p((1 << 20) + 4)
    eps = ctypes.c_float(1e-6)
    assert L.uwc_qkv_post(odd, fake, fake, fake, fake, fake, fake, 1, 64, 4, 2, 128, eps, 1, fake, fake, fake, fake,
                          fake, fake, None, None) == -1
    assert "16-byte aligned" in L.uwc_last_error().decode()
    assert L.uwc_qkv_post(fake, fake, fake, fake, fake, fake, odd, 1, 64, 4, 2, 128, eps, 1, fake, fake, fake, fake,
                          fake, fake, None, None) == -1
    assert "16-byte aligned" in L.uwc_last_error().decode()


def test_python_surface_matches_reference_names():
    """The reference's ops.py / detrt names a caller imports are all here."""
    from uwc_amd import detrt, ops
    for name in ("BM", "BN", "BK", "limbs_for", "WIN_WORDS", "CHUNKS_PER_CTA", "FLAG_HASH", "FLAG_DENOISE", "OUT_NONE",
                 "OUT_I32", "OUT_BF16", "CONFIGS", "DEFAULT_CFG", "words", "words_to_bytes", "LABEL_A", "LABEL_B",
                 "SALT_A", "SALT_B", "consts", "b3_root_and_seed", "noise_uniform", "noise_perm", "noise_rows", "gemm",
                 "proj_matrix", "project", "nonce_noise", "noise_project",
                 "MinedWeight", "GraphedForward", "quant_rows_had"):
        assert hasattr(ops, name), name
    for name in ("quant_act", "DetLinear"):
        assert hasattr(detrt, name), name
    from uwc_amd import model
    for name in ("QMAX", "hadamard", "rotate", "quant_rows", "MinedLinear", "convert_qwen3"):
        assert hasattr(model, name), name


def test_salt_constants_match_oracle():
    import oracle as O
    from uwc_amd import ops
    assert ops.SEED_SALT_A == O.SEED_SALT_A and ops.SEED_SALT_B == O.SEED_SALT_B
    assert ops.SEED_LABEL_A == O.SEED_LABEL_A and ops.SEED_LABEL_B == O.SEED_LABEL_B


def test_product_does_not_import_oracle():
    """The product path never routes through the CPU oracle."""
    pkg = os.path.join(ROOT, "useful-work-coin_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                src = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in re.sub(r"#.*|//.*", "", src).lower(), f


def test_host_limb_rule_and_bound_words_match_oracle():
    """The host-side limb rule and difficulty-bound packing the bench uses agree with the oracle's
    (kernels.cu:602-607, pearl_glue.py:65-66), at every limb boundary."""
    import oracle as O
    from uwc_amd import ops
    for mx in (0, 63, 64, 8127, 8128, 1040319, 1040320, 1 << 30):
        assert ops.limbs_for_max(mx) == O.limbs_needed(mx), mx
    for m, n, w in ((4096, 4096, 12), (256, 512, 20), (128, 128, 1)):
        want = O.bound_for_wins(m, n, w)
        got = ops.bound_words(((1 << 256) - 1) * w // ((m // 8) * (n // 16)))
        assert got.dtype == want.dtype and (got == want).all()


def test_loader_refuses_library_of_another_header(tmp_path, monkeypatch):
    """A header that differs from the one the library was built from (one changed byte) makes
    the loader raise instead of binding the library."""
    from uwc_amd import _lib
    other = tmp_path / "uwc.h"
    other.write_bytes(open(HEADER, "rb").read() + b"\n")
    monkeypatch.setattr(_lib, "HEADER_PATH", str(other))
    monkeypatch.setattr(_lib, "_LIB", None)
    with pytest.raises(ImportError, match="another include/uwc.h"):
        _lib.lib()
