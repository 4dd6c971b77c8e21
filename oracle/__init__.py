"""CPU oracle for the int8 GEMM hot path (NoisyGEMM mining + detrt linear).

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this package, and only as the checker: the product path
(useful-work-coin_amd/uwc_amd) never imports it and fails loudly without its HIP library.

The arithmetic lives in oracle/uwc_oracle.c (built by oracle/build.sh into liboracle.so);
this module composes it into the reference's algorithms, each citing the reference
file:line it restates (paths relative to the reference repository root). What pins each
function is listed in the C file's header and exercised by tests/test_oracle.py.

Parity status. BLAKE3 itself is pinned by the BLAKE3 team's published test vectors
(tests/golden/blake3_official_vectors.json: unkeyed inputs of 0 to 102400 bytes, keyed inputs of 0,
1, 1024 and 2048 bytes) and by two independent restatements (C recursive tree, Python streaming
stack) that agree on every tree shape up to 129 chunks. Those vectors pin the hash function only,
not the messages this path feeds it. The reference stores no vectors of its BLAKE3-derived values
(its only check compares against the `blake3` package live, miner/ampere/tests/test_kernels.py:13-20,
and that package is not installed here), so these rest on restatement alone and are
PARITY UNPINNED:
  * the random_hash message layout behind E and P (reference.py:67-93, kernels.cu:246-301; the
    value rules derived from it are checked by distribution: E uniform on [-32, 31], P's first index
    uniform and its XOR distance uniform on [1, r - 1]);
  * the salted seed chain a_seed / b_seed (reference.py:41-64: root binding, salts, labels);
  * the tile-message encoding fed to the tile digest (reference.py:124-125, kernels.cu:574-596; the
    fold itself is checked by brute force).
Pearl's job_key serialization and penalised bound (pearl_glue.py:44-62) are not restated: callers
pass job_key and target words, as the kernels do.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

u8p = ctypes.POINTER(ctypes.c_uint8)
i8p = ctypes.POINTER(ctypes.c_int8)
u16p = ctypes.POINTER(ctypes.c_uint16)
u32p = ctypes.POINTER(ctypes.c_uint32)
i32p = ctypes.POINTER(ctypes.c_int32)
f32p = ctypes.POINTER(ctypes.c_float)
I64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is missing: run oracle/build.sh (or __graft_entry__.build())")
        L = ctypes.CDLL(path)
        sig = {
            "or_b3_compress": [u32p, u32p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32, u32p],
            "or_b3_hash": [u8p, ctypes.c_uint64, u32p, u32p],
            "or_noise_uniform": [i8p, ctypes.c_uint32, u32p, u32p],
            "or_noise_perm": [u32p, ctypes.c_uint32, ctypes.c_uint32, u32p, u32p],
            "or_noise_apply": [i8p, I64, I64, I64, i8p, u32p, i8p],
            "or_project": [i8p, I64, I64, I64, u32p, i32p],
            "or_limbs": [i32p, I64, I64, ctypes.c_int, i8p, I64],
            "or_igemm_i32": [i8p, i8p, I64, I64, I64, i32p],
            "or_transcript": [i8p, i8p, I64, I64, I64, I64, u32p],
            "or_tile_hashes": [u32p, I64, u32p, u32p],
            "or_hash_le": [u32p, u32p],
            "or_quant_act_f32": [f32p, I64, I64, ctypes.c_int, ctypes.c_int, i8p, f32p],
            "or_dequant_f32": [i32p, f32p, f32p, I64, I64, f32p],
            "or_scale_bf16": [i32p, f32p, f32p, I64, I64, u16p],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int if name == "or_hash_le" else None
        _LIB = L
    return _LIB


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


# ------------------------------------------------------------------ words / bytes
def words(b: bytes) -> np.ndarray:
    return np.frombuffer(b, dtype="<u4").astype(np.uint32)


def to_bytes(w: np.ndarray) -> bytes:
    return np.ascontiguousarray(w, dtype=np.uint32).astype("<u4").tobytes()


# ------------------------------------------------------------------ BLAKE3
def b3(data: bytes, key: bytes | None = None) -> bytes:
    """BLAKE3 digest (keyed if key is given). C restatement of the spec."""
    buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    buf = np.ascontiguousarray(buf)
    out = np.zeros(8, np.uint32)
    kw = None if key is None else np.ascontiguousarray(words(key))
    lib().or_b3_hash(_p(buf, u8p), len(data), None if kw is None else _p(kw, u32p), _p(out, u32p))
    return to_bytes(out)


def b3_compress(cv, msg, counter: int, blen: int, flags: int) -> np.ndarray:
    cv = np.ascontiguousarray(cv, np.uint32)
    msg = np.ascontiguousarray(msg, np.uint32)
    out = np.zeros(16, np.uint32)
    lib().or_b3_compress(_p(cv, u32p), _p(msg, u32p), counter, blen, flags, _p(out, u32p))
    return out


# ------------------------------------------------------------------ cuPOW constants
# miner/ampere/uwc_ampere/reference.py:19-30
JACKPOT_SIZE = 16
LROT_PER_TILE = 13
CHUNK_LEN = 1024
SEED_LABEL_A = b"A_tensor" + b"\x00" * 24
SEED_LABEL_B = b"B_tensor" + b"\x00" * 24
SEED_SALT_A = b3(b"pearl/cert-v3/noise-seed/A") if os.path.exists(os.path.join(_HERE, "liboracle.so")) else None
SEED_SALT_B = b3(b"pearl/cert-v3/noise-seed/B") if SEED_SALT_A is not None else None
WIN_WORDS = 10


def limbs_for(k: int) -> int:
    """Balanced base-128 limbs that cover |projection| <= 127 k (ops.py:18-24)."""
    bound, L, cap = 127 * k, 1, 63
    while cap < bound:
        L += 1
        cap = cap * 128 + 63
    return L


def limbs_needed(mx: int) -> int:
    """Limbs the denoise pass uses for a runtime max |projection| (kernels.cu:602-607)."""
    return 1 if mx <= 63 else 2 if mx <= 8127 else 3 if mx <= 1040319 else 4


def denoise(noisy: np.ndarray, corrA: np.ndarray, corrB: np.ndarray, maxabs, lmax: int | None = None) -> np.ndarray:
    """The exact denoise of kernels.cu:598-673: L from the runtime max |projection| (:602-607,
    capped at lmax = the correction buffers' limb count), then
    noisy - sum_{li < L} 128^li corrA[li] @ corrB[li]^T, Horner over the limbs from L - 1 down, all
    mod 2^32. noisy is the int32 (or wider) noisy product; corrA (lmax, m, 2r), corrB (lmax, n, 2r)
    int8."""
    lmax = corrA.shape[0] if lmax is None else lmax
    L = min(limbs_needed(max(int(maxabs[0]), int(maxabs[1]))), lmax)
    tmp = np.zeros(noisy.shape, np.int64)
    for li in range(L - 1, -1, -1):
        # |corrA corrB^T| <= 64 * 64 * 2r: exact in float64 for any r here
        part = corrA[li].astype(np.float64) @ corrB[li].astype(np.float64).T
        tmp = (tmp << 7) + part.astype(np.int64)
    return ((noisy.astype(np.int64) - tmp) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)


def pad_to_chunk(data: bytes) -> bytes:
    return data + b"\x00" * (-len(data) % CHUNK_LEN)


def bind_root(root: bytes, dim: int, salt: bytes) -> bytes:
    """reference.py:46-47."""
    return b3(root + dim.to_bytes(4, "little") + b"\x00" * 28, salt)


def commitment(job_key: bytes, A: np.ndarray, Bt: np.ndarray):
    """(a_seed, b_seed, root_A, root_B), salted v3 derivation (reference.py:50-64)."""
    m, n = A.shape[0], Bt.shape[0]
    ha = b3(pad_to_chunk(np.ascontiguousarray(A, np.int8).tobytes()), job_key)
    hb = b3(pad_to_chunk(np.ascontiguousarray(Bt, np.int8).tobytes()), job_key)
    b_seed = b3(job_key + bind_root(hb, n, SEED_SALT_B))
    a_seed = b3(b_seed + bind_root(ha, m, SEED_SALT_A))
    return a_seed, b_seed, ha, hb


def uniform_matrix(label: bytes, key: bytes, rows: int, r: int) -> np.ndarray:
    """rows x r int8 in [-32, 31] (reference.py:74-79)."""
    assert (rows * r) % 32 == 0
    out = np.empty((rows, r), np.int8)
    lib().or_noise_uniform(_p(out, i8p), rows * r // 32, _p(words(label), u32p), _p(words(key), u32p))
    return out


def perm_packed(label: bytes, key: bytes, k: int, r: int) -> np.ndarray:
    """k u32, first | second << 16 (reference.py:82-93, kernels.cu:284-301)."""
    out = np.empty(k, np.uint32)
    lib().or_noise_perm(_p(out, u32p), k, r, _p(words(label), u32p), _p(words(key), u32p))
    return out


def noise_apply(src: np.ndarray, E: np.ndarray, P: np.ndarray) -> np.ndarray:
    rows, k = src.shape
    r = E.shape[1]
    dst = np.empty_like(src, dtype=np.int8)
    lib().or_noise_apply(_p(np.ascontiguousarray(src, np.int8), i8p), rows, k, r, _p(np.ascontiguousarray(E), i8p),
                         _p(np.ascontiguousarray(P, np.uint32), u32p), _p(dst, i8p))
    return dst


def project(src: np.ndarray, P: np.ndarray, r: int) -> np.ndarray:
    rows, k = src.shape
    out = np.empty((rows, r), np.int32)
    lib().or_project(_p(np.ascontiguousarray(src, np.int8), i8p), rows, k, r, _p(np.ascontiguousarray(P, np.uint32), u32p),
                     _p(out, i32p))
    return out


def write_limbs(proj: np.ndarray, corr: np.ndarray, corr_off: int):
    rows, r = proj.shape
    lib().or_limbs(_p(np.ascontiguousarray(proj, np.int32), i32p), rows, r, corr.shape[0], _p(corr, i8p), corr_off)


def igemm(A: np.ndarray, B: np.ndarray) -> np.ndarray:
    """Exact A @ B^T (int8 -> int32, mod 2^32)."""
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    m, k = A.shape
    n = B.shape[0]
    C = np.empty((m, n), np.int32)
    lib().or_igemm_i32(_p(A, i8p), _p(B, i8p), m, n, k, _p(C, i32p))
    return C


def transcript(Ap: np.ndarray, Bp: np.ndarray, r: int) -> np.ndarray:
    """Per-tile jackpot messages [m/64, 8, n/64, 4, 16] u32 (reference.py:111-121, 138-165)."""
    Ap = np.ascontiguousarray(Ap, np.int8)
    Bp = np.ascontiguousarray(Bp, np.int8)
    m, k = Ap.shape
    n = Bp.shape[0]
    assert m % 64 == 0 and n % 64 == 0 and k % r == 0 and r % 64 == 0
    out = np.empty((m // 64, 8, n // 64, 4, 16), np.uint32)
    lib().or_transcript(_p(Ap, i8p), _p(Bp, i8p), m, n, k, r, _p(out, u32p))
    return out


def tile_hashes(msgs: np.ndarray, key: bytes) -> np.ndarray:
    msgs = np.ascontiguousarray(msgs, np.uint32)
    nt = msgs.size // 16
    out = np.empty(msgs.shape[:-1] + (8,), np.uint32)
    lib().or_tile_hashes(_p(msgs, u32p), nt, _p(words(key), u32p), _p(out, u32p))
    return out


def hash_le(h: np.ndarray, target: np.ndarray) -> bool:
    return bool(lib().or_hash_le(_p(np.ascontiguousarray(h, np.uint32), u32p),
                                 _p(np.ascontiguousarray(target, np.uint32), u32p)))


def winners(digests: np.ndarray, target: np.ndarray) -> set:
    """{(row_off, col_off, hash)} of tiles whose digest <= target (kernels.cu:579-595)."""
    tv = sum(int(w) << (32 * i) for i, w in enumerate(target))
    # little-endian U256 compare, vectorised over tiles: most significant word first
    d = digests.reshape(-1, 8)
    le = np.ones(d.shape[0], bool)
    decided = np.zeros(d.shape[0], bool)
    for i in range(7, -1, -1):
        t = np.uint32(target[i])
        ne = (d[:, i] != t) & ~decided
        le[ne] = d[ne, i] < t
        decided |= ne
    out = set()
    MB, _, NB, _, _ = digests.shape
    for idx in np.nonzero(le)[0]:
        rb, g, cb, t = np.unravel_index(idx, (MB, 8, NB, 4))
        h = to_bytes(d[idx])
        assert int.from_bytes(h, "little") <= tv
        out.add((int(rb * 64 + g), int(cb * 64 + 2 * t), h))
    return out


def bound_for_wins(m: int, n: int, wins: float = 12.0) -> np.ndarray:
    """Target words giving about `wins` winning 8 x 16 tiles (miner/ampere/tests/test_proj_gemm.py:194-197)."""
    b = ((1 << 256) - 1) * int(wins) // ((m // 8) * (n // 16))
    return np.array([(b >> (32 * i)) & 0xFFFFFFFF for i in range(8)], dtype=np.uint32)


def block_side(job_key: bytes, Bt: np.ndarray, r: int) -> dict:
    """MinedWeight.setup_block on the CPU (ops.py:237-256): b_seed, EBRt, PB, BpEBt, corrB (E copy)."""
    n, k = Bt.shape
    hb = b3(pad_to_chunk(np.ascontiguousarray(Bt, np.int8).tobytes()), job_key)
    b_seed = b3(job_key + bind_root(hb, n, SEED_SALT_B))
    EBRt = uniform_matrix(SEED_LABEL_B, b_seed, n, r)
    PB = perm_packed(SEED_LABEL_B, b_seed, k, r)
    BpEBt = noise_apply(Bt, EBRt, PB)
    return dict(b_seed=b_seed, root_B=hb, EBRt=EBRt, PB=PB, BpEBt=BpEBt)


def mined_forward(A: np.ndarray, Bt: np.ndarray, job_key: bytes, target: np.ndarray, r: int,
                  hash_tiles: bool = True, blk: dict | None = None) -> dict:
    """MinedWeight._forward restated (ops.py:316-347): commit A, noise both sides, the hashed
    noisy GEMM's winners, the exact denoise. Returns every intermediate."""
    m, k = A.shape
    n = Bt.shape[0]
    blk = blk or block_side(job_key, Bt, r)
    ha = b3(pad_to_chunk(np.ascontiguousarray(A, np.int8).tobytes()), job_key)
    a_seed = b3(blk["b_seed"] + bind_root(ha, m, SEED_SALT_A))
    EAL = uniform_matrix(SEED_LABEL_A, a_seed, m, r)
    PA = perm_packed(SEED_LABEL_A, a_seed, k, r)
    ApEA = noise_apply(A, EAL, PA)
    lmax = limbs_for(k)
    X = project(A, blk["PB"], r)
    Y = project(blk["BpEBt"], PA, r)
    corrA = np.zeros((lmax, m, 2 * r), np.int8)
    corrB = np.zeros((lmax, n, 2 * r), np.int8)
    write_limbs(X, corrA, 0)
    write_limbs(Y, corrB, r)
    for li in range(lmax):
        corrA[li, :, r:] = EAL
        corrB[li, :, :r] = blk["EBRt"]
    res = dict(a_seed=a_seed, root_A=ha, EAL=EAL, PA=PA, ApEA=ApEA, X=X, Y=Y, corrA=corrA, corrB=corrB,
               maxabs=np.array([np.abs(X).max(), np.abs(Y).max()], np.int32), **blk)
    # noisy product minus the exact low-rank correction = A @ Bt^T
    noisy = igemm(ApEA, blk["BpEBt"]).astype(np.int64)
    corr = X.astype(np.int64) @ blk["EBRt"].astype(np.int64).T + EAL.astype(np.int64) @ Y.astype(np.int64).T
    res["out"] = ((noisy - corr) & 0xFFFFFFFF).astype(np.uint32).view(np.int32)
    if hash_tiles:
        msgs = transcript(ApEA, blk["BpEBt"], r)
        dig = tile_hashes(msgs, a_seed)
        res.update(msgs=msgs, digests=dig, winners=winners(dig, target))
    return res


# ------------------------------------------------------------------ detrt linear
def quant_act(x: np.ndarray, bs: int, qmax: int = 64):
    """runtime/detrt/core.py:188-195 (fwht + quant_sym + 1/sqrt(bs) fold). -> (int8 q, f32 scale)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    assert bs <= 1 or k % bs == 0
    q = np.empty((rows, k), np.int8)
    s = np.empty(rows, np.float32)
    lib().or_quant_act_f32(_p(x, f32p), rows, k, bs, qmax, _p(q, i8p), _p(s, f32p))
    return q, s


def hadamard_bs(hadamard_block: int, k: int) -> int:
    """DetLinear's block size min(Bs, k & -k) (runtime/detrt/qwen3.py:76)."""
    return min(hadamard_block, k & -k) if hadamard_block else 0


def quant_weight(W: np.ndarray, hadamard_block: int):
    """DetLinear.__init__ (qwen3.py:72-86): Wq = quant_sym(fwht(W, bs), 64), sw folded by 1/sqrt(bs).
    That is quant_act applied to each weight row."""
    bs = hadamard_bs(hadamard_block, W.shape[1])
    Wq, sw = quant_act(W, bs)
    return Wq, sw, bs


def dequant(acc: np.ndarray, sx: np.ndarray, sw: np.ndarray) -> np.ndarray:
    """fmul(fmul(f32(acc), s_x), s_w) (qwen3.py:125)."""
    acc = np.ascontiguousarray(acc, np.int32)
    m, n = acc.shape
    y = np.empty((m, n), np.float32)
    lib().or_dequant_f32(_p(acc, i32p), _p(np.ascontiguousarray(sx, np.float32), f32p),
                         _p(np.ascontiguousarray(sw, np.float32), f32p), m, n, _p(y, f32p))
    return y


def scale_bf16(acc: np.ndarray, a_scale: np.ndarray, b_scale: np.ndarray) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.int32)
    m, n = acc.shape
    out = np.empty((m, n), np.uint16)
    lib().or_scale_bf16(_p(acc, i32p), _p(np.ascontiguousarray(a_scale, np.float32), f32p),
                        _p(np.ascontiguousarray(b_scale, np.float32), f32p), m, n, _p(out, u16p))
    return out


def det_linear(x: np.ndarray, Wq: np.ndarray, sw: np.ndarray, bs: int):
    """DetLinear.__call__ (qwen3.py:121-126): quant_act -> exact int GEMM -> dequant."""
    q, sx = quant_act(x, bs)
    acc = igemm(q, Wq)
    return q, sx, acc, dequant(acc, sx, sw)
