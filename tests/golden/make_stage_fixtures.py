"""Extract whole-stage golden vectors (every leaf row, the weights and the Merkle roots) from the
reference's Go-referee fixtures, for the decoder-layer ops and the stage commitments.

The reference ships cross-language fixtures (gzip JSON written by its
runtime/bench/export_fixtures.py:30-51) as git binary hunks inside chain/patches/0003-*.patch
(tiny.json.gz, qwen3_1p7b.json.gz) and 0021-*.patch (llama_tiny.json.gz). They are data: this
script applies only those hunks into a temporary git tree and decodes them; it imports no
reference code. Run it in the build container (it reads /root/reference); tests only read the
.npz files it writes.

Written per fixture (tests/golden/stage_<name>.npz):
  cfg            [D, H, Hkv, hd, I, L, V, eps_bits, Bs, MaxPos, Arch]
  w_<name>[_l]   weight rows: embed, in_norm/post_norm/q_norm/k_norm per layer, rope_cos/rope_sin
                 (fp32); linears qkv/o/gu/down per layer as int8 q and fp32 scale
                 (w_<lin>_<l>_q, w_<lin>_<l>_s, w_<lin>_<l>_rows: which rows are present)
  s<i>_meta      [T, L0, L1] of stage i; s<i>_tokens (T,) or s<i>_input (T, D) fp32
  s<i>_root      the stage trace root (32 bytes) committed by the referee
  s<i>_words     all leaf rows of the stage, concatenated as u32 words, in program order
  s<i>_offs      word offset of each leaf row (len = leaves + 1)
Stages whose rows equal a concatenation of others (the tiny [0, 2) stage) keep only their
meta, tokens and root.

    python tests/golden/make_stage_fixtures.py [/root/reference]
"""
from __future__ import annotations

import base64
import glob
import gzip
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def words(s: str) -> np.ndarray:
    return np.frombuffer(base64.b64decode(s), dtype="<u4").astype(np.uint32)


def extract(path: str, name: str, rows_for: list[int]) -> dict:
    d = json.load(gzip.open(path))
    cfg = d["cfg"]
    out = {"cfg": np.array([cfg["D"], cfg["H"], cfg["Hkv"], cfg["Hd"], cfg["I"], cfg["L"], cfg["V"], cfg["EpsBits"],
                            cfg["Bs"], cfg["MaxPos"], cfg.get("Arch", 0)], np.int64)}
    groups: dict = {}
    for w in d["weights"]:
        groups.setdefault((w["name"], w["layer"]), []).append((w["row"], words(w["w"])))
    for (nm, layer), rows in groups.items():
        rows.sort(key=lambda x: x[0])
        idx = np.array([r for r, _ in rows], np.int64)
        mat = np.stack([w for _, w in rows])
        key = nm.replace(".", "_")
        if nm in ("qkv", "o", "gu", "down"):
            p = f"w_{key}_{layer}"
            out[p + "_rows"] = idx
            out[p + "_q"] = mat[:, :-1].view(np.int32).astype(np.int8)
            out[p + "_s"] = mat[:, -1].view(np.float32).copy()
        elif nm in ("in_norm", "post_norm", "q_norm", "k_norm"):
            out[f"w_{key}_{layer}"] = mat.view(np.float32)[0]
        else:  # embed, rope.cos, rope.sin: row-indexed fp32 tables
            out[f"w_{key}_rows"] = idx
            out[f"w_{key}"] = mat.view(np.float32)
    for si, st in enumerate(d["stages"]):
        out[f"s{si}_meta"] = np.array([st["T"], st["L0"], st["L1"]], np.int64)
        out[f"s{si}_root"] = np.frombuffer(bytes.fromhex(st["root"]), np.uint8)
        if st.get("tokens") is not None:
            out[f"s{si}_tokens"] = np.array(st["tokens"], np.int64)
        if st.get("input") is not None:
            out[f"s{si}_input"] = np.stack([words(r).view(np.float32) for r in st["input"]])
        if si in rows_for:
            rws = [words(r) for r in st["rows"]]
            out[f"s{si}_offs"] = np.cumsum([0] + [len(r) for r in rws]).astype(np.int64)
            out[f"s{si}_words"] = np.concatenate(rws)
    print(f"{name}: {len(out)} arrays, {sum(v.nbytes for v in out.values()) / 1e6:.2f} MB")
    return out


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    with tempfile.TemporaryDirectory() as tmp:
        subprocess.run(["git", "init", "-q"], cwd=tmp, check=True)
        for pat in ("0003-*.patch", "0021-*.patch"):
            patch = glob.glob(os.path.join(ref, "chain", "patches", pat))[0]
            subprocess.run(["git", "apply", "--include=node/jobstate/testdata/*", patch], cwd=tmp, check=True)
        td = os.path.join(tmp, "node", "jobstate", "testdata")
        for fn, name, rows_for in (("tiny.json.gz", "stage_tiny_qwen3", [0, 1]),
                                   ("llama_tiny.json.gz", "stage_tiny_llama", [0, 1]),
                                   ("qwen3_1p7b.json.gz", "stage_qwen3_1p7b", [0, 1])):
            arrs = extract(os.path.join(td, fn), name, rows_for)
            np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)


if __name__ == "__main__":
    main()
