"""Extract golden vectors for the detrt linear path from the reference's Go-referee fixtures.

The reference ships cross-language fixtures (gzip JSON written by its
runtime/bench/export_fixtures.py:30-51) as git binary hunks inside
chain/patches/0003-*.patch (tiny.json.gz, qwen3_1p7b.json.gz) and 0021-*.patch
(llama_tiny.json.gz). They are data: this script applies only those hunks into a temporary
git tree, decodes the rows and keeps what the int8 linear path needs. It imports no
reference code. Run it in the build container (it reads /root/reference); the GPU box only
reads the .npz files it writes.

Each stage trace is a fixed list of leaves (runtime/detrt/stage.py:93-110); a row is the
leaf's output as little-endian u32 words (float32 bits, or int32 values). Kept per
(stage, layer):
  N1, O (per-head rows concatenated), N2, SM     fp32 inputs of the four quant_act calls
  QA1..QA4                                       their int8 q and fp32 scale (last word)
  QKV, OP, GU, DN                                 fp32 outputs of the four linears
  W_<name>_rows / _q / _s                         int8 weight rows and fp32 scales
For the real Qwen3-1.7B fixture only the 24 committed weight rows per linear exist, so the
linear outputs are kept at those columns only.

    python tests/golden/make_fixtures.py [/root/reference]
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

# leaf op codes in program order (runtime/detrt/stage.py:26-27)
OPS = ["EMBED", "N1", "QA1", "QKV", "QN", "KN", "QR", "KR", "KQ", "VQ", "QQ", "VT", "VS", "S", "P", "O",
       "QA2", "OP", "R1", "N2", "QA3", "GU", "SM", "QA4", "DN", "R2"]


def program(H: int, Hkv: int, hd: int, T: int, l0: int, l1: int) -> list[tuple]:
    """Leaf list (op, layer, t, h) of a stage, in the order runtime/detrt/stage.py:89-110 fixes."""
    out = []
    if l0 == 0:
        out += [("EMBED", 0, t, -1) for t in range(T)]
    for l in range(l0, l1):
        per_t = lambda op: [(op, l, t, -1) for t in range(T)]
        per_th = lambda op, nh: [(op, l, t, h) for t in range(T) for h in range(nh)]
        out += per_t("N1") + per_t("QA1") + per_t("QKV")
        out += per_th("QN", H) + per_th("KN", Hkv) + per_th("QR", H) + per_th("KR", Hkv)
        out += per_th("KQ", Hkv) + per_th("VQ", Hkv) + per_th("QQ", H)
        out += [("VT", l, d, h) for h in range(Hkv) for d in range(hd)]
        out += [("VS", l, -1, h) for h in range(Hkv)]
        out += per_th("S", H) + per_th("P", H) + per_th("O", H)
        for op in ("QA2", "OP", "R1", "N2", "QA3", "GU", "SM", "QA4", "DN", "R2"):
            out += per_t(op)
    return out


def words(s: str) -> np.ndarray:
    return np.frombuffer(base64.b64decode(s), dtype="<u4").astype(np.uint32)


def extract(path: str, stages: list[int], name: str, max_t: int | None = None) -> dict:
    d = json.load(gzip.open(path))
    cfg = d["cfg"]
    H, Hkv, hd, D, I, Bs = cfg["H"], cfg["Hkv"], cfg["Hd"], cfg["D"], cfg["I"], cfg["Bs"]
    out = {"cfg": np.array([D, H, Hkv, hd, I, Bs, cfg.get("Arch", 0)], np.int64)}
    W: dict = {}
    for w in d["weights"]:
        if w["name"] in ("qkv", "o", "gu", "down"):
            W.setdefault((w["name"], w["layer"]), []).append((w["row"], words(w["w"])))
    for si in stages:
        st = d["stages"][si]
        T, l0, l1 = st["T"], st["L0"], st["L1"]
        leaves = program(H, Hkv, hd, T, l0, l1)
        assert len(leaves) == len(st["rows"]), (len(leaves), len(st["rows"]))
        rows = {lf: words(r) for lf, r in zip(leaves, st["rows"])}
        TT = T if max_t is None else min(T, max_t)
        f32 = lambda op, l: np.stack([rows[(op, l, t, -1)].view(np.float32) for t in range(TT)])
        for l in range(l0, l1):
            p = f"l{l}_"
            qa = {}
            for qn in ("QA1", "QA2", "QA3", "QA4"):
                r = np.stack([rows[(qn, l, t, -1)] for t in range(TT)])
                q = r[:, :-1].view(np.int32)
                assert np.abs(q).max() <= 64
                qa[qn] = (q.astype(np.int8), r[:, -1].view(np.float32).copy())
                out[p + qn + "_q"], out[p + qn + "_s"] = qa[qn]
            out[p + "N1"] = f32("N1", l)
            out[p + "O"] = np.stack([np.concatenate([rows[("O", l, t, h)].view(np.float32) for h in range(H)])
                                     for t in range(TT)])
            out[p + "N2"] = f32("N2", l)
            out[p + "SM"] = f32("SM", l)
            for lin, op in (("qkv", "QKV"), ("o", "OP"), ("gu", "GU"), ("down", "DN")):
                wr = sorted(W[(lin, l)], key=lambda x: x[0])
                idx = np.array([r for r, _ in wr], np.int64)
                mat = np.stack([w for _, w in wr])
                out[p + f"W_{lin}_rows"] = idx
                out[p + f"W_{lin}_q"] = mat[:, :-1].view(np.int32).astype(np.int8)
                out[p + f"W_{lin}_s"] = mat[:, -1].view(np.float32).copy()
                out[p + op] = f32(op, l)[:, idx]
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
        jobs = [("tiny.json.gz", [0, 1], "detrt_tiny_qwen3", None),
                ("llama_tiny.json.gz", [0, 1], "detrt_tiny_llama", None),
                ("qwen3_1p7b.json.gz", [0, 1], "detrt_qwen3_1p7b", None)]
        for fn, stages, name, mt in jobs:
            arrs = extract(os.path.join(td, fn), stages, name, mt)
            np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrs)


if __name__ == "__main__":
    main()
