"""Write tests/golden/dsv2_ref.npz (2 MoE layers) and dsv2_ref_dense.npz (a
dense first layer, then 2 MoE layers): the greedy trajectory and top-2
logits of the compiled reference DSV2 decode step (bench/dsv2_decode_bench.c, CPU
backend, built by oracle/Makefile into oracle/_ref/dsv2_bench) on a seeded
synthetic model small enough for the CPU.  The model is regenerated from the
seed by tests/_dsv2_weights.py (only ids, logits and a weight checksum are
stored) and handed to the reference as a DSV2PK01 weight pack.

Run in the build container (the reference tree is not on the GPU box):
    python tests/golden/make_dsv2_golden.py
"""
import hashlib
import os
import re
import subprocess
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "tests"))
import _dsv2_weights as W  # noqa: E402

CFG = dict(n_layers=2, dim=128, n_heads=8, kv_lora=64, d_nope=32, d_rope=16, d_v=32, n_experts=8,
           n_shared=2, top_k=3, moe_inter=64, ffn=256, first_dense=0, vocab=1024, max_seq=64,
           batch=1, eps=1e-6, init_std=0.02)
# the second fixture pins the dense first layer (its SwiGLU runs as bf16 uops
# in the reference: bench/dsv2_decode_bench.c:2042-2049, :2370-2378)
FIXTURES = {"dsv2_ref.npz": CFG, "dsv2_ref_dense.npz": dict(CFG, n_layers=3, first_dense=1)}
SEED = 20261201
PROMPT = [5, 17, 300, 911, 42, 7, 640, 128]
COUNT = 12


def weight_digest(t) -> str:
    h = hashlib.sha256()
    for k in sorted(t):
        if k.endswith(("ckv", "kpe")):
            continue
        h.update(k.encode())
        h.update(np.ascontiguousarray(t[k]).tobytes())
    return h.hexdigest()


def main():
    exe = ROOT / "oracle" / "_ref" / "dsv2_bench"
    if not exe.exists():
        subprocess.run(["make", "-C", str(ROOT / "oracle"), "_ref/dsv2_bench"], check=True)
    for name, cfg in FIXTURES.items():
        write_fixture(exe, name, cfg)


def write_fixture(exe, name, CFG):
    t = W.make_dsv2(CFG, SEED)
    with tempfile.TemporaryDirectory() as d:
        pack = os.path.join(d, "dsv2.pack")
        W.write_pack(t, CFG, pack)
        env = dict(os.environ, DEV="cpu", DSV2_WEIGHTS=pack, DSV2_PROMPT_IDS=",".join(map(str, PROMPT)),
                   DSV2_COUNT=str(COUNT), DSV2_TOP2="1", DSV2_DIM=str(CFG["dim"]),
                   DSV2_LAYERS=str(CFG["n_layers"]), DSV2_HEADS=str(CFG["n_heads"]),
                   DSV2_KVLORA=str(CFG["kv_lora"]), DSV2_DNOPE=str(CFG["d_nope"]),
                   DSV2_DROPE=str(CFG["d_rope"]), DSV2_DV=str(CFG["d_v"]),
                   DSV2_EXPERTS=str(CFG["n_experts"]), DSV2_NSHARED=str(CFG["n_shared"]),
                   DSV2_TOPK=str(CFG["top_k"]), DSV2_MOEINTER=str(CFG["moe_inter"]),
                   DSV2_DENSEINTER=str(CFG["ffn"]), DSV2_FIRSTDENSE=str(CFG["first_dense"]),
                   DSV2_VOCAB=str(CFG["vocab"]), DSV2_MAXSEQ=str(CFG["max_seq"]))
        out = subprocess.run([str(exe)], env=env, capture_output=True, text=True, timeout=600).stdout
    print(out)
    ids = [int(x) for x in re.search(r"thvm gen ids: \[([^\]]*)\]", out).group(1).split(",")]
    top2 = [(int(m[0]), int(m[1]), float(m[2]), int(m[3]), float(m[4]))
            for m in re.findall(r"top2 step (\d+): tok=-?\d+\s+(\d+):(-?[\d.]+)\s+(-?\d+):(-?[\d.]+)", out)]
    np.savez_compressed(ROOT / "tests" / "golden" / name, seed=SEED, prompt=np.array(PROMPT),
                        gen_ids=np.array(ids, np.int32), top2=np.array(top2, np.float64),
                        digest=np.array(weight_digest(t)),
                        cfg=np.array(sorted(CFG.items()), dtype=object).astype(str))
    print(name, "gen ids", ids)


if __name__ == "__main__":
    main()
