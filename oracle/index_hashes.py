"""Checker: SHA-256 prefixes of every generated input and index table of the config-2 workload (1M x 1536,
NC 4096: rows, queries, cell tables, int8 codes and scales, PCA basis, stage-2 records) and of the config-3
trellis index on the same rows. Run it in two processes (or on two boxes) and compare the outputs: equal
lines mean the index build is bit-reproducible across processes.

    python oracle/index_hashes.py > a.txt; python oracle/index_hashes.py > b.txt; diff a.txt b.txt
"""
import hashlib
import os
import sys

import numpy as np
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from fanarvse_paper_amd import datagen, index, trellis  # noqa: E402


def H(t):
    if torch.is_tensor(t):
        t = t.detach().contiguous().cpu().numpy()
    return hashlib.sha256(np.ascontiguousarray(t).view(np.uint8).tobytes()).hexdigest()[:16]

dev = "cuda"
n = int(sys.argv[1]) if len(sys.argv) > 1 else 1_000_000
X = datagen.gen(n, 1536, 1024, 0.7, seed=0, device=dev)
Q = datagen.gen(2000, 1536, 1024, 0.7, seed=1, device=dev, dtype=torch.float32)
out = {"X": H(X), "Q": H(Q)}
s1, code, Z, zs, Vr = index.build_index(X, nlist=4096)
for k in ("order", "off_t", "means16", "inv_mnorm", "c", "cell"):
    if k in s1: out["s1." + k] = H(s1[k])
out.update({"Z": H(Z), "zs": H(zs), "Vr": H(Vr), "rec": H(code["rec"]), "V": H(code["V"]), "VP16": H(code["VP16"])})
ts1, tcode = trellis.build_index(X, nlist=4096)
for k in ("order", "off_t", "means16", "W1", "words", "scale1"):
    if k in ts1: out["tr." + k] = H(ts1[k])
out["tr.rec"] = H(tcode["rec"])
for k, v in out.items():
    print(f"{k} {v}", flush=True)
