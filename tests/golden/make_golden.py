"""Writes tests/golden/tiny_search.npz: the inputs and every stage output of one small batched search,
computed by the CPU oracle (oracle/oracle.c) on tables built by the product's host code.

The reference ships no unit-level vectors for this path, so these fixtures are the build's own pins:
test_golden.py checks that the oracle still reproduces them on the CPU and that the GPU kernels
reproduce them bit for bit. Regenerate only when a canonical operation order changes on purpose:
    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

N, D, NC, B = 512, 256, 8, 12
K, Z, NPROBE, KK = 48, 1.5, 4, 5
KNOBS = dict(MSZ=512, RHO=0.6, DELTA=0.07, LUTF=True, LUTH=True)


def main():
    import torch

    from fanarvse_paper_amd import datagen, index
    from oracle import oracle as orc

    X = datagen.gen(N, D, 6, 0.7, seed=0)
    Q = datagen.gen(B, D, 6, 0.7, seed=1, dtype=torch.float32).numpy()
    s1, code, _, _, Vr = index.build_index(X, nlist=NC, with_codes=False)
    Zc, zs = orc.build_codes(X.numpy(), s1["order"].numpy(), s1["cell"].numpy(), s1["means16"].numpy(), Vr.numpy())
    idx = orc.index_from_tables(s1, code, Zc, zs, Vr, X)
    out = orc.pipeline(idx, Q, K, Z, NPROBE, KK, knobs=KNOBS, fallback=False)
    TS = np.array(idx["TS"], np.int32)
    inputs = dict(Q=Q, c=idx["c"], order=idx["order"], off=idx["off"], mnorm=idx["mnorm"], Zc=idx["Z"], zs=idx["zs"],
                  rec=idx["rec"], TS=TS, deltas=idx["deltas"], toff=idx["toff"], soff=np.int32(idx["soff"]),
                  H=idx["H"], zq=out["z"], QM=out["QM"], Zq=out["Zq"],
                  params=np.array([K, NPROBE, KK, KNOBS["MSZ"]], np.int32), zval=np.float32(Z),
                  knobs=np.array([KNOBS["RHO"], KNOBS["DELTA"]], np.float64))
    keep = ["q8", "qs", "qc", "probe", "bm", "t0", "cnt", "pos", "est1", "ok", "ncnt", "L", "qsum", "qn2", "est",
            "sd", "ids", "I", "scores", "reads"]
    outputs = {f"out_{k}": out[k] for k in keep}
    outputs["out_n1"] = np.int32(out["n1"])
    outputs["out_r"] = np.int32(out["r"])
    # the emitted sets (order-free): sorted (pos) of the first min(cnt, M) buffer entries
    M = KNOBS["MSZ"]
    outputs["out_emitted"] = np.concatenate([np.sort(out["bpos"][q, :min(int(out["cnt"][q]), M)]) for q in range(B)])
    path = os.path.join(HERE, "tiny_search.npz")
    np.savez_compressed(path, **inputs, **outputs)
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
