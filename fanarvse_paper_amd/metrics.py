"""Recall and read statistics (src/rev_fanardb.py:134-142)."""
import numpy as np


def recall(I, GT, k=10):
    """Mean over queries of |I[:k] intersect GT[:k]| / k, rounded to 4 decimals (src/rev_fanardb.py:134-136)."""
    I = np.asarray(I)
    GT = np.asarray(GT)
    return round(float(np.mean([len(set(I[i, :k].tolist()) & set(GT[i, :k].tolist())) / k for i in range(len(I))])), 4)


def cand_recall(C, GT, k=10):
    """Share of the true top-k inside the candidate set (src/rev_fanardb.py:137-139)."""
    C = np.asarray(C)
    GT = np.asarray(GT)
    return round(float(np.mean([len(set(C[i].tolist()) & set(GT[i, :k].tolist())) / k for i in range(len(C))])), 4)


def read_stats(r):
    """Distribution of exact reads per query (src/rev_fanardb.py:140-142)."""
    r = np.asarray(r)
    return {"reads_mean": round(float(r.mean()), 2), "reads_p50": float(np.percentile(r, 50)),
            "reads_p90": float(np.percentile(r, 90)), "reads_p99": float(np.percentile(r, 99)),
            "reads_max": int(r.max()), "frac_zero_reads": round(float((r == 0).mean()), 4)}
