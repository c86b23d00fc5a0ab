"""Synthetic base/query sets of the benchmark configurations (no dataset ships with the reference).

gen(n, d, n_clusters, alpha, seed): a mixture of n_clusters Gaussian clusters with centres N(0, I_d);
each point is its centre plus N(0, 0.5^2 * diag(lam)), lam_i proportional to i^-alpha normalised to
mean 1; one fixed random orthogonal rotation (QR of a Gaussian matrix with the sign fix, so it is
Haar), then L2 normalisation. Seed streams: clusters `cluster_seed` (3), rotation `rot_seed` (2),
points `seed` (base 0, queries 1). Rows are generated in chunks of `chunk`, each chunk from its own
numpy PCG64 stream keyed by (seed, chunk index), so the output does not depend on the device used
for the rotation product.
"""
import numpy as np
import torch

CHUNK = 65536


def spectrum(d, alpha):
    lam = np.arange(1, d + 1, dtype=np.float64) ** (-alpha)
    return (lam / lam.mean()).astype(np.float32)


def rotation(d, rot_seed=2):
    g = np.random.default_rng(rot_seed).standard_normal((d, d))
    q, r = np.linalg.qr(g)
    return (q * np.sign(np.diag(r))[None, :]).astype(np.float32)


def centres(n_clusters, d, cluster_seed=3):
    return np.random.default_rng(cluster_seed).standard_normal((n_clusters, d), dtype=np.float32)


def gen(n, d, n_clusters, alpha, seed, device="cpu", dtype=torch.float16, cluster_seed=3, rot_seed=2, chunk=CHUNK):
    """n x d unit vectors (torch tensor on `device`, fp16 by default)."""
    C = torch.from_numpy(centres(n_clusters, d, cluster_seed)).to(device)
    Q = torch.from_numpy(rotation(d, rot_seed)).to(device)
    sl = torch.from_numpy(0.5 * np.sqrt(spectrum(d, alpha))).to(device)
    out = torch.empty((n, d), dtype=dtype, device=device)
    for ci, j in enumerate(range(0, n, chunk)):
        m = min(chunk, n - j)
        rng = np.random.default_rng([seed, ci])
        a = torch.from_numpy(rng.integers(0, n_clusters, m)).to(device)
        noise = torch.from_numpy(rng.standard_normal((m, d), dtype=np.float32)).to(device)
        p = C[a] + noise * sl
        x = p @ Q
        x = x / x.norm(dim=1, keepdim=True)
        out[j:j + m] = x.to(dtype)
    return out


def ground_truth(X16, Qf, k, chunk=262144):
    """Exact inner-product top-k (ids, descending) of fp32 queries against the fp16 base cast to fp32
    (the convention of the reference's src/v16_prep.py:44)."""
    best_v = None
    best_i = None
    for j in range(0, X16.shape[0], chunk):
        s = Qf.float() @ X16[j:j + chunk].float().T
        v, i = s.topk(min(k, s.shape[1]), dim=1)
        i = i + j
        if best_v is None:
            best_v, best_i = v, i
        else:
            cv = torch.cat([best_v, v], 1)
            ci = torch.cat([best_i, i], 1)
            t = cv.topk(k, dim=1)
            best_v, best_i = t.values, ci.gather(1, t.indices)
    return best_i
