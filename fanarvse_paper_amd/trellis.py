"""Bitshift-trellis cell-residual codes of the default engine (latency mode, benchmark config 3).

A vector's stage-1 code is the Viterbi path of its normalised cell residual through a 2^L-state
bitshift trellis with one bit per coordinate: the stream holds the L bits of the first state and then
the newest bit of each later state; coordinate j decodes to tab[state_j] with tab = alpha * T and T a
fixed pseudo-random Gaussian table (src/trellis.py:12-15, src/trellis_scan.py:10-18). The words and
the per-vector fp16 scale are written by the GPU encoder (fvs_trellis_encode); this module holds the
table, the step-size choice and the index build driver (src/rev_fanardb.py:33-61,
src/engine_cell.py:8-32).
"""
import numpy as np
import torch
from scipy.stats import norm

from . import _lib, index

L_DEFAULT = 10
R_DEFAULT = 256


def make_table(L=L_DEFAULT, seed=0):
    """T[s] = Phi^-1((perm[s] + 1/2) / 2^L), perm = numpy PCG64(seed).permutation(2^L) (src/trellis.py:12-15)."""
    S = 2 ** L
    perm = np.random.default_rng(seed).permutation(S)
    return norm.ppf((perm + 0.5) / S).astype(np.float32)


def n_words(R, L):
    return (R + L - 1 + 31) // 32


def paths_to_words(path, L):
    """Host packing of state paths [n, R] into words [n, W] uint32 (src/trellis_scan.py:10-18)."""
    path = np.asarray(path, dtype=np.int64)
    n, R = path.shape
    nbits = R + L - 1
    W = n_words(R, L)
    bits = np.zeros((n, W * 32), dtype=np.uint64)
    bits[:, :L] = (path[:, :1] >> np.arange(L - 1, -1, -1)) & 1
    bits[:, L:nbits] = path[:, 1:] & 1
    w = (bits.reshape(n, W, 32) << np.arange(31, -1, -1, dtype=np.uint64)).sum(2)
    return (w & 0xFFFFFFFF).astype(np.uint32)


def decode_states(words, R, L):
    """Host decode of the state windows [n, R] (src/trellis_scan.py:36-44)."""
    words = np.asarray(words, dtype=np.uint64)
    n, W = words.shape
    j = np.arange(R)
    wi, off = j // 32, j % 32
    w0 = words[:, wi]
    w1 = np.where(wi + 1 < W, words[:, np.minimum(wi + 1, W - 1)], 0).astype(np.uint64)
    comb = (w0 << np.uint64(32)) | w1
    return ((comb >> (np.uint64(64 - L) - off.astype(np.uint64))) & np.uint64(2 ** L - 1)).astype(np.int64)


def encode(Zs, nz, tab, L=L_DEFAULT, paths=False):
    """(words [n, W] uint32 as int32 tensor, scale1 [n] fp16[, paths [n, R] int32]) of normalised rows Zs [n, R]
    (f32, |row| = sqrt(R)) with norms nz, on the GPU."""
    n, R = Zs.shape
    W = n_words(R, L)
    words = torch.empty((n, W), dtype=torch.int32, device=Zs.device)
    scale1 = torch.empty((n,), dtype=torch.float16, device=Zs.device)
    pth = torch.empty((n, R), dtype=torch.int32, device=Zs.device) if paths else None
    _lib.trellis_encode(Zs, nz, tab, L, words, scale1, pth)
    return (words, scale1, pth) if paths else (words, scale1)


def choose_alpha(T, L=L_DEFAULT, R=R_DEFAULT, n=512, seed=0, device="cuda"):
    """Step size alpha minimising the trellis MSE of n Gaussian rows over linspace(0.6, 1.3, 15)
    (src/rev_fanardb.py:39-42; the rows come from numpy PCG64 here, a CUDA generator there)."""
    G = torch.from_numpy(np.random.default_rng(seed).standard_normal((n, R), dtype=np.float32)).to(device)
    Tt = torch.from_numpy(T).to(device)
    nz = torch.ones(n, device=device)
    best = None
    for a in np.linspace(0.6, 1.3, 15):
        tab = (float(a) * Tt).contiguous()
        _, _, pth = encode(G, nz, tab, L, paths=True)
        m = float(((G - tab[pth.long()]) ** 2).mean())
        if best is None or m < best[0]:
            best = (m, float(a))
    return best[1]


def rotation_basis(X16, c, R=R_DEFAULT, seed=0, n=50000):
    """W1 = V[:, :R] @ Q: the top-R PCA basis of the first n centred rows times a Haar rotation of R^R
    (src/rev_fanardb.py:36-37; Q from numpy PCG64 here)."""
    S = X16[:n].float() - c
    cov = torch.cov(S.T).double().cpu().numpy()
    ev, V = np.linalg.eigh(cov)
    V = V[:, ::-1][:, :R].copy()
    q, r = np.linalg.qr(np.random.default_rng(200 + seed).standard_normal((R, R)))
    q = q * np.sign(np.diag(r))[None, :]
    return torch.from_numpy((V @ q).astype(np.float32)).to(X16.device)


def encode_cells(X16, s1, W1, tab, L=L_DEFAULT, chunk=16384, means=None):
    """Trellis codes of the cell residuals x - means[cell] in sorted order (src/engine_cell.py:8-24):
    Z = (x - m) @ W1, nz = |Z|, Zs = Z / nz * sqrt(R), words and scale1 from the GPU encoder. means: the fp32
    cell means (default: s1["means16"]); X16 on the GPU or the host (rows gathered there)."""
    dev = W1.device
    order = s1["order"].long().to(X16.device)
    cell = index.sorted_cells(s1).long().to(dev)
    means = s1["means16"].float() if means is None else means
    N = len(order)
    R = W1.shape[1]
    words = torch.empty((N, n_words(R, L)), dtype=torch.int32, device=dev)
    scale1 = torch.empty((N,), dtype=torch.float16, device=dev)
    for j in range(0, N, chunk):
        Z = (X16[order[j:j + chunk]].to(dev).float() - means[cell[j:j + chunk]]) @ W1
        nz = Z.norm(dim=1).clamp(min=1e-6)
        Zs = (Z / nz[:, None] * R ** 0.5).contiguous()
        words[j:j + len(Z)], scale1[j:j + len(Z)] = encode(Zs, nz.contiguous(), tab, L)
    return words, scale1


def cellify(s1, host16, L=L_DEFAULT):
    """The reference's cellify(s1) (src/engine_cell.py:8-24): the stage-1 trellis codes of an index already
    routed to its final cells, re-encoded against the cell means. s1 needs order, off, W1 and tab; the
    reference reads the base vectors and L from its `rf` module, here they are arguments (host16 fp16
    [N, d] in id order, on the GPU or the host). Returns dict(s1) with words and scale1 (codes of
    x - mean(cell), fp32 means), means16 (the fp16 means) and cell."""
    out = dict(s1)
    W1, tab = s1["W1"], s1["tab"]
    dev = W1.device
    off = torch.as_tensor(np.asarray(s1["off"]), dtype=torch.int64, device=dev)
    NC = len(off) - 1
    N = int(off[-1])
    cell = (torch.searchsorted(off, torch.arange(N, device=dev), right=True) - 1).to(torch.int32).contiguous()
    means = index.cell_means(host16, s1["order"], cell, off, NC)
    out["cell"] = cell
    out["words"], out["scale1"] = encode_cells(host16, out, W1, tab, L, means=means)
    out["means16"] = means.half().contiguous()
    out["L"] = L
    return out


def compact(s1c):
    """The reference's compact(s1c) (src/engine_cell.py:26-32): one fp16 table of cell means serves routing
    (key q.mean / |mean|) and the stage-1 pair term; inv_mnorm = 1 / |means16| (>= 1e-12), int32 ids,
    cen = inv_mnorm. Also the int32 offsets off_t the kernels read."""
    out = dict(s1c)
    nrm = out["means16"].float().norm(dim=1).clamp(min=1e-12)
    out["inv_mnorm"] = (1.0 / nrm).contiguous()
    out["order"] = out["order"].to(torch.int32).contiguous()
    out["cen"] = out["inv_mnorm"]
    out["off"] = np.asarray(out["off"]).astype(np.int64)
    out["off_t"] = torch.as_tensor(out["off"], dtype=torch.int32, device=nrm.device).contiguous()
    return out


def build_index(X16, nlist=4096, R=R_DEFAULT, L=L_DEFAULT, bits_per_dim=2.5, seed=0):
    """The default engine's tables: (s1, code). s1 holds the cell tables of index.build_stage1_cells plus
    W1, tab, alpha, words, scale1 (cell residual trellis codes); code is the Lloyd-Max tiered stage-2 code
    of x - c (src/v19_final.py:27-29: make -> cellify -> compact)."""
    from . import s2lut

    s1 = index.build_stage1_cells(X16, nlist, seed=seed)
    c = s1["c"]
    W1 = rotation_basis(X16, c, R, seed)
    T = make_table(L)
    alpha = choose_alpha(T, L, R, device=X16.device)
    tab = (alpha * torch.from_numpy(T)).to(X16.device).contiguous()
    s1.update(W1=W1, tab=tab, alpha=alpha, L=L)
    s1 = compact(cellify(s1, X16, L))
    lam, V = s2lut.pca_basis(X16, c)
    TS = s2lut.allocate(lam, int(bits_per_dim * X16.shape[1]))
    code = s2lut.encode_lloyd(X16, s1["order"], c, V, TS, seed=seed)
    return s1, code
