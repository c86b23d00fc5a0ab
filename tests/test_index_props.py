"""Properties that pin the index-build tables a1 and a2 on the CPU (the builders are torch code that runs on
any device): the stage-1 cell tables of build_stage1_cells (src/engine_cell.py:8-32, src/ideas_engine2.py:27-40)
and the PCA basis of pca_int8_basis (throughput/e_brute.py:8-10), each against an independent float64
numpy restatement of what the table must hold."""
import numpy as np
import torch

from fanarvse_paper_amd import datagen, index


def small_set(n=6000, d=64, seed=4):
    return datagen.gen(n, d, 16, 0.7, seed=seed)


def test_stage1_cells_tables():
    X = small_set()
    NC = 24
    s1 = index.build_stage1_cells(X, NC, seed=3)
    N = X.shape[0]
    order = s1["order"].numpy().astype(np.int64)
    cell = s1["cell"].numpy().astype(np.int64)
    off = s1["off"]
    assert np.array_equal(np.sort(order), np.arange(N))                     # a permutation of the ids
    assert np.all(np.diff(cell) >= 0) and cell.min() >= 0 and cell.max() < NC  # sorted by cell
    # off[c] = number of rows in cells below c, i.e. searchsorted over the sorted cells
    assert np.array_equal(off, np.searchsorted(cell, np.arange(NC + 1), side="left"))
    assert np.array_equal(s1["off_t"].numpy(), off.astype(np.int32))
    # cell means: the float64 mean of each cell's members, rounded once to fp16 (empty cells: zero)
    X64 = X.float().numpy().astype(np.float64)
    means64 = np.zeros((NC, X.shape[1]))
    for c in range(NC):
        mem = order[off[c]:off[c + 1]]
        if len(mem):
            means64[c] = X64[mem].mean(0)
    m16 = s1["means16"].float().numpy().astype(np.float64)
    ulp = np.spacing(np.abs(means64).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(m16 - means64) <= ulp + 1e-6)
    # inv_mnorm = 1 / ||means16|| in fp32
    inv = 1.0 / np.maximum(np.linalg.norm(m16, axis=1), 1e-12)
    assert np.allclose(s1["inv_mnorm"].numpy(), inv, rtol=2e-6)
    # c = mean of the first 50k rows (all of them here)
    assert np.allclose(s1["c"].numpy(), X64[:50000].mean(0), atol=1e-6)
    # every row sits in the cell whose centroid gives it the largest inner product: the assignment is
    # consistent with the rows' own cells up to ties, so the per-cell member means are closer (by inner
    # product) to their own rows than a random other cell's mean is on average
    own = np.einsum("nd,nd->n", X64[order], m16[cell])
    other = np.einsum("nd,nd->n", X64[order], m16[(cell + 7) % NC])
    assert own.mean() > other.mean()


def test_stage1_cells_deterministic():
    X = small_set(n=3000, seed=5)
    a = index.build_stage1_cells(X, 16, seed=1)
    b = index.build_stage1_cells(X, 16, seed=1)
    for k in ("order", "cell", "off_t", "means16", "inv_mnorm", "c"):
        assert torch.equal(a[k], b[k]), k


def test_pca_basis_orthonormal_descending():
    X = small_set(n=8000, d=48, seed=6)
    R = 20
    V = index.pca_int8_basis(X, R=R, nmean=5000, step=3).numpy().astype(np.float64)
    assert V.shape == (48, R)
    assert np.allclose(V.T @ V, np.eye(R), atol=1e-5)                        # orthonormal columns
    # the covariance it diagonalises: every 3rd row minus the mean of the first 5000, as float64 numpy
    X64 = X.float().numpy().astype(np.float64)
    mu = X64[:5000].mean(0)
    C = np.cov((X64[::3] - mu).T)
    lam = np.einsum("dr,de,er->r", V, C, V)                                  # Rayleigh quotients
    assert np.all(np.diff(lam) <= 1e-9 * lam[0])                             # descending eigen-order
    assert np.allclose(C @ V, V * lam, atol=1e-6 * lam[0])                   # eigenvectors of C
    ev = np.sort(np.linalg.eigvalsh(C))[::-1]
    assert np.allclose(lam, ev[:R], rtol=1e-6, atol=1e-9 * ev[0])            # the top R eigenvalues
