"""Index build for the throughput-mode search path (runs once; its outputs are the tables the kernels read).

Mirrors, in order:
  * global centre c = mean of the first 50k vectors (src/rev_fanardb.py:37);
  * 4,096-cell spherical k-means over a 200k sample, 15 iterations, then every vector assigned to its
    best cell and the index sorted by cell (src/ideas_engine2.py:27-40);
  * cell means of the members (src/engine_cell.py:8-15) and their norms (src/engine_cell.py:26-32);
  * the tiered refinement code with uniform codebooks (throughput/s2lut.py:18-29, src/tiered.py);
  * the 256-direction PCA basis of the int8 code (throughput/e_brute.py:71-73) and the int8
    cell-residual codes (throughput/enginei8.py:19-27, on the GPU through libfvs);
  * the static (cell, block) work list (src/s1cell.py:157-168).
Random draws use numpy PCG64 seeds (the reference draws some from a CUDA generator, which cannot be
reproduced on another device).
"""
import numpy as np
import torch

from . import _lib, s2lut


def segment_sum(x, seg, n):
    """Row sums of x per segment id (seg sorted ascending, ids < n) as an [n, cols] tensor. Each segment is
    reduced on its own and written to its own row, so the result is the same on every run (a float
    index_add_ on the GPU adds with atomics, in an order that changes from run to run)."""
    out = torch.zeros((n, x.shape[1]), dtype=x.dtype, device=x.device)
    if len(seg):
        ids, counts = torch.unique_consecutive(seg, return_counts=True)
        out[ids] = torch.segment_reduce(x, "sum", lengths=counts, axis=0)
    return out


def spherical_kmeans(X16, nlist, seed=0, iters=15, sample=200000, chunk=50000):
    """Spherical k-means centroids (unit rows) fitted on a random sample (src/ideas_engine2.py:27-33)."""
    g = np.random.default_rng(seed)
    N = X16.shape[0]
    idx = torch.from_numpy(g.permutation(N)[:sample]).to(X16.device)
    samp = X16[idx].float()
    cen = samp[torch.from_numpy(g.permutation(len(samp))[:nlist]).to(X16.device)].clone()
    for _ in range(iters):
        a = torch.cat([(samp[j:j + chunk] @ cen.T).argmax(1) for j in range(0, len(samp), chunk)])
        o = torch.argsort(a, stable=True)
        cen = torch.nn.functional.normalize(segment_sum(samp[o], a[o], nlist) + 1e-9, dim=1)
    return cen


def assign(X16, cen, chunk=100000):
    return torch.cat([(X16[j:j + chunk].float() @ cen.T).argmax(1) for j in range(0, X16.shape[0], chunk)])


def cell_means(X16, order, cell, off, nlist, chunk=65536):
    """fp32 means of each cell's members (src/engine_cell.py:12-15): the rows X16[order] are in cell order,
    so each chunk's segment sums are added in chunk order (reproducible). X16 on the GPU or the host (rows
    gathered there and copied to cell's device); empty cells get the zero vector."""
    dev = cell.device
    means = torch.zeros(nlist, X16.shape[1], device=dev)
    oc = order.long().to(X16.device)
    N = order.shape[0]
    for j in range(0, N, chunk):
        means += segment_sum(X16[oc[j:j + chunk]].to(dev).float(), cell[j:j + chunk].long(), nlist)
    cnt = (off[1:] - off[:-1]).clamp(min=1).float().to(dev)
    return means / cnt[:, None]


def build_stage1_cells(X16, nlist=4096, seed=0):
    """Stage-1 tables: c, order (sorted position -> id, int32), off (numpy int64 [NC+1]), off_t (int32
    tensor), cell (cell of each sorted position), means16 (fp16 cell means), inv_mnorm."""
    dev = X16.device
    N = X16.shape[0]
    c = X16[:50000].float().mean(0)
    cen = spherical_kmeans(X16, nlist, seed)
    A = assign(X16, cen)
    order = torch.argsort(A, stable=True)
    off = torch.searchsorted(A[order].contiguous(), torch.arange(nlist + 1, device=dev))
    cell = A[order]
    means = cell_means(X16, order, cell, off, nlist)
    means16 = means.half().contiguous()
    inv_mnorm = (1.0 / means16.float().norm(dim=1).clamp(min=1e-12)).contiguous()
    return dict(c=c.contiguous(), order=order.to(torch.int32).contiguous(), off=off.cpu().numpy().astype(np.int64),
                off_t=off.to(torch.int32).contiguous(), cell=cell.to(torch.int32).contiguous(), means16=means16,
                inv_mnorm=inv_mnorm)


def pca_int8_basis(X16, R=256, nmean=200000, step=10):
    """Top-R principal directions of x - mu, mu = mean of the first 200k vectors, covariance of every
    10th vector (throughput/e_brute.py:71-73). The eigendecomposition runs in float64 on the host."""
    mu = X16[:nmean].float().mean(0)
    S = X16[::step].float() - mu
    cov = torch.cov(S.T).double().cpu().numpy()
    ev, V = np.linalg.eigh(cov)
    V = V[:, ::-1][:, :R].copy()
    return torch.from_numpy(V).float().to(X16.device).contiguous()


def sorted_cells(s1):
    """Cell of each sorted position (int32 tensor): s1["cell"], or searchsorted over the offsets as the
    reference derives it (throughput/enginei8.py:21)."""
    if s1.get("cell") is not None:
        return s1["cell"].to(torch.int32).contiguous()
    off = torch.as_tensor(np.asarray(s1["off"]) if "off" in s1 else s1["off_t"].cpu(), dtype=torch.int64)
    dev = s1["means16"].device
    N = int(off[-1])
    off = off.to(dev)
    return (torch.searchsorted(off, torch.arange(N, device=dev), right=True) - 1).to(torch.int32).contiguous()


def build_codes(s1, X16, V, R=256, chunk=65536):
    """(Z, zs, Vr): int8 codes of the cell residuals in sorted order, their scales and Vr = V[:, :R]; the
    reference's build_codes(s1, X16, V, R) (throughput/enginei8.py:19-27), on the GPU (fvs_build_codes).
    X16 fp16 [n_ids, d] in id order, on the GPU or in host memory (then gathered and copied chunk by chunk,
    as the reference does); s1 needs order, means16 and the cell offsets."""
    dev = s1["means16"].device
    Vr = V[:, :R].to(device=dev, dtype=torch.float32).contiguous()
    order = s1["order"].to(device=dev, dtype=torch.int32).contiguous()
    cell = sorted_cells(s1)
    means16 = s1["means16"].contiguous()
    if X16.is_cuda:
        Z, zs = _lib.build_codes(X16, order, cell, means16, Vr)
        return Z, zs, Vr
    N = order.shape[0]
    Z = torch.empty((N, R), dtype=torch.int8, device=dev)
    zs = torch.empty((N,), dtype=torch.float32, device=dev)
    oc = order.long().cpu()
    for j in range(0, N, chunk):
        xs = X16[oc[j:j + chunk]].to(dev).contiguous()
        n = xs.shape[0]
        ident = torch.arange(n, dtype=torch.int32, device=dev)
        Z[j:j + n], zs[j:j + n] = _lib.build_codes(xs, ident, cell[j:j + n].contiguous(), means16, Vr)
    return Z, zs, Vr


def emit_buffer(B, K, budget=1 << 29):
    """Emit buffer entries per query of the trellis engines' stage 1: the reference's max(4096, 16 K)
    (src/s1cell.py:180), raised towards the fallback's 65,536 while B * M * 8 bytes stay within `budget`.
    Results do not depend on it: a query that emits cnt >= K candidates above its threshold t0 holds the
    top-K (by estimate, then position) of all its probed rows, whatever t0 was, so the fallback the
    reference runs for an overflowing query (cnt > M) returns the same top-K. A larger buffer only saves
    that second stage-1 pass; underflows (cnt < K) still take it. B=None: the reference's size."""
    ref = max(4096, 16 * K)
    if B is None or B <= 0:
        return ref
    return max(ref, min(65536, budget // (8 * B)))


def static_blocks(off_t, BN=32):
    """All (cell, block) items of the index: cell, global block id, cell start and end, and MB = max blocks
    per cell + 1 (src/s1cell.py:161-168)."""
    off = off_t.long()
    s, e = off[:-1], off[1:]
    nb = torch.where(e > s, (e - 1) // BN - s // BN + 1, torch.zeros_like(s))
    cell = torch.repeat_interleave(torch.arange(len(s), device=off.device), nb)
    first = torch.cumsum(nb, 0) - nb
    blk = s[cell] // BN + torch.arange(len(cell), device=off.device) - first[cell]
    MB = int((int((e - s).max()) + BN - 1) // BN + 1)
    i32 = lambda x: x.to(torch.int32).contiguous()
    return (i32(cell), i32(blk), i32(s[cell]), i32(e[cell])), MB


def static_chunks(off_t, BN=32, CB=4):
    """Work items of the first pass: every cell's static blocks (static_blocks) grouped into chunks of up
    to CB consecutive global blocks (the first-pass kernel's items span four). Returns (cell, first row = BN * first global block, cell start, cell
    end) int32 tensors; each item covers blocks [blk0, min(blk0 + CB, last block of the cell + 1))."""
    off = off_t.long()
    s, e = off[:-1], off[1:]
    nb = torch.where(e > s, (e - 1) // BN - s // BN + 1, torch.zeros_like(s))
    nch = (nb + CB - 1) // CB
    cell = torch.repeat_interleave(torch.arange(len(s), device=off.device), nch)
    first = torch.cumsum(nch, 0) - nch
    blk0 = s[cell] // BN + CB * (torch.arange(len(cell), device=off.device) - first[cell])
    i32 = lambda x: x.to(torch.int32).contiguous()
    return i32(cell), i32(blk0 * BN), i32(s[cell]), i32(e[cell])


def row_chunks(off_t, rows=128):
    """Work items of the emit pass: every non-empty cell's rows in chunks of `rows` from its first row.
    Returns (cell, first row, cell start, cell end) int32 tensors. The emitted set is per row, so any
    grouping gives the same candidates; starting at the cell's first row leaves no block that straddles
    the cell start, and a cell of up to `rows` rows is a single item (the emit kernel's items span 128)."""
    off = off_t.long()
    s, e = off[:-1], off[1:]
    nch = (e - s + rows - 1) // rows
    cell = torch.repeat_interleave(torch.arange(len(s), device=off.device), nch)
    first = torch.cumsum(nch, 0) - nch
    r0 = s[cell] + rows * (torch.arange(len(cell), device=off.device) - first[cell])
    i32 = lambda x: x.to(torch.int32).contiguous()
    return i32(cell), i32(r0), i32(s[cell]), i32(e[cell])


def build_index(X16, nlist=4096, R=256, bits_per_dim=2.5, seed=0, with_codes=True):
    """Everything EngineI8 needs: (s1, code, Z, zs, Vr). X16: fp16 [N, d] in id order."""
    s1 = build_stage1_cells(X16, nlist, seed)
    lam, V = s2lut.pca_basis(X16, s1["c"])
    TS = s2lut.allocate(lam, int(bits_per_dim * X16.shape[1]))
    code = s2lut.encode_uniform_tiers(X16, s1["order"], s1["c"], V, TS, seed)
    s2lut.prepare_u(code)
    Vr = pca_int8_basis(X16, R)
    Z = zs = None
    if with_codes:
        Z, zs, Vr = build_codes(s1, X16, Vr, R)
    return s1, code, Z, zs, Vr
