"""Uniform tiered refinement code (build side) and the LUT stage-2 entry points.

Mirrors throughput/s2lut.py (uniform_cb, encode_uniform, prepare_u, luts_fused, score_lut) and the
pieces of src/tiered.py it relies on (pca_basis, allocate, the bit-plane layout), plus the packed
record layout of src/tiered_fused.py:112-125 that the GPU scorer reads.

Build-time arithmetic runs in torch on whatever device the data is on; the search-time entry points
(luts_fused, score_lut) call the gfx950 kernels of libfvs.so.
"""
import math

import numpy as np
import torch
from scipy.special import ndtr
from scipy.stats import norm

from . import _lib

G = 32  # coordinates per allocation group (src/tiered.py:139)


# --------------------------------------------------------------------------- scalar quantiser tables
def lloyd_max(b, iters=20000, tol=1e-13):
    """Lloyd-Max quantiser of N(0, 1) with 2^b levels, iterated on the exact density from the
    asymptotically optimal (companding) start, levels at the quantiles of N(0, 3).
    Returns (levels, mse). The reference fits the same quantiser with faiss k-means on 400k samples
    (src/tiered.py:132-136)."""
    n = 2 ** b
    y = np.sqrt(3.0) * norm.ppf((np.arange(n) + 0.5) / n)
    pdf = lambda x: np.exp(-0.5 * x * x) / np.sqrt(2 * np.pi)
    for _ in range(iters):
        t = np.concatenate([[-np.inf], (y[1:] + y[:-1]) / 2, [np.inf]])
        p = ndtr(t[1:]) - ndtr(t[:-1])
        ynew = (pdf(t[:-1]) - pdf(t[1:])) / p
        if np.max(np.abs(ynew - y)) < tol:
            y = ynew
            break
        y = ynew
    t = np.concatenate([[-np.inf], (y[1:] + y[:-1]) / 2, [np.inf]])
    p = ndtr(t[1:]) - ndtr(t[:-1])
    return y, float(1.0 - np.sum(p * y * y))


_DIST = None


def dist_table():
    """DIST[b] = Lloyd-Max distortion of a unit Gaussian at b bits, DIST[0] = 1 (src/tiered.py:132)."""
    global _DIST
    if _DIST is None:
        _DIST = {0: 1.0}
        for b in range(1, 9):
            _DIST[b] = lloyd_max(b)[1]
    return _DIST


def gaussian_mse(levels):
    """Exact E[(g - Q(g))^2], g ~ N(0, 1), for nearest-level quantisation to the sorted `levels`."""
    y = np.asarray(levels, dtype=np.float64)
    t = np.concatenate([[-np.inf], (y[1:] + y[:-1]) / 2, [np.inf]])
    a, b_ = t[:-1], t[1:]
    P = norm.cdf(b_) - norm.cdf(a)
    pa, pb = norm.pdf(a), norm.pdf(b_)
    with np.errstate(invalid="ignore"):  # inf * 0 at the outer cells, replaced by 0
        apa = np.where(np.isinf(a), 0.0, a * pa)
        bpb = np.where(np.isinf(b_), 0.0, b_ * pb)
    # integral over [a, b] of (g - y)^2 phi(g) = (1 + y^2) P + a phi(a) - b phi(b) - 2 y (phi(a) - phi(b))
    return float(np.sum((1 + y * y) * P + apa - bpb - 2 * y * (pa - pb)))


def uniform_cb(b, grid=None):
    """Uniform codebook Delta_b * (j - (2^b - 1)/2): Delta_b minimises the Gaussian distortion over the
    reference's grid linspace(0.02, 2.5, 600) (throughput/s2lut.py:9-16). The reference estimates the
    distortion by Monte Carlo on 2M CUDA-RNG samples; here it is the exact integral.
    Returns (mse, delta, levels, thresholds)."""
    grid = np.linspace(0.02, 2.5, 600) if grid is None else grid
    mid = (2 ** b - 1) / 2
    best = None
    for delta in grid:
        lv = (np.arange(2 ** b) - mid) * delta
        m = gaussian_mse(lv)
        if best is None or m < best[0]:
            best = (m, float(delta))
    m, delta = best
    lv = (np.arange(2 ** b) - mid) * delta
    return m, delta, lv, (lv[1:] + lv[:-1]) / 2


# --------------------------------------------------------------------------- basis and bit allocation
def pca_basis(X16, c, n=50000):
    """Eigenvalues (descending) and basis of the normalised residuals x - c over the first n rows
    (src/tiered.py:141-143). The eigendecomposition runs in float64 on the host."""
    S = X16[:n].float() - c
    S = S / S.norm(dim=1, keepdim=True)
    cov = torch.cov(S.T).double().cpu().numpy()
    ev, V = np.linalg.eigh(cov)
    ev = np.clip(ev[::-1].copy(), 1e-12, None)
    V = V[:, ::-1].copy()
    return torch.from_numpy(ev).float(), torch.from_numpy(V).float().to(X16.device)


def allocate(lam, B, bmin=1, bmax=8):
    """Greedy reverse water-filling of B bits over groups of 32 coordinates (src/tiered.py:145-153).
    Returns the tiers [(start, end, bits)] of consecutive groups with equal width."""
    DIST = dist_table()
    lam = np.asarray(lam.cpu() if torch.is_tensor(lam) else lam, dtype=np.float64)
    d = len(lam)
    NG = d // G
    lamg = lam[:NG * G].reshape(NG, G).sum(1)
    b = np.full(NG, bmin)
    left = B - bmin * d
    while left >= G:
        gain = [lamg[i] * (DIST[b[i]] - DIST[b[i] + 1]) if b[i] < bmax else -1 for i in range(NG)]
        i = int(np.argmax(gain))
        b[i] += 1
        left -= G
    T, st = [], 0
    for i in range(1, NG + 1):
        if i == NG or b[i] != b[st]:
            T.append((st * G, i * G, int(b[st])))
            st = i
    return T


def tier_rotations(TS, seed=0):
    """One Haar-like rotation per tier: Q of the QR factorisation of a Gaussian matrix
    (src/tiered.py:157-158 draws it from a CUDA generator seeded 100 + seed; this build uses numpy PCG64)."""
    rng = np.random.default_rng(100 + seed)
    return [torch.from_numpy(np.linalg.qr(rng.standard_normal((e - s, e - s)))[0].astype(np.float32))
            for s, e, _ in TS]


# --------------------------------------------------------------------------- encoding and packing
def record_layout(TS):
    """Byte offsets of each tier's planes, of the (scale, sigma) pairs, and the record size rounded to
    64 bytes (src/tiered_fused.py:112-116)."""
    toff, o = [], 0
    for s, e, b in TS:
        toff.append(o)
        o += b * (e - s) // 8
    soff = o
    RB = (o + 4 * len(TS) + 63) // 64 * 64
    return toff, soff, RB


_SH = torch.arange(7, -1, -1, dtype=torch.uint8)


def _pack_bits(bit):
    """(n, m) bool -> (n, m/8) uint8, first coordinate in the most significant bit (src/tiered.py:137-138)."""
    sh = _SH.to(bit.device)
    return (bit.reshape(bit.shape[0], -1, 8).to(torch.uint8) << sh).sum(2).to(torch.uint8)


def lloyd_cb(b):
    """(levels, thresholds) of the b-bit Lloyd-Max quantiser of N(0, 1) (the reference's tiered.CB[b],
    src/tiered.py:6-10, fitted there by faiss k-means on 400k samples; here the exact fixed point)."""
    y, _ = lloyd_max(b)
    return y, (y[1:] + y[:-1]) / 2


def encode_uniform(code, host16, order, c, seed=0):
    """The reference's encode_uniform(code, host16, order, c, seed) (throughput/s2lut.py:18-29): the tiered
    refinement of `code` (its tiers TS and PCA basis V) re-encoded with uniform codebooks. Returns a new
    code dict: `code`'s entries plus the uniform tables (records, deltas, rotations)."""
    out = dict(code)
    out.pop("VP", None)
    out.pop("VP16", None)
    out.update(encode_uniform_tiers(host16, order, c, code["V"], code["TS"], seed))
    return out


def encode_uniform_tiers(X16, order, c, V, TS, seed=0, chunk=16384):
    """Uniform-codebook tiered code of x - c for the vectors in sorted order (throughput/s2lut.py:18-29
    with src/tiered.py:155-170), written straight into packed records.
    Returns the code dict: TS, V, rots, deltas, cb_uniform, rec [N, RB] uint8, RB, soff, toff, bytes."""
    return encode_tiered(X16, order, c, V, TS, seed, chunk, kind="uniform")


def encode_lloyd(X16, order, c, V, TS, seed=0, chunk=16384):
    """Lloyd-Max tiered code of x - c (src/tiered.py:29-44, the default engine's stage 2) in the same
    packed record layout (src/tiered_fused.py:112-125). The code dict has `levels` {b: levels} and `cb`,
    the [T, 256] f32 table of each tier's levels that the GPU scorer reads."""
    return encode_tiered(X16, order, c, V, TS, seed, chunk, kind="lloyd")


def encode_tiered(X16, order, c, V, TS, seed=0, chunk=16384, kind="uniform"):
    """Tier records of the vectors X16[order] (X16 on the GPU, or in host memory: rows are gathered on the
    host and the encode runs on V's device)."""
    dev = V.device
    N = len(order)
    rots = tier_rotations(TS, seed)
    deltas, cbs, levels = {}, {}, {}
    for b in sorted({bb for _, _, bb in TS}):
        if kind == "uniform":
            _, delta, lv, th = uniform_cb(b)
            deltas[b] = delta
        else:
            lv, th = lloyd_cb(b)
        levels[b] = np.asarray(lv, dtype=np.float32)
        cbs[b] = (torch.tensor(lv, dtype=torch.float32, device=dev), torch.tensor(th, dtype=torch.float32, device=dev))
    toff, soff, RB = record_layout(TS)
    rec = torch.zeros((N, RB), dtype=torch.uint8, device=dev)
    ss = torch.empty((N, len(TS), 2), dtype=torch.float16, device=dev)
    oc = order.long().to(X16.device)
    Pt = [P.to(dev) for P in rots]
    c = c.to(dev)
    for j in range(0, N, chunk):
        Zc = (X16[oc[j:j + chunk]].to(dev).float() - c) @ V
        n = len(Zc)
        for t, ((s, e, bb), P) in enumerate(zip(TS, Pt)):
            F = Zc[:, s:e] @ P
            nf = F.norm(dim=1).clamp(min=1e-12)
            dt = e - s
            Fu = F / nf[:, None] * dt ** 0.5
            cb, th = cbs[bb]
            q = torch.bucketize(Fu, th)
            Y = cb[q]
            yn = Y.norm(dim=1)
            ct = (Fu * Y).sum(1) / (yn * dt ** 0.5)
            kb = dt // 8
            for p in range(bb):
                o = toff[t] + p * kb
                rec[j:j + n, o:o + kb] = _pack_bits(((q >> (bb - 1 - p)) & 1).bool())
            ss[j:j + n, t, 0] = (nf / (ct * yn)).half()
            ss[j:j + n, t, 1] = (nf * torch.sqrt((1 - ct ** 2).clamp(min=0)) / (ct * (dt - 1) ** 0.5)).half()
    rec[:, soff:soff + 4 * len(TS)] = ss.reshape(N, -1).view(torch.uint8)
    nbytes = sum((e - s) * bb for s, e, bb in TS) / 8 + 4 * len(TS)
    cbt = torch.zeros((len(TS), 256), dtype=torch.float32)
    for t, (_, _, bb) in enumerate(TS):
        cbt[t, :2 ** bb] = torch.from_numpy(levels[bb])
    if kind == "lloyd":
        return dict(TS=TS, V=V, rots=rots, kind=kind, levels=levels, cb=cbt.to(dev), rec=rec, RB=RB, soff=soff,
                    toff=toff, bytes=nbytes)
    cb_uniform = {b: (torch.arange(2 ** b).float() - (2 ** b - 1) / 2) * d_ for b, d_ in deltas.items()}
    return dict(TS=TS, V=V, rots=rots, kind=kind, deltas=deltas, cb_uniform=cb_uniform, rec=rec, RB=RB, soff=soff, toff=toff,
                bytes=nbytes)


def prepare_u(code):
    """Fold the PCA basis and the tier rotations into one query-side matrix VP = V @ diag(P_t) and keep
    its fp16 copy VP16 (throughput/s2lut.py:31-37)."""
    if "VP16" in code:
        return
    V = code["V"]
    d = V.shape[0]
    D = torch.zeros(d, d, device=V.device)
    for (s, e, _), P in zip(code["TS"], code["rots"]):
        D[s:e, s:e] = P.to(V.device)
    VP = V @ D
    code["VP16"] = VP.half().contiguous()
    if code.get("kind") == "lloyd":
        code["VP"] = VP.contiguous()  # the default engine rotates fp32 queries (src/tiered_fused.py:47-57)


# --------------------------------------------------------------------------- search-time entry points
def rotate(code, Qh):
    """Rotated tier queries Zq = Qh @ VP16[:, :D], an fp16 GEMM with fp16 output (throughput/s2lut.py:122)."""
    prepare_u(code)
    D = code["TS"][-1][1]
    return (Qh @ code["VP16"][:, :D]).contiguous()


def luts_fused(code, Qh, half=False):
    """(L, qsum, qn2) of fp16 queries (throughput/s2lut.py:118-126): the rotated queries, then the nibble
    tables on the GPU."""
    return _lib.lut_build(rotate(code, Qh), code["TS"], half)


def score_lut(code, qc, pos, pre, ncnt=None, nt=None):
    """(est, sd) of candidates `pos` [B, K] (throughput/s2lut.py:92-106); nt: over the first nt tiers only
    (the reference's TS[:nt], throughput/s2lut.py:93), with the full tables `pre`."""
    return _lib.lut_score(pos, qc, pre, code, ncnt, nt)
