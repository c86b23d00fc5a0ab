"""CPU oracle of the FanarVSE throughput-mode search path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may import this module; the
product (fanarvse_paper_amd) never does. Integer bookkeeping is restated here in numpy; every
floating-point stage calls oracle.c (built by oracle/Makefile into liboracle.so), which follows the
reference's arithmetic with the canonical operation order of include/fvs.h.

References (under /root/reference):
    static_blocks      src/s1cell.py:161-168
    pairs              throughput/enginei8.py:11-16
    params             throughput/enginei8.py:40-47
    pipeline           throughput/enginei8.py:36-120 (stage1_i8, _gpu NROUTE branch, _finish, _fallback)
    recall             src/rev_fanardb.py:134-136
    tr_params          src/s1cell.py:176-190, src/engine_cell.py:78
    tr_pipeline        src/engine_cell.py:74-102 (EngineS._gpu and its fallback), src/engine3.py:135-146
Pinned by tests/test_oracle_*.py (closed forms, brute force, the paper's lemmas, planted mistakes).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a


I64, I32, F32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float


# ------------------------------------------------------------------------------------ numpy parts
def static_blocks(off, BN=32):
    """(pcell, pblk, ps, pe, MB): every (cell, BN-row block) of a cell-sorted index (src/s1cell.py:161-168)."""
    off = np.asarray(off, dtype=np.int64)
    s, e = off[:-1], off[1:]
    nb = np.where(e > s, (e - 1) // BN - s // BN + 1, 0)
    cell = np.repeat(np.arange(len(s)), nb)
    first = np.cumsum(nb) - nb
    blk = s[cell] // BN + np.arange(len(cell)) - first[cell]
    MB = int((int((e - s).max()) + BN - 1) // BN + 1)
    return cell.astype(np.int32), blk.astype(np.int32), s[cell].astype(np.int32), e[cell].astype(np.int32), MB


def pairs(probe, NC, QM16, mnorm=None, qadd=None):
    """(qid, coff, ccnt, qcp, o) of the (query, cell) pairs (throughput/enginei8.py:11-16): a stable sort of
    the flattened cell ids, per-cell counts and offsets, qcp = f32(QM[q, c]) * |m_c|."""
    B, npr = probe.shape
    flat = probe.reshape(-1).astype(np.int64)
    o = np.argsort(flat, kind="stable")
    qid = (o // npr).astype(np.int32)
    ccnt = np.bincount(flat, minlength=NC).astype(np.int32)
    coff = (np.cumsum(ccnt) - ccnt).astype(np.int32)
    fo = flat[o]
    qcp = np.asarray(QM16).view(np.float16)[qid, fo].astype(np.float32)
    if mnorm is not None:
        qcp = qcp * np.asarray(mnorm, np.float32)[fo]
    if qadd is not None:
        qcp = (qcp.astype(np.float32) + np.asarray(qadd, np.float32)[qid]).astype(np.float32)
    return qid, coff, ccnt, qcp.astype(np.float32), o


def params(K, nprobe, N, NC, BN=32, MSZ=3072, BETA=None, RHO=0.6, rho_override=None, M_override=None):
    """(M, n1, r) of throughput/enginei8.py:40-47,53."""
    M = M_override or MSZ or max(4096, 16 * K)
    beta, rho = (1.1, 0.75) if K <= 400 else (0.7, 0.5)
    if BETA:
        beta = BETA
    if RHO:
        rho = RHO
    if rho_override:
        beta, rho = 1.5, rho_override
    n1 = min(max(int(np.ceil(beta * K / (N / NC / BN + 1))), 1), nprobe)
    return M, n1, int(np.ceil(rho * K))


def recall(I, GT, k=10):
    I, GT = np.asarray(I), np.asarray(GT)
    return round(float(np.mean([len(set(I[i, :k].tolist()) & set(GT[i, :k].tolist())) / k for i in range(len(I))])), 4)


# ------------------------------------------------------------------------------------ C stages
def project(Q, Vr):
    Q = _c(Q, np.float32)
    Vr = _c(Vr, np.float32)
    B, d = Q.shape
    R = Vr.shape[1]
    z = np.empty((B, R), np.float32)
    lib().or_project(_p(Q), I64(B), I32(d), _p(Vr), I32(R), _p(z))
    return z


def query_prep(Q, Vr, c, z=None):
    """(q8, qs, qc, qh); z = Q @ Vr is computed here (sequential fp32) unless given (then Vr is unused)."""
    Q = _c(Q, np.float32)
    c = _c(c, np.float32)
    z = project(Q, Vr) if z is None else _c(z, np.float32)
    B, d = Q.shape
    R = z.shape[1]
    q8 = np.empty((B, R), np.int8)
    qs = np.empty(B, np.float32)
    qc = np.empty(B, np.float32)
    qh = np.empty((B, d), np.uint16)
    lib().or_query_prep(_p(Q), I64(B), I32(d), _p(z), I32(R), _p(c), _p(q8), _p(qs), _p(qc), _p(qh))
    return q8, qs, qc, qh


def build_codes(X16, order, cell, means16, Vr):
    X16 = _c(np.asarray(X16).view(np.uint16), np.uint16)
    means16 = _c(np.asarray(means16).view(np.uint16), np.uint16)
    order = _c(order, np.int32)
    cell = _c(cell, np.int32)
    Vr = _c(Vr, np.float32)
    N = len(order)
    d = X16.shape[1]
    R = Vr.shape[1]
    Z = np.empty((N, R), np.int8)
    zs = np.empty(N, np.float32)
    lib().or_build_codes(_p(X16), _p(order), _p(cell), I64(N), I32(d), _p(means16), _p(Vr), I32(R), _p(Z), _p(zs))
    return Z, zs


def fp16_gemm_nt(A16, Bt16):
    A16 = _c(np.asarray(A16).view(np.uint16), np.uint16)
    Bt16 = _c(np.asarray(Bt16).view(np.uint16), np.uint16)
    M, K = A16.shape
    Nn = Bt16.shape[0]
    out = np.empty((M, Nn), np.uint16)
    lib().or_fp16_gemm_nt(_p(A16), _p(Bt16), I64(M), I64(Nn), I32(K), _p(out))
    return out


def fp16_gemm_nn(A16, Bm16):
    A16 = _c(np.asarray(A16).view(np.uint16), np.uint16)
    Bm16 = _c(np.asarray(Bm16).view(np.uint16), np.uint16)
    M, K = A16.shape
    Nn = Bm16.shape[1]
    out = np.empty((M, Nn), np.uint16)
    lib().or_fp16_gemm_nn(_p(A16), _p(Bm16), I64(M), I64(Nn), I32(K), I32(Bm16.shape[1]), _p(out))
    return out


def route_topk(QM16, nprobe):
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    B, NC = QM16.shape
    probe = np.empty((B, nprobe), np.int32)
    lib().or_route_topk(_p(QM16), I64(B), I32(NC), I32(nprobe), _p(probe))
    return probe


def first_pass(q8, qs, probe, n1, off, Z, zs, QM16, mnorm, MB):
    q8 = _c(q8, np.int8)
    qs = _c(qs, np.float32)
    probe = _c(probe, np.int32)
    off = _c(off, np.int32)
    Z = _c(Z, np.int8)
    zs = _c(zs, np.float32)
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    B, npr = probe.shape
    NC = QM16.shape[1]
    mn = None if mnorm is None else _c(mnorm, np.float32)
    bm = np.full((B, n1, MB), -1e30, np.float32)
    lib().or_first_pass(_p(q8), _p(qs), _p(probe), I32(npr), I32(n1), _p(off), _p(Z), _p(zs), I32(Z.shape[1]),
                        _p(QM16), I32(NC), _p(mn) if mn is not None else None, I64(B), I32(MB), _p(bm))
    return bm


def threshold(bm, probe, off, n1, MB, r):
    bm = _c(bm, np.float32)
    probe = _c(probe, np.int32)
    off = _c(off, np.int32)
    B, npr = probe.shape
    t0 = np.empty(B, np.float32)
    lib().or_threshold(_p(bm), _p(probe), I32(npr), _p(off), I32(len(off) - 1), I64(B), I32(n1), I32(MB), I32(r),
                       _p(t0))
    return t0


def emit(q8, qs, probe, off, Z, zs, QM16, mnorm, t0, M):
    """(cnt, bval, bpos): every probed row with est >= t0, canonical order, first M kept."""
    q8 = _c(q8, np.int8)
    qs = _c(qs, np.float32)
    probe = _c(probe, np.int32)
    off = _c(off, np.int32)
    Z = _c(Z, np.int8)
    zs = _c(zs, np.float32)
    t0 = _c(t0, np.float32)
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    B, npr = probe.shape
    NC = QM16.shape[1]
    mn = None if mnorm is None else _c(mnorm, np.float32)
    cnt = np.empty(B, np.int32)
    bval = np.empty((B, M), np.float32)
    bpos = np.empty((B, M), np.int32)
    lib().or_emit(_p(q8), _p(qs), _p(probe), I32(npr), I32(npr), _p(off), _p(Z), _p(zs), I32(Z.shape[1]), _p(QM16),
                  I32(NC), _p(mn) if mn is not None else None, _p(t0), I64(B), I32(M), _p(cnt), _p(bval), _p(bpos))
    return cnt, bval, bpos


def select(bval, bpos, cnt, K, kd, delta):
    bval = _c(bval, np.float32)
    bpos = _c(bpos, np.int32)
    cnt = _c(cnt, np.int32)
    B, M = bval.shape
    pos = np.empty((B, K), np.int32)
    est1 = np.empty((B, K), np.float32)
    ok = np.empty(B, np.uint8)
    ncnt = np.empty(B, np.int32)
    lib().or_select(_p(bval), _p(bpos), _p(cnt), I64(B), I32(M), I32(K), I32(kd), F32(-1.0 if delta is None else delta),
                    _p(pos), _p(est1), _p(ok), _p(ncnt))
    return pos, est1, ok, ncnt


# ------------------------------------------------------------------------- routing-free dense scan
def quantize_rows(z):
    """(q int8 [n, R], scale f32 [n]) (throughput/brute.py:46-47, :51-52)."""
    z = _c(z, np.float32)
    n, R = z.shape
    q = np.empty((n, R), np.int8)
    a = np.empty(n, np.float32)
    lib().or_quantize_rows(_p(z), I64(n), I32(R), _p(q), _p(a))
    return q, a


def dense_scores(Q, qs, Z, zs16):
    """est f32 [B, N] = ((float)(Q @ Z.T) * qs[q]) * (float)zs16[n] (throughput/brute.py:16-17)."""
    Q, qs, Z = _c(Q, np.int8), _c(qs, np.float32), _c(Z, np.int8)
    zs16 = _c(np.asarray(zs16).view(np.uint16), np.uint16)
    B, R = Q.shape
    N = Z.shape[0]
    out = np.empty((B, N), np.float32)
    lib().or_dense_scores(_p(Q), _p(qs), I64(B), _p(Z), _p(zs16), I64(N), I32(R), _p(out))
    return out


def row_kth(S, r):
    """The r-th largest of each row of S (throughput/brute.py:59: topk(r).values[:, -1])."""
    S = np.asarray(S, np.float32)
    return np.sort(S, axis=1)[:, S.shape[1] - r].copy()


def dense_emit(Q, qs, Z, zs16, t0, M):
    """(cnt, bval, bpos): every (q, n) with est >= t0[q] (throughput/brute.py:31-37), canonical order, first M."""
    Q, qs, Z, t0 = _c(Q, np.int8), _c(qs, np.float32), _c(Z, np.int8), _c(t0, np.float32)
    zs16 = _c(np.asarray(zs16).view(np.uint16), np.uint16)
    B, R = Q.shape
    N = Z.shape[0]
    cnt = np.empty(B, np.int32)
    bval = np.empty((B, M), np.float32)
    bpos = np.empty((B, M), np.int32)
    lib().or_dense_emit(_p(Q), _p(qs), I64(B), _p(Z), _p(zs16), I64(N), I32(R), _p(t0), I32(M), _p(cnt), _p(bval),
                        _p(bpos))
    return cnt, bval, bpos


def brute_search(q, qs, Z, zs16, K, over=2.0, M=None, sidx=None, sample_every=20):
    """throughput/brute.py:56-63 on the CPU from the codes (q, qs) of the queries and (Z, zs16) of the stored
    rows: (pos, est, ok, cnt), pos and est in the canonical order (est descending, position ascending)."""
    N = len(Z)
    sidx = np.arange(0, N, sample_every) if sidx is None else np.asarray(sidx)
    zs16 = np.asarray(zs16).view(np.uint16)
    M = M or max(4096, 8 * K)
    r = max(1, int(round(over * K * (len(sidx) / N))))
    t0 = row_kth(dense_scores(q, qs, np.asarray(Z)[sidx], zs16[sidx]), r)
    cnt, bval, bpos = dense_emit(q, qs, Z, zs16, t0, M)
    pos, est, ok, _ = select(bval, bpos, cnt, K, 0, None)
    return pos, est, ok.astype(bool), cnt


def _tiers(TS):
    return np.asarray([[s, e, b] for s, e, b in TS], dtype=np.int32).reshape(-1)


def lut_build(Zq16, TS, half):
    Zq16 = _c(np.asarray(Zq16).view(np.uint16), np.uint16)
    B, D = Zq16.shape
    T = len(TS)
    L = np.empty((B, D // 4 * 16), np.uint16 if half else np.float32)
    qsum = np.empty((T, B), np.float32)
    qn2 = np.empty((T, B), np.float32)
    tiers = _tiers(TS)
    lib().or_lut_build(_p(Zq16), I64(B), I32(D), I32(T), _p(tiers), I32(int(half)), _p(L), _p(qsum), _p(qn2))
    return L, qsum, qn2


def lut_score(pos, qc, L, half, qsum, qn2, rec, soff, TS, deltas, toff, ncnt=None):
    pos = _c(pos, np.int32)
    qc = _c(qc, np.float32)
    L = _c(L, np.uint16 if half else np.float32)
    qsum = _c(qsum, np.float32)
    qn2 = _c(qn2, np.float32)
    rec = _c(rec, np.uint8)
    tiers = _tiers(TS)
    dl = _c(deltas, np.float32)
    to = _c(toff, np.int32)
    B, K = pos.shape
    est = np.empty((B, K), np.float32)
    sd = np.empty((B, K), np.float32)
    nc = None if ncnt is None else _c(ncnt, np.int32)
    lib().or_lut_score(_p(pos), _p(qc), _p(L), I32(int(half)), I32(L.shape[1]), _p(qsum), _p(qn2), _p(rec),
                       I32(rec.shape[1]), I32(soff), I32(len(TS)), _p(tiers), _p(dl), _p(to),
                       _p(nc) if nc is not None else None, I64(B), I32(K), _p(est), _p(sd))
    return est, sd


def refine(est, sd, pos, order, H16, Q, z, k):
    est = _c(est, np.float32)
    sd = _c(sd, np.float32)
    pos = _c(pos, np.int32)
    order = _c(order, np.int32)
    H16 = _c(np.asarray(H16).view(np.uint16), np.uint16)
    Q = _c(Q, np.float32)
    B, K = est.shape
    d = Q.shape[1]
    ids = np.empty((B, K), np.int32)
    I = np.empty((B, k), np.int32)
    scores = np.empty((B, k), np.float32)
    reads = np.empty(B, np.int32)
    lib().or_refine(_p(est), _p(sd), _p(pos), _p(order), _p(H16), _p(Q), I64(B), I32(K), I32(d), F32(z), I32(k),
                    _p(ids), _p(I), _p(scores), _p(reads))
    return ids, I, scores, reads


# ------------------------------------------------------------------------------------ whole path
def index_from_tables(s1, code, Z, zs, Vr, H):
    """Host copies (numpy) of the tables an EngineI8 searches, in the oracle's layout."""
    import torch

    t = lambda x: x.detach().cpu().numpy() if torch.is_tensor(x) else np.asarray(x)
    TS = code["TS"]
    meansN = (s1["means16"].float() * s1["inv_mnorm"][:, None]).half()
    mnorm = (1.0 / s1["inv_mnorm"]).float()
    return dict(order=t(s1["order"]).astype(np.int32), off=np.asarray(s1["off"]).astype(np.int32),
                meansN=t(meansN).view(np.uint16), mnorm=t(mnorm), c=t(s1["c"]).astype(np.float32),
                means16=t(s1["means16"]).view(np.uint16), inv_mnorm=t(s1["inv_mnorm"]).astype(np.float32),
                Vr=t(Vr).astype(np.float32), Z=t(Z), zs=t(zs), TS=list(TS),
                deltas=np.array([code["deltas"][b] for _, _, b in TS], np.float32),
                toff=np.array(code["toff"], np.int32), soff=int(code["soff"]), rec=t(code["rec"]),
                VP16=t(code["VP16"]).view(np.uint16), H=t(H).view(np.uint16))


def stage1(idx, q8, qs, QM16, probe, K, knobs, rho_override=None, M_override=None, delta=None, kd=9):
    N = idx["Z"].shape[0]
    NC = len(idx["off"]) - 1
    M, n1, r = params(K, probe.shape[1], N, NC, MSZ=knobs.get("MSZ", 3072), BETA=knobs.get("BETA"),
                      RHO=knobs.get("RHO", 0.6), rho_override=rho_override, M_override=M_override)
    MB = static_blocks(idx["off"])[4]
    # NROUTE scores against normalised means: pair constants scaled back by |m_c|; otherwise QM as is
    # (throughput/enginei8.py:47-48)
    mn = idx["mnorm"] if knobs.get("NROUTE", True) else None
    bm = first_pass(q8, qs, probe[:, :n1], n1, idx["off"], idx["Z"], idx["zs"], QM16, mn, MB)
    t0 = threshold(bm, probe, idx["off"], n1, MB, r)
    cnt, bval, bpos = emit(q8, qs, probe, idx["off"], idx["Z"], idx["zs"], QM16, mn, t0, M)
    pos, est1, ok, ncnt = select(bval, bpos, cnt, K, min(kd, K - 1), delta)
    return dict(n1=n1, r=r, M=M, MB=MB, bm=bm, t0=t0, cnt=cnt, bval=bval, bpos=bpos, pos=pos, est1=est1, ok=ok,
                ncnt=ncnt)


def route(idx, QM16, nprobe, knobs):
    """Probe lists of EngineI8's routing variants (throughput/enginei8.py:66-76): NROUTE ranks QM (normalised
    means) directly; otherwise the key is (float)QM * inv_mnorm, rounded to fp16 when ROUTE16; UNSORTED
    lists the chosen cells in cell order."""
    if knobs.get("NROUTE", True):
        probe = route_topk(QM16, nprobe)
    elif knobs.get("ROUTE16", True):
        with np.errstate(over="ignore"):  # keys beyond the fp16 range become +-inf, as the kernel rounds them
            keys = (np.asarray(QM16).view(np.float16).astype(np.float32) * idx["inv_mnorm"][None, :]).astype(np.float16)
        probe = route_topk(keys.view(np.uint16), nprobe)
    else:
        probe = route_topk_scaled(QM16, idx["inv_mnorm"], nprobe)
    if knobs.get("UNSORTED", False):
        probe = np.sort(probe, axis=1)
    return probe


def pipeline(idx, Q, K, z, nprobe, k, knobs=None, QM16=None, Zq16=None, zq=None, fallback=True, QMfb16=None):
    """Every intermediate of one batch (EngineI8._gpu + _fallback). zq (f32) is the projection, computed here
    in the library's order (one sequential fmaf chain per output) unless given; QM16 / Zq16 (fp16 as uint16)
    are the two BLAS products; when given (e.g. read back from the GPU) they are used as shared inputs,
    otherwise computed here with sequential fp32 accumulation."""
    knobs = dict(knobs or {})
    delta = knobs.get("DELTA", 0.07)
    half = knobs.get("LUTF", True) and knobs.get("LUTH", True)
    if zq is None:
        zq = project(Q, idx["Vr"])
    q8, qs, qc, qh = query_prep(Q, idx["Vr"], idx["c"], zq)
    D = idx["TS"][-1][1]
    nroute = knobs.get("NROUTE", True)
    if QM16 is None:
        QM16 = fp16_gemm_nt(qh, idx["meansN"] if nroute else idx["means16"])
    if Zq16 is None:
        Zq16 = fp16_gemm_nn(qh, np.ascontiguousarray(idx["VP16"][:, :D]))
    probe = route(idx, QM16, nprobe, knobs)
    s1 = stage1(idx, q8, qs, QM16, probe, K, knobs, delta=delta, kd=k - 1)
    L, qsum, qn2 = lut_build(Zq16, idx["TS"], half)
    pos, ncnt = s1["pos"], (s1["ncnt"] if delta is not None else None)
    K2 = knobs.get("K2")
    if K2 is not None and K2 < K:
        # progressive stage 2 (throughput/enginei8.py:82-85): the partial estimate over the first NT tiers
        # (score_lut(..., nt=self.NT), throughput/s2lut.py:92-93: TS[:nt] with the full tables, whose tier-t
        # rows of qsum/qn2 and table offsets are those of the full code) ranks the candidates
        nt = min(knobs.get("NT", 3), len(idx["TS"]))
        e_all, _ = lut_score(pos, qc, L, half, qsum[:nt], qn2[:nt], idx["rec"], idx["soff"], idx["TS"][:nt],
                             idx["deltas"][:nt], idx["toff"][:nt], None)
        pos = select(e_all, pos, np.full(len(pos), K, np.int32), K2, 0, None)[0]
        if ncnt is not None:
            ncnt = np.minimum(ncnt, K2).astype(np.int32)
    s1["pos2"] = pos
    est, sd = lut_score(pos, qc, L, half, qsum, qn2, idx["rec"], idx["soff"], idx["TS"], idx["deltas"],
                        idx["toff"], ncnt)
    ids, I, scores, reads = refine(est, sd, pos, idx["order"], idx["H"], Q, z, k)
    out = dict(z=zq, q8=q8, qs=qs, qc=qc, qh=qh, QM=QM16, Zq=Zq16, probe=probe, L=L, qsum=qsum, qn2=qn2, est=est, sd=sd,
               ids=ids, I=I.copy(), scores=scores.copy(), reads=reads.copy(), cand=ids.copy(), **s1)
    bad = np.nonzero(s1["ok"] == 0)[0]
    out["bad"] = bad
    if fallback and len(bad):
        # the reference's fallback routes on the plain QM with fp32 keys, sorted (throughput/enginei8.py:110-112)
        QMf = np.asarray(QM16 if QMfb16 is None else QMfb16)[bad]
        pf = route(idx, QMf, nprobe, dict(NROUTE=nroute, ROUTE16=False))
        f1 = stage1(idx, q8[bad], qs[bad], QMf, pf, K, knobs, rho_override=1.0, M_override=65536,
                    delta=None)
        Lf, qsf, qnf = lut_build(Zq16[bad], idx["TS"], False)
        estf, sdf = lut_score(f1["pos"], qc[bad], Lf, False, qsf, qnf, idx["rec"], idx["soff"], idx["TS"],
                              idx["deltas"], idx["toff"], None)
        idsf, If, scf, rf_ = refine(estf, sdf, f1["pos"], idx["order"], idx["H"], np.asarray(Q)[bad], z, k)
        out["I"][bad], out["scores"][bad], out["reads"][bad], out["cand"][bad] = If, scf, rf_, idsf
        out["fallback_ok"] = f1["ok"]
    return out


# ------------------------------------------------------------------------------------ trellis engine
def trellis_encode(Zs, nz, tab, L):
    """(words [n, W] uint32, scale1 [n] fp16 bits, paths [n, R] int32) of normalised rows (or_trellis_encode)."""
    Zs = _c(Zs, np.float32)
    nz = _c(nz, np.float32)
    tab = _c(tab, np.float32)
    n, R = Zs.shape
    W = (R + L - 1 + 31) // 32
    words = np.empty((n, W), np.uint32)
    scale1 = np.empty(n, np.uint16)
    paths = np.empty((n, R), np.int32)
    lib().or_trellis_encode(_p(Zs), _p(nz), I64(n), I32(R), _p(tab), I32(L), I32(W), _p(words), _p(scale1), _p(paths))
    return words, scale1, paths


def trellis_decode(words, R, L):
    words = _c(words, np.uint32)
    n, W = words.shape
    st = np.empty((n, R), np.int32)
    lib().or_trellis_decode(_p(words), I64(n), I32(W), I32(R), I32(L), _p(st))
    return st


def route_topk_scaled(QM16, scale, nprobe, qadd=None):
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    scale = _c(scale, np.float32)
    qa = None if qadd is None else _c(qadd, np.float32)
    B, NC = QM16.shape
    probe = np.empty((B, nprobe), np.int32)
    lib().or_route_topk_scaled(_p(QM16), _p(scale), _p(qa) if qa is not None else None, I64(B), I32(NC), I32(nprobe),
                               _p(probe))
    return probe


def tr_first_pass(Qr, probe, n1, off, words, scale1, tab, L, QM16, MB, qadd=None, half=False):
    Qr = _c(Qr, np.float32)
    probe = _c(probe, np.int32)
    off = _c(off, np.int32)
    words = _c(words, np.uint32)
    scale1 = _c(np.asarray(scale1).view(np.uint16), np.uint16)
    tab = _c(tab, np.float32)
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    B, npr = probe.shape
    bm = np.full((B, n1, MB), -1e30, np.float32)
    qa = None if qadd is None else _c(qadd, np.float32)
    lib().or_tr_first_pass(_p(Qr), _p(probe), I32(npr), I32(n1), _p(off), _p(words), I32(words.shape[1]), _p(scale1),
                           _p(tab), I32(L), I32(Qr.shape[1]), I32(int(bool(half))), _p(QM16), I32(QM16.shape[1]),
                           _p(qa) if qa is not None else None, I64(B), I32(MB), _p(bm))
    return bm


def tr_emit(Qr, probe, off, words, scale1, tab, L, QM16, t0, M, qadd=None, half=False):
    Qr = _c(Qr, np.float32)
    probe = _c(probe, np.int32)
    off = _c(off, np.int32)
    words = _c(words, np.uint32)
    scale1 = _c(np.asarray(scale1).view(np.uint16), np.uint16)
    tab = _c(tab, np.float32)
    QM16 = _c(np.asarray(QM16).view(np.uint16), np.uint16)
    t0 = _c(t0, np.float32)
    B, npr = probe.shape
    cnt = np.empty(B, np.int32)
    bval = np.empty((B, M), np.float32)
    bpos = np.empty((B, M), np.int32)
    qa = None if qadd is None else _c(qadd, np.float32)
    lib().or_tr_emit(_p(Qr), _p(probe), I32(npr), I32(npr), _p(off), _p(words), I32(words.shape[1]), _p(scale1), _p(tab),
                     I32(L), I32(Qr.shape[1]), I32(int(bool(half))), _p(QM16), I32(QM16.shape[1]),
                     _p(qa) if qa is not None else None, _p(t0),
                     I64(B), I32(M), _p(cnt), _p(bval), _p(bpos))
    return cnt, bval, bpos


def tiered_score(pos, qc, Zq, rec, soff, TS, toff, cb, ncnt=None):
    pos = _c(pos, np.int32)
    qc = _c(qc, np.float32)
    Zq = _c(Zq, np.float32)
    rec = _c(rec, np.uint8)
    cb = _c(cb, np.float32)
    tiers = _tiers(TS)
    to = _c(toff, np.int32)
    B, K = pos.shape
    est = np.empty((B, K), np.float32)
    sd = np.empty((B, K), np.float32)
    nc = None if ncnt is None else _c(ncnt, np.int32)
    lib().or_tiered_score(_p(pos), _p(qc), _p(Zq), I32(Zq.shape[1]), _p(rec), I32(rec.shape[1]), I32(soff), I32(len(TS)),
                          _p(tiers), _p(to), _p(cb), _p(nc) if nc is not None else None, I64(B), I32(K), _p(est), _p(sd))
    return est, sd


def trellis_index_from_tables(s1, code, H):
    """Host copies of the default engine's tables (fanarvse_paper_amd.trellis.build_index)."""
    import torch

    t = lambda x: x.detach().cpu().numpy() if torch.is_tensor(x) else np.asarray(x)
    return dict(order=t(s1["order"]).astype(np.int32), off=np.asarray(s1["off"]).astype(np.int32),
                inv_mnorm=t(s1["inv_mnorm"]).astype(np.float32), c=t(s1["c"]).astype(np.float32),
                W1=t(s1["W1"]).astype(np.float32), tab=t(s1["tab"]).astype(np.float32), L=int(s1["L"]),
                words=t(s1["words"]).view(np.uint32), scale1=t(s1["scale1"]).view(np.uint16),
                means16=t(s1["means16"]).view(np.uint16), TS=list(code["TS"]), toff=np.array(code["toff"], np.int32),
                soff=int(code["soff"]), rec=t(code["rec"]), cb=t(code["cb"]).astype(np.float32), H=t(H).view(np.uint16))


def tr_params(K, nprobe, N, NC, M=None, rho_override=None, M_override=None, BN=32):
    """(M, n1, r) of search_static (src/s1cell.py:176-190) with the reference's (beta, rho) by K
    (src/engine_cell.py:78) and the fallback's (1.5, 1.0)."""
    M = M_override or M or max(4096, 16 * K)
    beta, rho = (1.1, 0.75) if K <= 400 else (0.7, 0.5)
    if rho_override:
        beta, rho = 1.5, rho_override
    n1 = min(max(int(np.ceil(beta * K / (N / NC / BN + 1))), 1), nprobe)
    return M, n1, int(np.ceil(rho * K))


def tr_stage1(idx, Qr, QM16, probe, K, M=None, rho_override=None, M_override=None, qadd=None, half=False):
    N = idx["words"].shape[0]
    NC = len(idx["off"]) - 1
    M, n1, r = tr_params(K, probe.shape[1], N, NC, M, rho_override, M_override)
    MB = static_blocks(idx["off"])[4]
    bm = tr_first_pass(Qr, probe[:, :n1], n1, idx["off"], idx["words"], idx["scale1"], idx["tab"], idx["L"], QM16, MB,
                       qadd, half)
    t0 = threshold(bm, probe, idx["off"], n1, MB, r)
    cnt, bval, bpos = tr_emit(Qr, probe, idx["off"], idx["words"], idx["scale1"], idx["tab"], idx["L"], QM16, t0, M,
                              qadd, half)
    pos, est1, ok, ncnt = select(bval, bpos, cnt, K, 0, None)
    return dict(n1=n1, r=r, M=M, MB=MB, bm=bm, t0=t0, cnt=cnt, bval=bval, bpos=bpos, pos=pos, est1=est1, ok=ok)


def tr_pipeline(idx, Q, K, z, nprobe, k, Qr, QM16, Zq, M=None, fallback=True, proj=False, order=True, half=None,
                fb_half=True, fb_rho=1.0, fb_M=65536):
    """The default engine's batch (EngineS._gpu + the fallback): Qr = Q @ W1 (f32), QM16 = fp16(Q) @ means16.T
    (fp16), Zq = Q @ VP (f32) are the shared dense products. proj: QM16 = fp16(Qr) @ meansR.T and the pair term
    and routing key add <q, c> (host_resident/space_x.py:33-39). order=False: ids are sorted positions.
    half: fp16 stage-1 operands (None: the reference's choice by batch size, fp16 above 8 queries,
    src/engine_cell.py:48-53,82-83); fb_half: the same for the fallback pass. fb_rho / fb_M: the fallback's
    rho and buffer, (1.0, 65536) for EngineS; the host-resident engine reruns its flagged queries with the
    main pass's rho and a 1 << 20 buffer (fb_rho=None, fb_M=1 << 20: host_resident/space_x.py:63-70)."""
    Q = _c(Q, np.float32)
    _, _, qc, _ = query_prep(Q, None, idx["c"], Qr)
    qadd = qc if proj else None
    probe = route_topk_scaled(QM16, idx["inv_mnorm"], nprobe, qadd)
    if half is None:
        half = len(Q) > 8
    s1 = tr_stage1(idx, Qr, QM16, probe, K, M, qadd=qadd, half=half)
    est, sd = tiered_score(s1["pos"], qc, Zq, idx["rec"], idx["soff"], idx["TS"], idx["toff"], idx["cb"])
    ordr = idx["order"] if order else np.arange(len(idx["order"]), dtype=np.int32)
    H = idx["H"] if order else idx["Hs"]
    ids, I, scores, reads = refine(est, sd, s1["pos"], ordr, H, Q, z, k)
    out = dict(qc=qc, probe=probe, est=est, sd=sd, ids=ids, I=I.copy(), scores=scores.copy(), reads=reads.copy(),
               cand=ids.copy(), **s1)
    bad = np.nonzero(s1["ok"] == 0)[0]
    out["bad"] = bad
    if fallback and len(bad):
        f1 = tr_stage1(idx, np.asarray(Qr)[bad], np.asarray(QM16)[bad], probe[bad], K, M, rho_override=fb_rho,
                       M_override=fb_M, qadd=None if qadd is None else qadd[bad], half=fb_half)
        estf, sdf = tiered_score(f1["pos"], qc[bad], np.asarray(Zq)[bad], idx["rec"], idx["soff"], idx["TS"],
                                 idx["toff"], idx["cb"])
        idsf, If, scf, rf_ = refine(estf, sdf, f1["pos"], ordr, H, Q[bad], z, k)
        out["I"][bad], out["scores"][bad], out["reads"][bad], out["cand"][bad] = If, scf, rf_, idsf
        out["fallback_ok"] = f1["ok"]
    return out
