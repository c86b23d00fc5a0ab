"""ctypes binding of libfvs.so (include/fvs.h) with host-side shape checks.

Every wrapper takes torch tensors, checks device, dtype, contiguity and shapes before anything is
launched, passes raw pointers plus torch's current stream, and raises RuntimeError on a non-zero
return code. There is no fallback: if libfvs.so is missing or a tensor is not on the GPU, the call
fails.
"""
import ctypes
import os

import numpy as np
import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfvs.so")

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float
U32 = ctypes.c_uint32

# name -> argument types (return type is int for all but fvs_error_string)
SIGNATURES = {
    "fvs_abi_version": [],
    "fvs_error_string": [ctypes.c_int],
    "fvs_fill_u32": [P, I64, U32, P],
    "fvs_calib_mfma": [I32, I32, P, P],
    "fvs_pack_ids": [P, P, I64, I32, P, P],
    "fvs_dense_small": [P, I64, I32, P, I32, P, P, I32, P, P, I32, P, P, P, P],
    "fvs_query_prep": [P, I64, I32, P, I32, P, P, P, P, P, P],
    "fvs_query_code": [P, I64, I32, P, I32, P, P, P, P, P, P, P],
    "fvs_build_codes": [P, P, P, I64, I32, P, P, I32, P, P, P],
    "fvs_route_topk": [P, I64, I32, I32, P, P],
    "fvs_pairs_scratch_bytes": [I64, I32],
    "fvs_pairs_noalloc": [P, I64, I32, I32, I32, P, P, P, P, P, P, P, P, P],
    "fvs_pairs2": [P, I64, I32, I32, I32, P, P, P, P, I64] + [P] * 10 + [P],
    "fvs_pairs": [P, I64, I32, I32, I32, P, P, P, P, P, P, I64, P, P, P, P],
    "fvs_i8_scan_civf8": [I32, I32] + [P] * 17 + [I32, I32, P],
    "fvs_quantize_i8": [P, I64, I32, P, P, P, P],
    "fvs_route_keys": [P, P, P, I64, I32, P, P],
    "fvs_dense_pack": [P, I64, I32, I64, I32, P, P],
    "fvs_dense_threshold": [P, I64, I32, I32, P, P, P],
    "fvs_dense_scan": [I32, P, P, I64, I64, P, P, I64, I64, I32, P, P, P, P, I32, P, P],
    "fvs_i8_scan": [I32, I32, P, P, P, P, P, P, P, P, P, P, P, P, I64, I32, P, P, P, P, P, P, I32, I32, I32, P],
    "fvs_threshold": [P, P, I32, P, I32, I64, I32, I32, I32, P, P, P],
    "fvs_select": [P, P, P, I64, I32, I32, I32, F32, P, P, P, P, P],
    "fvs_lut_build": [P, I64, I32, I32, P, I32, P, P, P, P],
    "fvs_lut_score": [P, P, P, I32, I32, P, P, P, I64, I32, I32, I32, P, P, P, I32, P, I64, I32, P, P, P],
    "fvs_lut_score_zq": [P, P, P, I32, I32, P, I64, I32, I32, I32, P, P, P, I32, P, I64, I32, P, P, P],
    "fvs_refine": [P, P, P, P, P, P, I64, I32, I32, F32, I32, P, P, P, P, P],
    "fvs_classify": [P, P, P, P, I64, I32, F32, I32, P, P, P, P, P],
    "fvs_refine_rows": [P, P, P, P, P, P, P, P, I64, I32, I32, I32, P, P, P, P],
    "fvs_trellis_encode": [P, P, I64, I32, P, I32, P, I32, P, P, P],
    "fvs_tr_scan": [I32, I32, P, P, P, P, P, P, P, P, P, P, I64, I32, P, P, I32, I32, I32, P, P, P, P, P, P, I32, I32, I32,
                    I32, P],
    "fvs_tr_scan_streamed": [I32, I32, P, P, P, P, I64, P, P, P, P, P, P, P, P, P, P, I32, P, I32, I32, I32, P, P, P,
                             P, P, P, I32, I32, I32, I32, P],
    "fvs_route_topk_scaled": [P, P, P, I64, I32, I32, P, P],
    "fvs_tiered_score": [P, P, P, I32, P, I64, I32, I32, I32, P, P, P, P, I64, I32, P, P, P],
}

_lib = None


def lib():
    """Load libfvs.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                               "(or python fanarvse_paper_amd/build.py)")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = {"fvs_error_string": ctypes.c_char_p, "fvs_pairs_scratch_bytes": ctypes.c_int64}.get(
                name, ctypes.c_int)
        if L.fvs_abi_version() != 2:
            raise RuntimeError("libfvs.so ABI version mismatch")
        _lib = L
    return _lib


def _check(rc, name):
    if rc != 0:
        msg = lib().fvs_error_string(rc).decode()
        raise RuntimeError(f"{name} failed: {msg} (code {rc})")


def _stream():
    return P(torch.cuda.current_stream().cuda_stream)


def _dev(t, dtype, name, shape=None, host_ok=False):
    """Pointer of a contiguous tensor of the given dtype on the GPU (or pinned host if host_ok)."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    if not t.is_cuda and not (host_ok and t.is_pinned()):
        raise ValueError(f"{name}: tensor must be on the GPU" + (" or in pinned host memory" if host_ok else ""))
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    return P(t.data_ptr())


def _opt(t, dtype, name, shape=None):
    return P(None) if t is None else _dev(t, dtype, name, shape)


def _empty(shape, dtype, device):
    return torch.empty(shape, dtype=dtype, device=device)


# ------------------------------------------------------------------------------------------- ops
def fill_u32(t, value):
    if t.element_size() != 4:
        raise TypeError("fill_u32: 32-bit tensor expected")
    _check(lib().fvs_fill_u32(_dev(t, t.dtype, "dst"), t.numel(), U32(value), _stream()), "fvs_fill_u32")


def calib_mfma(out, iters):
    """The matrix-core calibration kernel: len(out) / 4 workgroups, `iters` rounds of sixteen MFMAs (four 4-step
    chains) per wave (2 * 16 * 16 * 16 * 64 int8 ops per wave and round); out int32 [4 * workgroups] receives the
    checksums."""
    if out.numel() % 4 != 0:
        raise ValueError("calib_mfma: out holds four checksums per workgroup")
    _check(lib().fvs_calib_mfma(out.numel() // 4, iters, _dev(out, torch.int32, "out"), _stream()), "fvs_calib_mfma")


def pack_ids(ok, I, out):
    """out int64 [B, k+1] = [ok | I] in one launch; out may be a pinned host tensor, written directly."""
    B, k = I.shape
    _check(lib().fvs_pack_ids(_dev(ok.view(torch.uint8), torch.uint8, "ok", (B,)), _dev(I, torch.int32, "I"), B, k,
                              _dev(out, torch.int64, "out", (B, k + 1), host_ok=True), _stream()), "fvs_pack_ids")
    return out


DENSE_MAX_B = 8


def dense_small(Q, W1T, M16, VPT, c):
    """(Qr f32 [B, R], QM fp16 [B, NC], Zq f32 [B, D], qc f32 [B]) = (Q @ W1T.T, fp16(fp16(Q) @ M16.T), Q @ VPT.T,
    query_prep's <Q, c>) in one launch, for B <= DENSE_MAX_B (the default engine's small-batch products)."""
    B, d = Q.shape
    R, NC, D = W1T.shape[0], M16.shape[0], VPT.shape[0]
    if B > DENSE_MAX_B or W1T.shape[1] != d or M16.shape[1] != d or VPT.shape[1] != d:
        raise ValueError("dense_small: shapes")
    Qr = _empty((B, R), torch.float32, Q.device)
    QM = _empty((B, NC), torch.float16, Q.device)
    Zq = _empty((B, D), torch.float32, Q.device)
    qc = _empty((B,), torch.float32, Q.device)
    _check(lib().fvs_dense_small(_dev(Q, torch.float32, "Q"), B, d, _dev(W1T, torch.float32, "W1T"), R,
                                 _dev(Qr, torch.float32, "Qr"), _dev(M16, torch.float16, "M16"), NC,
                                 _dev(QM, torch.float16, "QM"), _dev(VPT, torch.float32, "VPT"), D,
                                 _dev(Zq, torch.float32, "Zq"), _dev(c, torch.float32, "c", (d,)),
                                 _dev(qc, torch.float32, "qc"), _stream()), "fvs_dense_small")
    return Qr, QM, Zq, qc


def query_prep(Q, Vr, c, z=None, canonical=False):
    """q8 [B,R] int8, qs [B], qc [B], qh [B,d] fp16 and the projection z [B,R] (throughput/enginei8.py:38, :62).
    z = Q @ Vr is the fp32 BLAS product, as in the reference, unless given (rows of an earlier projection, or
    another engine's product); the code, centre term and fp16 copy are derived from it in one launch. With
    canonical=True (and no z) one launch computes everything, z as a sequential fp32 fmaf chain over d (the
    index build's order, which the oracle reproduces bit for bit)."""
    B, d = Q.shape
    R = z.shape[1] if z is not None else Vr.shape[1]
    dev = Q.device
    q8 = _empty((B, R), torch.int8, dev)
    qs = _empty((B,), torch.float32, dev)
    qc = _empty((B,), torch.float32, dev)
    qh = _empty((B, d), torch.float16, dev)
    if z is None and not canonical:
        z = Q @ Vr
    if z is None:
        z = _empty((B, R), torch.float32, dev)
        _check(lib().fvs_query_code(_dev(Q, torch.float32, "Q"), B, d, _dev(Vr, torch.float32, "Vr", (d, R)), R,
                                    _dev(c, torch.float32, "c", (d,)), _dev(z, torch.float32, "z"),
                                    _dev(q8, torch.int8, "q8"), _dev(qs, torch.float32, "qs"),
                                    _dev(qc, torch.float32, "qc"), _dev(qh, torch.float16, "qh"), _stream()),
               "fvs_query_code")
        return q8, qs, qc, qh, z
    z = z.contiguous()
    _check(lib().fvs_query_prep(_dev(Q, torch.float32, "Q"), B, d, _dev(z, torch.float32, "z", (B, R)), R,
                                _dev(c, torch.float32, "c", (d,)), _dev(q8, torch.int8, "q8"), _dev(qs, torch.float32, "qs"),
                                _dev(qc, torch.float32, "qc"), _dev(qh, torch.float16, "qh"), _stream()),
           "fvs_query_prep")
    return q8, qs, qc, qh, z


def build_codes(X16, order, cell, means16, Vr):
    """Z [N,R] int8 and zs [N] of the cell residuals in sorted order (throughput/enginei8.py:19-27)."""
    N = order.shape[0]
    d = X16.shape[1]
    NC = means16.shape[0]
    R = Vr.shape[1]
    if int(order.max()) >= X16.shape[0] or int(order.min()) < 0:
        raise ValueError("build_codes: order out of range")
    if int(cell.max()) >= NC or int(cell.min()) < 0:
        raise ValueError("build_codes: cell out of range")
    Z = _empty((N, R), torch.int8, X16.device)
    zs = _empty((N,), torch.float32, X16.device)
    _check(lib().fvs_build_codes(_dev(X16, torch.float16, "X16"), _dev(order, torch.int32, "order", (N,)),
                                 _dev(cell, torch.int32, "cell", (N,)), N, d,
                                 _dev(means16, torch.float16, "means16", (NC, d)), _dev(Vr, torch.float32, "Vr", (d, R)),
                                 R, _dev(Z, torch.int8, "Z"), _dev(zs, torch.float32, "zs"), _stream()),
           "fvs_build_codes")
    return Z, zs


def route_topk(QM, nprobe):
    B, NC = QM.shape
    probe = _empty((B, nprobe), torch.int32, QM.device)
    _check(lib().fvs_route_topk(_dev(QM, torch.float16, "QM"), B, NC, nprobe, _dev(probe, torch.int32, "probe"),
                                _stream()), "fvs_route_topk")
    return probe


def pairs_scratch(B, NC, device):
    """Scratch buffer for pairs() (a cell-major probe-rank matrix); reusable across calls on a stream."""
    nbytes = lib().fvs_pairs_scratch_bytes(B, NC)
    return torch.empty((nbytes,), dtype=torch.uint8, device=device)


def pairs(probe, n, NC, QM, mnorm, scratch=None, qadd=None):
    """(qid, qrank, coff, ccnt, qcp) of the first n probe columns (throughput/enginei8.py:11-16)."""
    B, npr = probe.shape
    dev = probe.device
    if QM.shape != (B, NC):
        raise ValueError("pairs: QM shape")
    if scratch is None:
        scratch = pairs_scratch(B, NC, dev)
    ccnt = _empty((NC,), torch.int32, dev)
    coff = _empty((NC,), torch.int32, dev)
    qid = _empty((B * n,), torch.int32, dev)
    qrank = _empty((B * n,), torch.int32, dev)
    qcp = _empty((B * n,), torch.float32, dev)
    _check(lib().fvs_pairs(_dev(probe, torch.int32, "probe"), B, npr, n, NC, _dev(QM, torch.float16, "QM"),
                           _opt(mnorm, torch.float32, "mnorm", (NC,)), _opt(qadd, torch.float32, "qadd", (B,)),
                           _dev(ccnt, torch.int32, "ccnt"),
                           _dev(coff, torch.int32, "coff"), _dev(scratch, torch.uint8, "scratch"), scratch.numel(),
                           _dev(qid, torch.int32, "qid"), _dev(qrank, torch.int32, "qrank"),
                           _dev(qcp, torch.float32, "qcp"), _stream()), "fvs_pairs")
    return qid, qrank, coff, ccnt, qcp


def pairs_noalloc(probe, n, NC, QM, mnorm, out, qadd=None):
    """pairs() through fvs_pairs_noalloc: the library's static scratch instead of a caller buffer, and the
    caller's output tensors out = (qid [B*n], qrank [B*n], coff [NC], ccnt [NC], qcp [B*n]); nothing is
    allocated on the device by this call."""
    B, npr = probe.shape
    if QM.shape != (B, NC):
        raise ValueError("pairs_noalloc: QM shape")
    qid, qrank, coff, ccnt, qcp = out
    _check(lib().fvs_pairs_noalloc(_dev(probe, torch.int32, "probe"), B, npr, n, NC, _dev(QM, torch.float16, "QM"),
                                   _opt(mnorm, torch.float32, "mnorm", (NC,)), _opt(qadd, torch.float32, "qadd", (B,)),
                                   _dev(ccnt, torch.int32, "ccnt", (NC,)), _dev(coff, torch.int32, "coff", (NC,)),
                                   _dev(qid, torch.int32, "qid", (B * n,)), _dev(qrank, torch.int32, "qrank", (B * n,)),
                                   _dev(qcp, torch.float32, "qcp", (B * n,)), _stream()), "fvs_pairs_noalloc")
    return out


def pairs2(probe, n1, NC, QM, mnorm, scratch=None, qadd=None):
    """The first-pass pairs (first n1 probe columns) and the emit pairs (all columns) of one batch, each as
    pairs() returns them, from one pass (throughput/enginei8.py:48,55)."""
    B, npr = probe.shape
    dev = probe.device
    if QM.shape != (B, NC):
        raise ValueError("pairs2: QM shape")
    if scratch is None:
        scratch = pairs_scratch(B, NC, dev)
    out = []
    for n in (n1, npr):
        out.append(dict(ccnt=_empty((NC,), torch.int32, dev), coff=_empty((NC,), torch.int32, dev),
                        qid=_empty((B * n,), torch.int32, dev), qrank=_empty((B * n,), torch.int32, dev),
                        qcp=_empty((B * n,), torch.float32, dev)))
    args = []
    for o in out:
        args += [_dev(o["ccnt"], torch.int32, "ccnt"), _dev(o["coff"], torch.int32, "coff"),
                 _dev(o["qid"], torch.int32, "qid"), _dev(o["qrank"], torch.int32, "qrank"),
                 _dev(o["qcp"], torch.float32, "qcp")]
    _check(lib().fvs_pairs2(_dev(probe, torch.int32, "probe"), B, npr, n1, NC, _dev(QM, torch.float16, "QM"),
                            _opt(mnorm, torch.float32, "mnorm", (NC,)), _opt(qadd, torch.float32, "qadd", (B,)),
                            _dev(scratch, torch.uint8, "scratch"), scratch.numel(), *args, _stream()), "fvs_pairs2")
    return tuple((o["qid"], o["qrank"], o["coff"], o["ccnt"], o["qcp"]) for o in out)


def i8_scan(mode, blocks, q8, qs, pr, Z, zs, t0=None, cnt=None, bval=None, bpos=None, bm=None, CAP=1, MB=1, n1=1):
    """First pass (mode 0) or emit (mode 1) over the stage-1 work items (throughput/civf8.py:89-91).

    `blocks` = (cell, first row, cell start, cell end): index.static_chunks(off, 32, 4) for mode 0 (items of four
    global 32-row blocks), items of at most 128 rows for mode 1 (index.row_chunks(off, 128), or static_chunks with
    CB = 4), over the same index as Z (its rows lie
    inside Z); no host synchronisation happens here, so the call can be captured in a graph."""
    pcell, prow, ps, pe = blocks
    qid, qrank, coff, ccnt, qcp = pr
    P_ = pcell.shape[0]
    N, R = Z.shape
    if q8.shape[1] != R:
        raise ValueError("i8_scan: code width mismatch")
    B = q8.shape[0]
    if mode == 0 and (bm is None or bm.numel() != B * n1 * MB):
        raise ValueError("i8_scan: bm must hold B*n1*MB values")
    if mode == 1 and (bval is None or bval.shape != (B, CAP) or bpos.shape != (B, CAP) or cnt.shape != (B,)):
        raise ValueError("i8_scan: emit buffers must be [B, CAP]")
    f32, i32 = torch.float32, torch.int32
    _check(lib().fvs_i8_scan(mode, P_, _dev(q8, torch.int8, "q8"), _dev(qs, f32, "qs", (B,)), _dev(qid, i32, "qid"),
                             _dev(qrank, i32, "qrank"), _dev(coff, i32, "coff"), _dev(ccnt, i32, "ccnt"),
                             _dev(pcell, i32, "pcell"), _dev(prow, i32, "prow"), _dev(ps, i32, "ps"),
                             _dev(pe, i32, "pe"), _dev(Z, torch.int8, "Z"), _dev(zs, f32, "zs", (N,)), N, R,
                             _dev(qcp, f32, "qcp"), _opt(t0, f32, "t0"), _opt(cnt, i32, "cnt"),
                             _opt(bval, f32, "bval"), _opt(bpos, i32, "bpos"), _opt(bm, f32, "bm"), CAP, MB, n1,
                             _stream()), "fvs_i8_scan")


def threshold(bm, probe, off, n1, MB, r, cnt=None):
    """t0 [B] from the first-pass block maxima; with cnt, also zeroes the emit pass's counters."""
    B, npr = probe.shape
    t0 = _empty((B,), torch.float32, probe.device)
    if off.dim() != 1 or off.numel() < 2:
        raise ValueError("threshold: off must hold NC + 1 cell offsets")
    _check(lib().fvs_threshold(_dev(bm, torch.float32, "bm"), _dev(probe, torch.int32, "probe"), npr,
                               _dev(off, torch.int32, "off"), off.numel() - 1, B, n1, MB, r, _dev(t0, torch.float32, "t0"),
                               _opt(cnt, torch.int32, "cnt", (B,)), _stream()), "fvs_threshold")
    return t0


def select(bval, bpos, cnt, K, kd, delta):
    B, M = bval.shape
    dev = bval.device
    pos = _empty((B, K), torch.int32, dev)
    est1 = _empty((B, K), torch.float32, dev)
    ok = _empty((B,), torch.uint8, dev)
    ncnt = _empty((B,), torch.int32, dev)
    _check(lib().fvs_select(_dev(bval, torch.float32, "bval"), _dev(bpos, torch.int32, "bpos", (B, M)),
                            _dev(cnt, torch.int32, "cnt", (B,)), B, M, K, kd, F32(-1.0 if delta is None else delta),
                            _dev(pos, torch.int32, "pos"), _dev(est1, torch.float32, "est1"),
                            _dev(ok, torch.uint8, "ok"), _dev(ncnt, torch.int32, "ncnt"), _stream()), "fvs_select")
    return pos, est1, ok, ncnt


def _tiers_arr(TS):
    arr = (ctypes.c_int32 * (3 * len(TS)))()
    for t, (s, e, b) in enumerate(TS):
        arr[3 * t], arr[3 * t + 1], arr[3 * t + 2] = int(s), int(e), int(b)
    return arr


def lut_build(Zq, TS, half):
    """L [B, D/4*16] (fp16 if half), qsum, qn2 [T, B] (throughput/s2lut.py:118-126)."""
    B, D = Zq.shape
    dev = Zq.device
    L = _empty((B, D // 4 * 16), torch.float16 if half else torch.float32, dev)
    qsum = _empty((len(TS), B), torch.float32, dev)
    qn2 = _empty((len(TS), B), torch.float32, dev)
    _check(lib().fvs_lut_build(_dev(Zq, torch.float16, "Zq"), B, D, len(TS), _tiers_arr(TS), int(bool(half)),
                               _dev(L, L.dtype, "L"), _dev(qsum, torch.float32, "qsum"),
                               _dev(qn2, torch.float32, "qn2"), _stream()), "fvs_lut_build")
    return L, qsum, qn2


class ZqTables:
    """Stand-in for lut_build's (L, qsum, qn2): the rotated queries Zq, from which fvs_lut_score_zq forms the
    same tables inside the scoring kernel (no table in memory, no build launch)."""

    def __init__(self, Zq, half):
        self.Zq, self.half = Zq, bool(half)


def lut_score(pos, qc, pre, code, ncnt=None, nt=None):
    """(est, sd) [B, K] of the candidates (throughput/s2lut.py:92-106), from the packed records; nt: the
    partial estimate over the first nt tiers (score_lut(..., nt=...), throughput/s2lut.py:92-93). `pre` is
    lut_build's (L, qsum, qn2) or a ZqTables (the same results, tables built inside the scorer)."""
    B, K = pos.shape
    TS = code["TS"]
    T = len(TS)
    rec = code["rec"]
    N, RB = rec.shape
    deltas = (ctypes.c_float * T)(*[float(code["deltas"][b]) for _, _, b in TS])
    toff = (ctypes.c_int32 * T)(*[int(x) for x in code["toff"]])
    est = _empty((B, K), torch.float32, pos.device)
    sd = _empty((B, K), torch.float32, pos.device)
    if isinstance(pre, ZqTables):
        Zq = pre.Zq
        if Zq.dim() != 2 or Zq.shape[0] != B:
            raise ValueError("lut_score: Zq must be [B, D]")
        _check(lib().fvs_lut_score_zq(_dev(pos, torch.int32, "pos"), _dev(qc, torch.float32, "qc", (B,)),
                                      _dev(Zq, torch.float16, "Zq"), Zq.shape[1], int(pre.half),
                                      _dev(rec, torch.uint8, "rec"), N, RB, int(code["soff"]), T, _tiers_arr(TS), deltas,
                                      toff, int(nt or 0), _opt(ncnt, torch.int32, "ncnt", (B,)), B, K,
                                      _dev(est, torch.float32, "est"), _dev(sd, torch.float32, "sd"), _stream()),
               "fvs_lut_score_zq")
        return est, sd
    L, qsum, qn2 = pre
    half = L.dtype == torch.float16
    _check(lib().fvs_lut_score(_dev(pos, torch.int32, "pos"), _dev(qc, torch.float32, "qc", (B,)),
                               _dev(L, L.dtype, "L"), int(half), L.shape[1], _dev(qsum, torch.float32, "qsum", (T, B)),
                               _dev(qn2, torch.float32, "qn2", (T, B)), _dev(rec, torch.uint8, "rec"), N, RB,
                               int(code["soff"]), T, _tiers_arr(TS), deltas, toff, int(nt or 0),
                               _opt(ncnt, torch.int32, "ncnt", (B,)), B, K, _dev(est, torch.float32, "est"),
                               _dev(sd, torch.float32, "sd"), _stream()), "fvs_lut_score")
    return est, sd


def refine(est, sd, pos, order, H, Q, z, k):
    """(ids [B,K], I [B,k], scores [B,k], reads [B]) (throughput/enginei8.py:92-95, src/stage3_zc.py)."""
    B, K = est.shape
    d = Q.shape[1]
    if H.shape[1] != d:
        raise ValueError("refine: H width")
    dev = est.device
    ids = _empty((B, K), torch.int32, dev)
    I = _empty((B, k), torch.int32, dev)
    scores = _empty((B, k), torch.float32, dev)
    reads = _empty((B,), torch.int32, dev)
    _check(lib().fvs_refine(_dev(est, torch.float32, "est"), _dev(sd, torch.float32, "sd", (B, K)),
                            _dev(pos, torch.int32, "pos", (B, K)), _opt(order, torch.int32, "order"),
                            _dev(H, torch.float16, "H", host_ok=True), _dev(Q, torch.float32, "Q", (B, d)), B, K, d,
                            F32(z), k, _dev(ids, torch.int32, "ids"), _dev(I, torch.int32, "I"),
                            _dev(scores, torch.float32, "scores"), _dev(reads, torch.int32, "reads"), _stream()),
           "fvs_refine")
    return ids, I, scores, reads


def classify(est, sd, pos, order, z, k):
    """(ids [B,K], flag u8 [B,K], namb [B], aslot [B,K]): the first half of refine for rows read by the
    host (src/engine3.py:204-216): flags 1 sure / 2 ambiguous, ambiguous slots in ascending order
    (entries of aslot past namb are 0)."""
    B, K = est.shape
    dev = est.device
    ids = _empty((B, K), torch.int32, dev)
    flag = _empty((B, K), torch.uint8, dev)
    namb = _empty((B,), torch.int32, dev)
    aslot = torch.zeros((B, K), dtype=torch.int32, device=dev)  # entries past namb stay 0 (a valid slot)
    _check(lib().fvs_classify(_dev(est, torch.float32, "est"), _dev(sd, torch.float32, "sd", (B, K)),
                              _dev(pos, torch.int32, "pos", (B, K)), _opt(order, torch.int32, "order"), B, K, F32(z), k,
                              _dev(ids, torch.int32, "ids"), _dev(flag, torch.uint8, "flag"),
                              _dev(namb, torch.int32, "namb"), _dev(aslot, torch.int32, "aslot"), _stream()),
           "fvs_classify")
    return ids, flag, namb, aslot


def refine_rows(est, flag, aslot, namb, roff, ids, rows, Q, k):
    """(I [B,k], scores [B,k], reads [B]): the second half (src/engine3.py:218-223): exact scores of the
    ambiguous slots from rows [sum namb, d] fp16 (device or pinned host), query q's at roff[q] + j."""
    B, K = est.shape
    d = Q.shape[1]
    if rows.dim() != 2 or rows.shape[1] != d:
        raise ValueError("refine_rows: rows width")
    dev = est.device
    I = _empty((B, k), torch.int32, dev)
    scores = _empty((B, k), torch.float32, dev)
    reads = _empty((B,), torch.int32, dev)
    _check(lib().fvs_refine_rows(_dev(est, torch.float32, "est"), _dev(flag, torch.uint8, "flag", (B, K)),
                                 _dev(aslot, torch.int32, "aslot", (B, K)), _dev(namb, torch.int32, "namb", (B,)),
                                 _dev(roff, torch.int64, "roff", (B,)), _dev(ids, torch.int32, "ids", (B, K)),
                                 _dev(rows, torch.float16, "rows", host_ok=True), _dev(Q, torch.float32, "Q", (B, d)),
                                 B, K, d, k, _dev(I, torch.int32, "I"), _dev(scores, torch.float32, "scores"),
                                 _dev(reads, torch.int32, "reads"), _stream()), "fvs_refine_rows")
    return I, scores, reads


# ------------------------------------------------------------------------------ trellis engine
def trellis_encode(Zs, nz, tab, L, words, scale1, paths=None):
    """Viterbi paths of normalised rows Zs [n, R] (f32) through the 2^L-state trellis with table tab, packed
    into words [n, W] (int32 bit patterns) and scale1 [n] fp16 (src/viterbi_fused.py, engine_cell.py:16-22)."""
    n, R = Zs.shape
    W = words.shape[1]
    _check(lib().fvs_trellis_encode(_dev(Zs, torch.float32, "Zs"), _dev(nz, torch.float32, "nz", (n,)), n, R,
                                    _dev(tab, torch.float32, "tab", (2 ** L,)), L, _dev(words, torch.int32, "words", (n, W)),
                                    W, _dev(scale1, torch.float16, "scale1", (n,)),
                                    _opt(paths, torch.int32, "paths", (n, R)), _stream()), "fvs_trellis_encode")


def tr_scan(mode, blocks, Qr, pr, words, scale1, tab, L, t0=None, cnt=None, bval=None, bpos=None, bm=None, CAP=1,
            MB=1, n1=1, row0=0, half=False, nsplit=1):
    """Trellis stage-1 first pass (mode 0) or emit (mode 1) over the static (cell, block) items
    (src/s1cell.py:121-154 semantics with the canonical fp32 dot of include/fvs.h). words/scale1 hold index
    rows row0 .. (device or pinned host memory). half: both dot operands rounded to fp16 first (the
    reference's tensor-core operands for batches above 8 queries). nsplit: waves per item, each taking a
    consecutive part of the item's queries (for launches over few items)."""
    pcell, pblk, ps, pe = blocks
    qid, qrank, coff, ccnt, qcp = pr
    P_ = pcell.shape[0]
    B, R = Qr.shape
    N, W = words.shape
    if mode == 0 and (bm is None or bm.numel() != B * n1 * MB):
        raise ValueError("tr_scan: bm must hold B*n1*MB values")
    if mode == 1 and (bval is None or bval.shape != (B, CAP) or bpos.shape != (B, CAP) or cnt.shape != (B,)):
        raise ValueError("tr_scan: emit buffers must be [B, CAP]")
    f32, i32 = torch.float32, torch.int32
    _check(lib().fvs_tr_scan(mode, P_, _dev(Qr, f32, "Qr"), _dev(qid, i32, "qid"), _dev(qrank, i32, "qrank"),
                             _dev(coff, i32, "coff"), _dev(ccnt, i32, "ccnt"), _dev(pcell, i32, "pcell"),
                             _dev(pblk, i32, "pblk"), _dev(ps, i32, "ps"), _dev(pe, i32, "pe"),
                             _dev(words, i32, "words", host_ok=True), row0, W,
                             _dev(scale1, torch.float16, "scale1", (N,), host_ok=True), _dev(tab, f32, "tab", (2 ** L,)), L, R,
                             int(bool(half)), _dev(qcp, f32, "qcp"), _opt(t0, f32, "t0"), _opt(cnt, i32, "cnt"), _opt(bval, f32, "bval"),
                             _opt(bpos, i32, "bpos"), _opt(bm, f32, "bm"), CAP, MB, n1, int(nsplit), _stream()),
           "fvs_tr_scan")


def tr_scan_streamed(mode, chunk_tab, stage_h, slots, side, blocks, Qr, pr, tab, L, W, t0=None, cnt=None, bval=None,
                     bpos=None, bm=None, CAP=1, MB=1, n1=1, half=True, nsplit=1):
    """One streamed stage-1 pass of the host-resident engine (fvs_tr_scan_streamed): chunk_tab int64 numpy
    [nchunks, 5] (first row, end row, first item, end item, byte offset in stage_h), stage_h pinned uint8,
    slots two device uint8 buffers, side the copy stream; the other arguments as tr_scan's."""
    pcell, pblk, ps, pe = blocks
    qid, qrank, coff, ccnt, qcp = pr
    B, R = Qr.shape
    tab_ = np.ascontiguousarray(chunk_tab, dtype=np.int64)
    if tab_.ndim != 2 or tab_.shape[1] != 5:
        raise ValueError("tr_scan_streamed: chunk table must be [nchunks, 5]")
    if mode == 0 and (bm is None or bm.numel() != B * n1 * MB):
        raise ValueError("tr_scan_streamed: bm must hold B*n1*MB values")
    if mode == 1 and (bval is None or bval.shape != (B, CAP) or bpos.shape != (B, CAP) or cnt.shape != (B,)):
        raise ValueError("tr_scan_streamed: emit buffers must be [B, CAP]")
    if slots[0].numel() != slots[1].numel():
        raise ValueError("tr_scan_streamed: slots of different sizes")
    f32, i32, u8 = torch.float32, torch.int32, torch.uint8
    _check(lib().fvs_tr_scan_streamed(
        mode, tab_.shape[0], tab_.ctypes.data_as(P), _dev(stage_h, u8, "stage_h", host_ok=True),
        _dev(slots[0], u8, "slot0"), _dev(slots[1], u8, "slot1"), slots[0].numel(), P(side.cuda_stream),
        _dev(Qr, f32, "Qr"), _dev(qid, i32, "qid"), _dev(qrank, i32, "qrank"), _dev(coff, i32, "coff"),
        _dev(ccnt, i32, "ccnt"), _dev(pcell, i32, "pcell"), _dev(pblk, i32, "pblk"), _dev(ps, i32, "ps"),
        _dev(pe, i32, "pe"), W, _dev(tab, f32, "tab", (2 ** L,)), L, R, int(bool(half)), _dev(qcp, f32, "qcp"),
        _opt(t0, f32, "t0"), _opt(cnt, i32, "cnt"), _opt(bval, f32, "bval"), _opt(bpos, i32, "bpos"),
        _opt(bm, f32, "bm"), CAP, MB, n1, int(nsplit), _stream()), "fvs_tr_scan_streamed")


def route_topk_scaled(QM, scale, nprobe, qadd=None):
    """Top-n_p cells by the fp32 key (float)QM * scale, or ((float)QM + qadd[q]) * scale
    (src/engine_cell.py:40-42, host_resident/space_x.py:33-39)."""
    B, NC = QM.shape
    probe = _empty((B, nprobe), torch.int32, QM.device)
    _check(lib().fvs_route_topk_scaled(_dev(QM, torch.float16, "QM"), _dev(scale, torch.float32, "scale", (NC,)),
                                       _opt(qadd, torch.float32, "qadd", (B,)), B,
                                       NC, nprobe, _dev(probe, torch.int32, "probe"), _stream()), "fvs_route_topk_scaled")
    return probe


def route_keys(QM, scale=None, qadd=None):
    """fp16 [B, NC] routing keys ((float)QM + qadd[q]) * scale[c], each term optional (throughput/enginei8.py:72-76)."""
    B, NC = QM.shape
    out = _empty((B, NC), torch.float16, QM.device)
    _check(lib().fvs_route_keys(_dev(QM, torch.float16, "QM"), _opt(scale, torch.float32, "scale", (NC,)),
                                _opt(qadd, torch.float32, "qadd", (B,)), B, NC, _dev(out, torch.float16, "out"),
                                _stream()), "fvs_route_keys")
    return out


def tiered_score(pos, qc, Zq, code, ncnt=None):
    """(est, sd) [B, K] of the Lloyd-Max tiered code (src/tiered_fused.py:47-72) from the packed records."""
    B, K = pos.shape
    D = Zq.shape[1]
    TS = code["TS"]
    T = len(TS)
    rec = code["rec"]
    N, RB = rec.shape
    toff = (ctypes.c_int32 * T)(*[int(x) for x in code["toff"]])
    est = _empty((B, K), torch.float32, pos.device)
    sd = _empty((B, K), torch.float32, pos.device)
    _check(lib().fvs_tiered_score(_dev(pos, torch.int32, "pos"), _dev(qc, torch.float32, "qc", (B,)),
                                  _dev(Zq, torch.float32, "Zq", (B, D)), D, _dev(rec, torch.uint8, "rec", host_ok=True), N, RB,
                                  int(code["soff"]), T, _tiers_arr(TS), toff, _dev(code["cb"], torch.float32, "cb", (T, 256)),
                                  _opt(ncnt, torch.int32, "ncnt", (B,)), B, K, _dev(est, torch.float32, "est"),
                                  _dev(sd, torch.float32, "sd"), _stream()), "fvs_tiered_score")
    return est, sd


# --------------------------------------------------------------------------- routing-free scan (brute force)
DENSE_QT, DENSE_NT = 128, 256  # query and row tile of fvs_dense_scan


def round_up(n, m):
    return -(-n // m) * m


def quantize_i8(z, half=False, q=None, scale=None):
    """(q int8 [n, R], scale [n]): per-row int8 code with scale max|z|/127 (throughput/brute.py:46-47, :51-52);
    the scale is f32, or fp16 (nearest even) when half. q and scale may be given (views into larger buffers)."""
    n, R = z.shape
    q = _empty((n, R), torch.int8, z.device) if q is None else q
    sdt = torch.float16 if half else torch.float32
    scale = _empty((n,), sdt, z.device) if scale is None else scale
    sp = _dev(scale, sdt, "scale", (n,))
    _check(lib().fvs_quantize_i8(_dev(z, torch.float32, "z"), n, R, _dev(q, torch.int8, "q", (n, R)),
                                 P(None) if half else sp, sp if half else P(None), _stream()), "fvs_quantize_i8")
    return q, scale


def dense_pack(X, npad, Rp=None, out=None):
    """Fragment-tiled copy (fvs_dense_pack) of X int8 [n, R], zero-padded to npad rows and Rp columns (default:
    R rounded up to 128): a flat int8 tensor of npad * Rp bytes."""
    n, R = X.shape
    Rp = round_up(R, 128) if Rp is None else Rp
    T = _empty((npad * Rp,), torch.int8, X.device) if out is None else out
    if T.numel() != npad * Rp:
        raise ValueError("dense_pack: output size")
    _check(lib().fvs_dense_pack(_dev(X, torch.int8, "X") if n else P(None), n, R, npad, Rp, _dev(T, torch.int8, "T"),
                                _stream()), "fvs_dense_pack")
    return T


def dense_threshold(S, r, cnt=None):
    """t0 [B] = r-th largest of each row of S f32 [B, n] (throughput/brute.py:59); zeroes cnt [B] if given."""
    B, n = S.shape
    t0 = _empty((B,), torch.float32, S.device)
    _check(lib().fvs_dense_threshold(_dev(S, torch.float32, "S"), B, n, r, _dev(t0, torch.float32, "t0"),
                                     _opt(cnt, torch.int32, "cnt", (B,)), _stream()), "fvs_dense_threshold")
    return t0


def dense_scan(mode, Qt, qs, B, Zt, zs, N, R, t0=None, cnt=None, bval=None, bpos=None, CAP=1, out=None):
    """Routing-free int8 scan (throughput/brute.py:7-35): mode 0 fills out f32 [B, N] with the scores, mode 1
    emits every (q, n) with est >= t0[q] into bval / bpos [B, CAP] and counts them in cnt [B]. Qt / Zt: packed
    codes (dense_pack) of Bpad / Npad rows; qs and t0 hold Bpad values and zs (fp16) Npad values."""
    Bpad = Qt.numel() // R
    Npad = Zt.numel() // R
    if Qt.numel() != Bpad * R or Zt.numel() != Npad * R or Bpad < B or Npad < N:
        raise ValueError("dense_scan: packed code sizes")
    if qs.numel() < Bpad or zs.numel() < Npad or (mode == 1 and t0.numel() < Bpad):
        raise ValueError("dense_scan: qs, t0 need Bpad values and zs Npad values")
    if mode == 0 and (out is None or out.shape != (B, N)):
        raise ValueError("dense_scan: out must be [B, N]")
    if mode == 1 and (bval.shape != (B, CAP) or bpos.shape != (B, CAP) or cnt.shape != (B,)):
        raise ValueError("dense_scan: emit buffers must be [B, CAP]")
    f32, i32 = torch.float32, torch.int32
    _check(lib().fvs_dense_scan(mode, _dev(Qt, torch.int8, "Qt"), _dev(qs, f32, "qs"), B, Bpad, _dev(Zt, torch.int8, "Zt"),
                                _dev(zs, torch.float16, "zs"), N, Npad, R, _opt(t0, f32, "t0"), _opt(cnt, i32, "cnt"),
                                _opt(bval, f32, "bval"), _opt(bpos, i32, "bpos"), CAP, _opt(out, f32, "out"),
                                _stream()), "fvs_dense_scan")
