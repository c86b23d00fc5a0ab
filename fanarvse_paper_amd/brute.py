"""Routing-free stage 1 (throughput/brute.py:41-63): every query's int8 code against every stored int8 code,
a dense contraction on MFMA (fvs_dense_scan), with the reference's per-query threshold from a fixed sample of
the stored rows and its exactness flag (K <= emitted <= M).

The class keeps the reference's constructor and methods (`qcode`, `scores`, `search`) and their results:
  * codes: z = (x - mu) @ V[:, :R]; a = max(max|z|, 1e-12) / 127; code = clamp(rint(z / a), -127, 127), the
    stored scale rounded to fp16 (brute.py:46-47), the query scale kept in fp32 (brute.py:51-52);
  * scores: est = ((float)acc * qs[q]) * (float)zs[n] with acc the exact int32 dot (brute.py:16-17);
  * threshold: t0[q] = the r-th largest sample score, r = max(1, round(over * K * frac)) (brute.py:58-59);
  * emit: every (q, n) with est >= t0[q] counted, the first M kept (brute.py:31-37), then the top K of the
    buffer by (est descending, position ascending) (brute.py:63).
The stored codes are also kept in the fragment-tiled layout the MFMA scan reads (fvs_dense_pack), padded to
multiples of 256 rows and 128 columns; the padding is zero and changes no dot product.

The projections (x - mu) @ V are torch products, as in the reference; everything after them runs in libfvs.
"""
import torch

from . import _lib


class Brute:
    """throughput/brute.py:41-63. `sidx` (optional): the sample rows, in place of every `sample_every`-th row
    (throughput/cbrute.py:73 draws a random 5% sample instead)."""

    def __init__(self, X16, mu, V, R=128, sample_every=20, chunk=65536, sidx=None):
        dev = V.device
        if dev.type != "cuda":
            raise ValueError("Brute: V must be on the GPU")
        self.R, self.mu, self.V = R, mu.to(dev, torch.float32), V[:, :R].contiguous().float()
        N = len(X16)
        self.N = N
        self.Rp = _lib.round_up(R, 128)
        self.Z = torch.empty(N, R, dtype=torch.int8, device=dev)
        self.zs = torch.empty(N, dtype=torch.float16, device=dev)
        for j in range(0, N, chunk):
            z = ((X16[j:j + chunk].to(dev).float() - self.mu) @ self.V).contiguous()
            _lib.quantize_i8(z, half=True, q=self.Z[j:j + chunk], scale=self.zs[j:j + chunk])
        self.Zt, self.zsp = self._pack_rows(self.Z, self.zs)
        if sidx is None:
            sidx = torch.arange(0, N, sample_every, device=dev)
        self.sidx = sidx.to(dev)
        self.Zs, self.zss = self.Z[self.sidx].contiguous(), self.zs[self.sidx].contiguous()
        self.Zst, self.zssp = self._pack_rows(self.Zs, self.zss)
        self.frac = len(self.sidx) / N

    def _pack_rows(self, Z, zs):
        n = len(Z)
        npad = _lib.round_up(max(n, 1), _lib.DENSE_NT)
        zsp = torch.zeros(npad, dtype=torch.float16, device=Z.device)
        zsp[:n] = zs
        return _lib.dense_pack(Z, npad, self.Rp), zsp

    def _pack_queries(self, q, qs, t0=None):
        B = len(q)
        Bpad = _lib.round_up(max(B, 1), _lib.DENSE_QT)
        qsp = torch.zeros(Bpad, dtype=torch.float32, device=q.device)
        qsp[:B] = qs
        t0p = None
        if t0 is not None:
            t0p = torch.full((Bpad,), 1e30, dtype=torch.float32, device=q.device)
            t0p[:B] = t0
        return _lib.dense_pack(q, Bpad, self.Rp), qsp, t0p

    def qcode(self, Qb):
        """(q int8 [B, R], qs f32 [B]) of the queries (throughput/brute.py:50-52)."""
        z = ((Qb.to(self.V.device).float() - self.mu) @ self.V).contiguous()
        return _lib.quantize_i8(z)

    def scores(self, q, qs, Z=None, zs=None):
        """Dense scores f32 [B, n] of codes q [B, R] (scales qs f32) against Z [n, R] (scales zs fp16), by
        default the stored rows (throughput/brute.py:53-55)."""
        if Z is None:
            Zt, zsp, n = self.Zt, self.zsp, self.N
        elif Z is self.Zs:
            Zt, zsp, n = self.Zst, self.zssp, len(Z)
        else:
            Zt, zsp = self._pack_rows(Z.contiguous(), zs.to(torch.float16).contiguous())
            n = len(Z)
        Qt, qsp, _ = self._pack_queries(q.contiguous(), qs.float())
        B = len(q)
        out = torch.empty(B, n, dtype=torch.float32, device=q.device)
        _lib.dense_scan(0, Qt, qsp, B, Zt, zsp, n, self.Rp, out=out)
        return out

    def threshold(self, q, qs, r):
        """(t0 f32 [B], cnt i32 [B] zeroed): the r-th largest sample score per query (throughput/brute.py:59)."""
        S = self.scores(q, qs, self.Zs, self.zss)
        cnt = torch.empty(len(q), dtype=torch.int32, device=q.device)
        return _lib.dense_threshold(S, r, cnt), cnt

    def search(self, Qb, K, over=2.0, M=None, mode=1):
        """(pos int64 [B, K], est f32 [B, K], ok bool [B], cnt i32 [B]) (throughput/brute.py:56-63). mode 1 and 3
        emit the same set (one atomic per kept pair; the reference's mode 3 only changes the buffer order)."""
        if mode not in (1, 3):
            raise ValueError("Brute.search: mode must be 1 or 3")
        q, qs = self.qcode(Qb)
        B = len(Qb)
        M = M or max(4096, 8 * K)
        r = max(1, int(round(over * K * self.frac)))
        t0, cnt = self.threshold(q, qs, r)
        Qt, qsp, t0p = self._pack_queries(q, qs, t0)
        bval = torch.empty(B, M, dtype=torch.float32, device=q.device)
        bpos = torch.empty(B, M, dtype=torch.int32, device=q.device)
        _lib.dense_scan(1, Qt, qsp, B, self.Zt, self.zsp, self.N, self.Rp, t0=t0p, cnt=cnt, bval=bval, bpos=bpos,
                        CAP=M)
        pos, est, ok, _ = _lib.select(bval, bpos, cnt, K, 0, None)
        return pos.long(), est, ok.bool(), cnt
