"""EngineS on MI355X: the default (trellis cell-residual) engine of FanarVSE, used by the latency mode.

Same entry points as the reference (src/engine_cell.py:70-102 EngineS, with Engine8's stage 2 and
stage 3, src/engine3.py:135-175):
    s1, code = trellis.build_index(X16, nlist)          # compact(cellify(...)) tables + Lloyd-Max code
    E = EngineS(s1, code, H=X16)
    I, reads, cand_ids = E.search(Qb, K, z, nprobe, k)
A batch is one hipGraph replay per (B, K, z, nprobe, k) and one host synchronisation on the exactness
flags; flagged queries are redone with rho = 1, beta = 1.5 and a 65,536-entry buffer, by a captured
graph too (flagged rows padded to a power of two, or a multiple of 64 beyond 64). search_host is the lean latency path
(src/engine_cell.py:130-165, EngineT.search_host): the graph itself copies the flags and the top-k ids
into pinned host memory, so a search is one replay and one stream synchronisation.

Stage 1 is the static work-list scan (src/s1cell.py:176-195) for every batch size. The reference
switches to per-(query, cell) programs for B <= 8 and to a dense probe mask for B <= 32
(src/s1small_cell.py:29-88); those kernels select by the same threshold-and-emit rule. Their operand
precision is kept: above TINY = 8 queries the reference's tensor-core dots take fp16 operands
(Qr.half() and the decoded table values .to(tl.float16), src/s1cell.py:127,131-132,
src/s1small_cell.py:57-59), at most 8 queries keep fp32 operands (src/s1small_cell.py:17-20). One work-list
kernel serves every size with one fp32 accumulation order; `half` selects the operand rounding. The
fallback of `search` rounds to fp16 too (the reference redoes flagged queries with search_guess, whose
queries are Qr.half(), src/engine3.py:45-48 via src/engine_cell.py:60-64); the lean path's fallback for a
lone query keeps fp32 (src/engine_cell.py:165 runs search_small again). The dense products differ by
batch size as well (fvs_dense_small up to 8 queries, library products above), so a query's estimates
can change between a batch of 8 and a batch of 9.
"""
import numpy as np
import torch

from . import _lib, index, s2lut
from .enginei8 import _fresh, capture, padded_rows


class EngineS:
    BN = 32
    M = None          # emit buffer size; None = index.emit_buffer(B, K)
    TINY = 8          # batches up to TINY keep fp32 stage-1 operands (src/engine_cell.py:48)
    SMALL_CAP = 8192  # their emit buffer in search(): search_small's CAP (src/s1small_cell.py:29)

    def __init__(self, s1, code, H=None):
        self.s1, self.code, self.H = s1, code, H
        s2lut.prepare_u(code)
        if "VP" not in code:
            raise ValueError("EngineS needs a Lloyd-Max tiered code (s2lut.encode_lloyd)")
        self.blocks, self.MB = index.static_blocks(s1["off_t"], self.BN)
        self.W1 = s1["W1"].contiguous()
        self.inv_mnorm = s1["inv_mnorm"].float().contiguous()
        self.means16 = s1["means16"].contiguous()
        # row-major transposes for the one-launch dense products of small batches (_lib.dense_small)
        self.W1T = self.W1.T.contiguous()
        self.VPT = code["VP"].float().T.contiguous()
        self.graphs = {}
        self.nbad = 0
        self._done = torch.cuda.Event() if torch.cuda.is_available() else None
        if int(s1["off_t"][-1]) != s1["words"].shape[0]:
            raise ValueError("EngineS: cell offsets do not match the code rows")

    def _params(self, K, nprobe, rho_override=None, M_override=None, B=None, lean=False):
        """(M, n1, r). M: a batch of at most TINY queries in search() keeps the reference's buffer, because
        its overflowing queries are redone with other operand precision (fp16, while the main pass keeps
        fp32), so the buffer size decides which arithmetic gives their candidates. Elsewhere the main pass
        and the fallback share one precision and a larger buffer (index.emit_buffer) changes no result."""
        NC = len(self.s1["off"]) - 1
        N = self.s1["words"].shape[0]
        small = B is not None and B <= self.TINY and not lean
        M = M_override or self.M or (self.SMALL_CAP if small else index.emit_buffer(B, K))
        beta, rho = (1.1, 0.75) if K <= 400 else (0.7, 0.5)
        if rho_override:
            beta, rho = 1.5, rho_override
        n1 = min(max(int(np.ceil(beta * K / (N / NC / self.BN + 1))), 1), nprobe)
        return M, n1, int(np.ceil(rho * K))

    def stage1(self, Qr, QM, probe, K, rho_override=None, M_override=None, half=True, lean=False):
        """Threshold-and-emit over the trellis codes (src/s1cell.py:176-195). Returns (pos, ok). half: fp16
        dot operands (src/s1cell.py:127,131-132); lean: the latency path's buffer rule (_params)."""
        s1 = self.s1
        NC = len(s1["off"]) - 1
        B = Qr.shape[0]
        dev = Qr.device
        M, n1, r = self._params(K, probe.shape[1], rho_override, M_override, B, lean)
        L = int(s1["L"])
        scratch = _lib.pairs_scratch(B, NC, dev)
        pr, prn = _lib.pairs2(probe, n1, NC, QM, None, scratch)
        bm = torch.empty((B, n1, self.MB), dtype=torch.float32, device=dev)
        _lib.tr_scan(0, self.blocks, Qr, pr, s1["words"], s1["scale1"], s1["tab"], L, bm=bm, MB=self.MB, n1=n1,
                     half=half)
        cnt = torch.empty((B,), dtype=torch.int32, device=dev)  # zeroed by the threshold kernel
        t0 = _lib.threshold(bm, probe, s1["off_t"], n1, self.MB, r, cnt)
        bval = torch.empty((B, M), dtype=torch.float32, device=dev)
        bpos = torch.empty((B, M), dtype=torch.int32, device=dev)
        pr = prn
        _lib.tr_scan(1, self.blocks, Qr, pr, s1["words"], s1["scale1"], s1["tab"], L, t0=t0, cnt=cnt, bval=bval,
                     bpos=bpos, CAP=M, half=half)
        pos, est1, ok, _ = _lib.select(bval, bpos, cnt, K, 0, None)
        self._bm, self._t0, self._cnt, self._bval, self._bpos, self._n1, self._M = bm, t0, cnt, bval, bpos, n1, M
        return pos, ok.view(torch.bool)  # the kernel writes 0 / 1 bytes: a view, no conversion kernel

    def _dense(self, Qb):
        """The dense products: Qr = Qb @ W1 (f32), QM = fp16(Qb) @ means16.T (fp16), Zq = Qb @ VP (f32);
        and qc = <Qb, c> (canonical double sum)."""
        if len(Qb) <= _lib.DENSE_MAX_B:  # one launch instead of three library products
            Qr, QM, Zq, QC = _lib.dense_small(Qb, self.W1T, self.means16, self.VPT, self.s1["c"])
            return Qr, QC, QM, Zq
        Qr = (Qb @ self.W1).contiguous()
        _, _, QC, Qh, _ = _lib.query_prep(Qb, self.W1, self.s1["c"], Qr)
        QM = (Qh @ self.means16.T).contiguous()
        Zq = (Qb @ self.code["VP"]).contiguous()
        return Qr, QC, QM, Zq

    def _finish(self, Qb, QC, Zq, pos, z, k):
        est, sd = _lib.tiered_score(pos, QC, Zq, self.code)
        self._est, self._sd = est, sd
        return _lib.refine(est, sd, pos, self.s1["order"], self.H, Qb, z, k)

    def _gpu(self, Qb, K, z, nprobe, k, lean=False):
        if self.H is None:
            raise RuntimeError("EngineS.H (fp16 vectors in id order) must be set before searching")
        Qr, QC, QM, Zq = self._dense(Qb)
        probe = _lib.route_topk_scaled(QM, self.inv_mnorm, nprobe)
        pos, ok = self.stage1(Qr, QM, probe, K, half=len(Qb) > self.TINY, lean=lean)
        ids, I, scores, reads = self._finish(Qb, QC, Zq, pos, z, k)
        return ok, I, reads, ids, scores, (Qr, QC, QM, Zq, probe)

    _capture = staticmethod(capture)

    def _main(self, Qb, K, z, nprobe, k, host=False):
        """The captured search of a (B, K, z, nprobe, k) batch. host: the graph also copies
        [ok | top-k ids] (int64) into pinned host memory."""
        B = len(Qb)
        key = ("host" if host else "dev", B, K, float(z), nprobe, k, self.M)  # a change of M captures anew
        if key not in self.graphs:
            qs = Qb.clone()
            # host: [ok | top-k ids] as int64; otherwise the flags alone (bool) reach the host in the graph
            hb = torch.empty((B, k + 1) if host else (B,), dtype=torch.int64 if host else torch.bool, pin_memory=True)

            def run():
                outs = self._gpu(qs, K, z, nprobe, k, lean=host and B == 1)
                if host:
                    _lib.pack_ids(outs[0], outs[1], hb)  # one launch writes the pinned buffer directly
                else:
                    hb.copy_(outs[0], non_blocking=True)
                return outs

            g, outs = self._capture(run)
            self.graphs[key] = (key, g, qs, outs, hb)
            # a lone flagged query needs no capture later. The fallback's warm-up runs read the main graph's
            # static outputs (probe lists included), which a capture leaves unwritten: replay it first.
            g.replay()
            self._fallback_graph(self.graphs[key], 1)
        return self.graphs[key]

    def _fallback_graph(self, entry, nbp):
        """The captured fallback of nbp rows gathered from the static inputs of the main graph `entry`."""
        key, _, qs, (ok, I, nr, ids, sc, dense), _ = entry
        fkey = ("fb", key, nbp)
        if fkey not in self.graphs:
            sel = torch.zeros(nbp, dtype=torch.int64, device=qs.device)
            K, z, k = key[2], key[3], key[5]
            half = not (key[0] == "host" and key[1] == 1)  # a lone lean-path query keeps fp32 operands

            def run():
                a = [t.index_select(0, sel) for t in (qs,) + tuple(dense)]
                return self._fallback(a[0], K, z, k, *a[1:], half=half)

            g, outs = self._capture(run)
            self.graphs[fkey] = (g, sel, outs)
        return self.graphs[fkey]

    def _fallback_rows(self, entry, bad):
        """Flagged rows `bad` (host int64) of the batch last replayed in `entry`, recomputed by a captured
        fallback graph over a padding of the rows (enginei8.padded_rows; the last row repeated). Returns the
        device tensors (I, reads, ids, scores) of the len(bad) rows."""
        nb = len(bad)
        nbp = padded_rows(nb)
        g, sel, outs = self._fallback_graph(entry, nbp)
        pad = np.concatenate([bad, np.full(nbp - nb, bad[-1], np.int64)])
        sel.copy_(torch.from_numpy(pad), non_blocking=False)
        g.replay()
        self.nbad += nb
        return [t[:nb] for t in outs]

    def search(self, Qb, K, z, nprobe, k, ret_scores=False):
        """(I [B,k], reads [B], cand_ids [B,K]) (+ scores) as src/engine_cell.py:85-102."""
        Qb = Qb.float().contiguous()
        entry = self._main(Qb, K, z, nprobe, k)
        _, g, qs, (ok, I, nr, ids, sc, dense), hb = entry
        qs.copy_(Qb)
        g.replay()
        done = self._done
        done.record()
        I, nr, ids, sc = _fresh(I, nr, ids, sc)  # runs while the host reads the flags
        done.synchronize()
        okh = hb.numpy()
        if not okh.all():
            bad = np.nonzero(~okh)[0].astype(np.int64)
            a, b, c, s = self._fallback_rows(entry, bad)
            bd = torch.from_numpy(bad).to(Qb.device)
            I[bd], nr[bd], ids[bd], sc[bd] = a, b, c, s
        return (I, nr, ids, sc) if ret_scores else (I, nr, ids)

    def search_host(self, Qb, K, z, nprobe, k):
        """Top-k ids [B, k] as an int64 numpy array: the latency path of src/engine_cell.py:152-165. One
        graph replay, which ends by copying the exactness flags and the ids into pinned host memory, and
        one stream synchronisation; flagged queries go through the captured fallback."""
        Qb = Qb.float().contiguous()
        entry = self._main(Qb, K, z, nprobe, k, host=True)
        _, g, qs, _, hb = entry
        qs.copy_(Qb)
        g.replay()
        torch.cuda.current_stream().synchronize()
        h = hb.numpy()
        out = h[:, 1:].copy()
        if not h[:, 0].all():
            bad = np.nonzero(h[:, 0] == 0)[0].astype(np.int64)
            out[bad] = self._fallback_rows(entry, bad)[0].cpu().numpy()
        return out

    def _fallback(self, Qb, K, z, k, Qr, QC, QM, Zq, probe, half=True):
        """Flagged queries again with rho = 1, beta = 1.5 and M = 65,536 (the reference recomputes them with
        the work-list path and a larger buffer, src/engine_cell.py:98-101)."""
        pos, _ = self.stage1(Qr, QM, probe, K, rho_override=1.0, M_override=65536, half=half)
        ids, I, scores, reads = self._finish(Qb, QC, Zq, pos, z, k)
        return I, reads, ids, scores

    def trace(self, Qb, K, z, nprobe, k):
        """Eager run of one batch returning every intermediate (parity tests)."""
        Qb = Qb.float().contiguous()
        Qr, QC, QM, Zq = self._dense(Qb)
        probe = _lib.route_topk_scaled(QM, self.inv_mnorm, nprobe)
        pos, ok = self.stage1(Qr, QM, probe, K, half=len(Qb) > self.TINY)
        ids, I, scores, reads = self._finish(Qb, QC, Zq, pos, z, k)
        return dict(Qr=Qr, QC=QC, QM=QM, Zq=Zq, probe=probe, bm=self._bm, n1=self._n1, M=self._M, t0=self._t0,
                    cnt=self._cnt, bval=self._bval, bpos=self._bpos, pos=pos, ok=ok, est=self._est, sd=self._sd,
                    ids=ids, I=I, scores=scores, reads=reads)

    def gpu_bytes(self):
        """Bytes per vector on the GPU (src/v19_final.py:29-32): trellis words + scale + id, the record, tables."""
        s1 = self.s1
        N = s1["words"].shape[0]
        per = s1["words"].shape[1] * 4 + 2 + 4 + self.code["RB"]
        tables = self.means16.numel() * 2 + self.W1.numel() * 4 + self.inv_mnorm.numel() * 4 + s1["tab"].numel() * 4
        return per + tables / N
