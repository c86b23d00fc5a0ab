"""EngineI8 on MI355X: the throughput-mode batched search of FanarVSE (FanarVSE-T).

Same entry points and knobs as the reference (throughput/enginei8.py:29-122):
    E = EngineI8(s1, code, Z, zs, Vr); E.H = <fp16 vectors in id order>
    I, reads, cand_ids = E.search(Qb, K, z, nprobe, k)
The search is one hipGraph replay per (B, K, z, nprobe, k) followed by one host synchronisation on
the exactness flags; flagged queries are recomputed by _fallback (rho = 1, beta = 1.5, a 65,536-entry
buffer, an fp32 LUT and no delta rule), as in the reference. A serving loop can keep the GPU busy
through that synchronisation with submit / collect: NINST (3) captured instances per key take turns,
each replayed on its own stream, so the next batches run on the GPU alongside batch i while batch i's
flags are read. Every stage runs in libfvs kernels; the
two plain fp16 GEMMs (routing scores and the rotated tier queries) use torch's BLAS.

The class attributes default to the final operating point of throughput/e_v3final.py:16,28-30
(NROUTE, LUTF, LUTH, DELTA = 0.07, RHO = 0.6, MSZ = 3072). The routing and stage-2 knobs of the reference
work as there (throughput/enginei8.py:66-86):
  * NROUTE = False: QM = fp16(Qb) @ means16.T, cells ranked by (float)QM * inv_mnorm (rounded to fp16 when
    ROUTE16), pair constants QM unscaled; PROJ (with NROUTE False) replaces QM by the stage-1 projection
    fp16(QC + fp16(fp16(Qb) @ W1) @ mproj) and needs s1["W1"]; the fallback keeps the plain QM and fp32 keys;
  * UNSORTED: the n_p probed cells in cell order instead of score order (the reference's unsorted topk
    order is unspecified; the first n1 of them seed the threshold either way);
  * SORTROUTE: sort-then-cut equals the sorted top-n_p under this build's (score desc, cell asc) order;
  * K2 < K: every candidate is ranked by the LUT estimate over the first NT tiers, and only the K2 best
    go on to the full stage 2, the delta rule and the exact reads.
"""
import math

import numpy as np
import torch

from . import _lib, index, s2lut


def pairs_fast(probe, NC, QM, scale=None):
    """(qid, coff, ccnt, qc, qrank) of the (query, cell) pairs, grouped by cell with queries ascending
    (throughput/enginei8.py:11-16). `qrank` replaces the permutation `o`: it is the rank of the cell in
    the query's probe row, which is all the first pass needs to place its block maxima."""
    qid, qrank, coff, ccnt, qcp = _lib.pairs(probe, probe.shape[1], NC, QM, scale)
    return qid, coff, ccnt, qcp, qrank


def capture(fn, stream=None):
    """Run fn three times on a side stream (allocations and lazy set-up happen there), then capture one
    more run into a hipGraph (on `stream` when given: the library GEMMs' workspaces belong to the stream
    they are captured on). Returns (graph, fn's outputs)."""
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        outs = fn()
    return g, outs


def padded_rows(nb):
    """Rows of a captured fallback graph for nb flagged queries: a power of two up to 64, then a
    multiple of 64 (so a handful of graphs serves every count)."""
    return 1 << (nb - 1).bit_length() if nb <= 64 else -(-nb // 64) * 64


def _fresh(*ts):
    """Copies of the graph's output tensors (int32 / float32) for the caller, made by one gather kernel into
    one new buffer instead of one copy per tensor."""
    flat = torch.cat([t.reshape(-1).view(torch.int32) for t in ts])
    out, at = [], 0
    for t in ts:
        out.append(flat[at:at + t.numel()].view(t.dtype).view(t.shape))
        at += t.numel()
    return out


class EngineI8:
    BQ, BN = 32, 32
    PROJ = False
    UNSORTED = False
    CUDA = False
    FASTPAIRS = True
    NW = 2
    SORTROUTE = False
    MSZ = 3072
    ROUTE16 = True
    LUTF = True
    K2 = None
    NT = 3
    BETA = None
    RHO = 0.6
    NROUTE = True
    DELTA = 0.07
    LUTH = True
    CB = 4  # 32-row blocks per first-pass work item (the first-pass kernel's item span)
    EROWS = 128  # rows per emit work item (the emit kernel's item span)
    NINST = 3  # graph instances per search shape: batches that submit / collect keep in flight
    # the projection z = Qb @ Vr of the query code: False, the fp32 library GEMM (as the reference's cuBLAS
    # product); True, fvs_query_code's sequential fmaf chain, which the oracle reproduces bit for bit (its VALU
    # work costs about 3.5 % of the pipelined throughput against the matrix-core GEMM)
    CANON_Z = False

    def __init__(self, s1, code, Z, zs, Vr, H=None):
        if self.BN != 32:
            raise NotImplementedError("the MFMA scan uses 32-row blocks")
        self.s1, self.code, self.Z, self.zs, self.Vr = s1, code, Z, zs, Vr.contiguous()
        self.H = H
        s2lut.prepare_u(code)
        _, self.MB = index.static_blocks(s1["off_t"], self.BN)
        self.blocks = index.static_chunks(s1["off_t"], self.BN, self.CB)  # first pass: global 32-row blocks
        self.rchunks = index.row_chunks(s1["off_t"], self.EROWS)  # emit: 128-row chunks from each cell's start
        N = Z.shape[0]
        if int(s1["off_t"][-1]) != N or int(self.blocks[3].max()) > N:
            raise ValueError("EngineI8: cell offsets do not match the code rows")
        self.meansN = (s1["means16"].float() * s1["inv_mnorm"][:, None]).half().contiguous()
        self.mnorm = (1.0 / s1["inv_mnorm"]).float().contiguous()
        self.graphs = {}
        self._pending = set()  # (key, instance) submitted and not yet collected
        self._side = None  # stream for the stage-2 tables (default priority)
        self.nbad = 0
        self.nbad2 = 0

    # ------------------------------------------------------------------ stages
    def _knobs(self):
        """The knob values captured work depends on: a search after a change captures new graphs."""
        return (self.MSZ, self.BETA, self.RHO, self.DELTA, self.LUTF, self.LUTH, self.NROUTE, self.ROUTE16,
                self.PROJ, self.UNSORTED, self.SORTROUTE, self.K2, self.NT, self.CANON_Z)

    def _check_knobs(self):
        if self.PROJ and not self.NROUTE and "W1" not in self.s1:
            raise ValueError("PROJ routing needs the stage-1 basis s1['W1'] (a trellis-built s1)")

    def _params(self, K, nprobe, rho_override=None, M_override=None):
        NC = len(self.s1["off"]) - 1
        N = self.Z.shape[0]
        M = M_override or self.MSZ or max(4096, 16 * K)
        beta, rho = (1.1, 0.75) if K <= 400 else (0.7, 0.5)
        if self.BETA:
            beta = self.BETA
        if self.RHO:
            rho = self.RHO
        if rho_override:
            beta, rho = 1.5, rho_override
        n1 = min(max(int(np.ceil(beta * K / (N / NC / self.BN + 1))), 1), nprobe)
        r = int(np.ceil(rho * K))
        return M, n1, r

    def stage1_i8(self, Qb, QM, probe, K, rho_override=None, M_override=None, qp=None, delta=None, kd=9):
        """Threshold-and-emit stage 1 (throughput/enginei8.py:36-60). Returns (pos [B,K] int32, ok bool);
        sets self._est1 and self._ncnt (the delta-rule count, K when delta is None)."""
        s1 = self.s1
        NC = len(s1["off"]) - 1
        B = Qb.shape[0]
        q8, qs = (qp if qp is not None else _lib.query_prep(Qb, self.Vr, s1["c"], canonical=self.CANON_Z))[:2]
        M, n1, r = self._params(K, probe.shape[1], rho_override, M_override)
        scratch = _lib.pairs_scratch(B, NC, Qb.device)
        # NROUTE: QM holds normalised-mean scores, the pair constants scale them back by |m_c|
        pr, prn = _lib.pairs2(probe, n1, NC, QM, self.mnorm if self.NROUTE else None, scratch)
        bm = torch.empty((B, n1, self.MB), dtype=torch.float32, device=Qb.device)
        _lib.i8_scan(0, self.blocks, q8, qs, pr, self.Z, self.zs, bm=bm, MB=self.MB, n1=n1)
        cnt = torch.empty((B,), dtype=torch.int32, device=Qb.device)  # zeroed by the threshold kernel
        t0 = _lib.threshold(bm, probe, s1["off_t"], n1, self.MB, r, cnt)
        bval = torch.empty((B, M), dtype=torch.float32, device=Qb.device)
        bpos = torch.empty((B, M), dtype=torch.int32, device=Qb.device)
        pr = prn
        _lib.i8_scan(1, self.rchunks, q8, qs, pr, self.Z, self.zs, t0=t0, cnt=cnt, bval=bval, bpos=bpos, CAP=M)
        pos, est1, ok, ncnt = _lib.select(bval, bpos, cnt, K, min(kd, K - 1), delta)
        self._est1, self._ncnt, self._t0, self._cnt = est1, ncnt, t0, cnt
        self._bm, self._bval, self._bpos, self._n1, self._M = bm, bval, bpos, n1, M
        return pos, ok.view(torch.bool)  # the kernel writes 0 / 1 bytes: a view, no conversion kernel

    def _plain_qm(self, Qh):
        """QM of the routing (NROUTE: against the normalised means; else against means16)."""
        return Qh @ (self.meansN if self.NROUTE else self.s1["means16"]).T

    def _route(self, Qh, QC, nprobe, QM=None):
        """(QM, probe) of the main pass (throughput/enginei8.py:66-76)."""
        if self.NROUTE:
            QM = self._plain_qm(Qh) if QM is None else QM
            probe = _lib.route_topk(QM, nprobe)
        else:
            if self.PROJ:
                if not hasattr(self, "mproj"):
                    s1 = self.s1
                    self.mproj = ((s1["means16"].float() - s1["c"]) @ s1["W1"].float()).half().T.contiguous()
                    self.W1h = s1["W1"].half().contiguous()
                QM = _lib.route_keys((Qh @ self.W1h) @ self.mproj, None, QC)
            elif QM is None:
                QM = self._plain_qm(Qh)
            if self.ROUTE16:
                probe = _lib.route_topk(_lib.route_keys(QM, self.s1["inv_mnorm"], None), nprobe)
            else:
                probe = _lib.route_topk_scaled(QM, self.s1["inv_mnorm"], nprobe)
        if self.UNSORTED:
            probe = torch.sort(probe, dim=1).values  # cell order
        return QM, probe

    def _gpu(self, Qb, K, z, nprobe, k):
        """One batch on the GPU without host synchronisation: (ok, I, reads, ids, scores, blas); blas holds the
        three BLAS products (z, QM, Zq) so that the fallback reuses their rows."""
        self._check_knobs()
        if self.H is None:
            raise RuntimeError("EngineI8.H (fp16 vectors in id order) must be set before searching")
        s1 = self.s1
        qp = _lib.query_prep(Qb, self.Vr, s1["c"], canonical=self.CANON_Z)
        q8, qs, QC, Qh, zq = qp
        # the stage-2 inputs depend only on the fp16 queries: a side stream computes the rotated queries while
        # stage 1 runs (the LUT scorer builds its tables from them). The routing product is issued before the
        # side branch: it heads the critical path, and a branch issued ahead of it was measured to hold it back
        # until the branch's first node had finished.
        main = torch.cuda.current_stream()
        if self._side is None:
            self._side = torch.cuda.Stream(device=Qb.device)
        prepped = torch.cuda.Event()
        prepped.record(main)
        QM0 = self._plain_qm(Qh)
        self._side.wait_event(prepped)
        half = self.LUTF and self.LUTH
        with torch.cuda.stream(self._side):
            Zq = s2lut.rotate(self.code, Qh)
        Zq.record_stream(main)  # made on the side stream, used on this one
        pre = _lib.ZqTables(Zq, half)
        QM, probe = self._route(Qh, QC, nprobe, QM0)
        pos, ok = self.stage1_i8(Qb, QM, probe, K, qp=qp, delta=self.DELTA, kd=k - 1)
        main.wait_stream(self._side)
        ok, I, reads, ids, scores = self._finish(Qb, Zq, QC, pos, ok, K, z, k, half=half,
                                                 ncnt=self._ncnt if self.DELTA is not None else None, pre=pre)
        return ok, I, reads, ids, scores, (zq, QM0, Zq)  # the fallback routes on the plain QM

    def _finish(self, Qb, Zq, QC, pos, ok, K, z, k, half, ncnt, pre=None):
        """LUT stage 2, error bars, exact reads and the final top-k (throughput/enginei8.py:80-95). The LUT scorer
        forms the tables of luts_fused (throughput/s2lut.py:108-126) from Zq itself (fvs_lut_score_zq)."""
        if pre is None:
            pre = _lib.ZqTables(Zq, half)
        if self.K2 is not None and self.K2 < K:
            # progressive stage 2 (throughput/enginei8.py:82-85): rank all K by the partial estimate over the
            # first NT tiers, keep the K2 best
            e_all, _ = s2lut.score_lut(self.code, QC, pos, pre, None, nt=min(self.NT, len(self.code["TS"])))
            cntK = torch.full((pos.shape[0],), K, dtype=torch.int32, device=pos.device)
            pos = _lib.select(e_all.contiguous(), pos.contiguous(), cntK, self.K2, 0, None)[0]
            if ncnt is not None:
                ncnt = ncnt.clamp(max=self.K2).contiguous()
        est, sd = s2lut.score_lut(self.code, QC, pos, pre, ncnt)
        self._est, self._sd = est, sd
        ids, I, scores, reads = _lib.refine(est, sd, pos, self.s1["order"], self.H, Qb, z, k)
        return ok, I, reads, ids, scores

    # ------------------------------------------------------------------ entry point
    def search(self, Qb, K, z, nprobe, k, ret_est=False, ret_scores=False):
        """(I [B,k] ids, reads [B], cand_ids [B,K]) (+ scores [B,k] when ret_scores): the exact scores of
        the picks read in full precision, the stage-2 estimates of the surely-in ones."""
        return self.collect(self.submit(Qb, K, z, nprobe, k), ret_scores=ret_scores)

    def _graph(self, key, inst, Qb):
        """The captured search of `key`, instance `inst` (0 .. NINST - 1): (graph, its query buffer, its outputs,
        the pinned exactness flags, the event recorded after its replay and output copies, the stream it
        is replayed on). Captured on first use, with Qb as the query values of the capture's runs.
        The instances of a key may run at the same time: each has its own buffers (its own graph memory
        pool) and is captured on streams of its own, main branch and side branch, so that the library
        GEMMs of two instances do not share a workspace."""
        gk = (key, inst)
        if gk not in self.graphs:
            _, K, z, nprobe, k, _ = key
            qs = Qb.clone()
            okh = torch.empty((len(Qb),), dtype=torch.bool, pin_memory=True)

            def run():
                outs = self._gpu(qs, K, z, nprobe, k)
                okh.copy_(outs[0], non_blocking=True)  # the flags reach the host inside the graph
                return outs

            side = self._side
            self._side = torch.cuda.Stream(device=qs.device)  # the instance's side branch
            try:
                g, outs = capture(run, stream=torch.cuda.Stream(device=qs.device))
            finally:
                self._side = side
            self.graphs[gk] = (g, qs, outs, okh.numpy(), torch.cuda.Event(), torch.cuda.Stream(device=qs.device))
        return self.graphs[gk]

    def submit(self, Qb, K, z, nprobe, k):
        """Queue the search of one batch and return its ticket without waiting for the GPU. A submit of one
        (B, K, z, nprobe, k) takes the lowest-numbered of its NINST graph instances that has no batch in
        flight, so at most NINST batches of a key are in flight (one more submit raises RuntimeError), and
        a caller that collects each batch before the next submit (search) only ever uses instance 0."""
        Qb = Qb.float().contiguous()
        key = (len(Qb), K, float(z), nprobe, k, self._knobs())
        inst = next((i for i in range(self.NINST) if (key, i) not in self._pending), None)
        if inst is None:
            raise RuntimeError("EngineI8.submit: NINST batches of this shape are in flight; collect one first")
        g, qs, (ok, I, nr, ids, sc, blas), okh, done, st = self._graph(key, inst, Qb)
        cur = torch.cuda.current_stream()
        st.wait_stream(cur)  # the caller's batch, and the instance's last use by the caller, are complete
        with torch.cuda.stream(st):
            qs.copy_(Qb)
            g.replay()
            I, nr, ids, sc = _fresh(I, nr, ids, sc)  # the caller's copies, queued behind the replay
            done.record()
        Qb.record_stream(st)
        for t in (I, nr, ids, sc):  # made on the instance's stream, used on the caller's
            t.record_stream(cur)
        self._pending.add((key, inst))
        return (key, inst, I, nr, ids, sc)

    def collect(self, ticket, ret_scores=False):
        """Wait for a submitted batch, recompute its flagged queries, and return what search returns."""
        key, inst, I, nr, ids, sc = ticket
        if (key, inst) not in self._pending:
            raise RuntimeError("EngineI8.collect: this ticket was already collected")
        g, qs, outs, okh, done, st = self.graphs[(key, inst)]
        blas = outs[5]
        done.synchronize()
        if not okh.all():
            bad = np.nonzero(~okh)[0].astype(np.int64)
            nb = len(bad)
            self.nbad += nb
            fg, sel, (a, b, c, s, ok2) = self._fallback_graph(key, inst, qs, blas, padded_rows(nb))
            cur = torch.cuda.current_stream()
            st.wait_stream(cur)
            with torch.cuda.stream(st):  # behind the instance's own work, beside the other instance's
                sel.copy_(torch.from_numpy(np.concatenate([bad, np.full(padded_rows(nb) - nb, bad[-1], np.int64)])))
                fg.replay()
                bd = torch.from_numpy(bad).to(qs.device)
                I[bd], nr[bd], ids[bd], sc[bd] = a[:nb], b[:nb], c[:nb], s[:nb]
            cur.wait_stream(st)
            self.nbad2 += int((~ok2[:nb]).sum())
        # the instance is free again only now: its flags and fallback inputs are read above
        self._pending.discard((key, inst))
        return (I, nr, ids, sc) if ret_scores else (I, nr, ids)

    def warm_fallbacks(self, B, K, z, nprobe, k, upto=64):
        """Capture the fallback graphs of 1, 2, 4, ... `upto` flagged rows of an already searched (B, K, z,
        nprobe, k), for every graph instance (NINST), ahead of time, so that no later search pays a capture (tens
        of milliseconds)."""
        key = (B, K, float(z), nprobe, k, self._knobs())
        have = [i for i in range(self.NINST) if (key, i) in self.graphs]
        if not have:
            raise KeyError("warm_fallbacks: search this (B, K, z, nprobe, k) once first")
        if self._pending:
            raise RuntimeError("warm_fallbacks: collect the submitted batches first")
        seed = self.graphs[(key, have[0])][1]
        for inst in range(self.NINST):
            g, qs, outs, _, _, _ = self._graph(key, inst, seed)
            qs.copy_(seed)
            g.replay()  # the captures' warm-up runs read the main graph's outputs
            nbp = 1
            while nbp <= upto:
                self._fallback_graph(key, inst, qs, outs[5], nbp)
                nbp *= 2

    def _fallback_graph(self, key, inst, qs, blas, nbp):
        """The captured fallback of nbp rows gathered (by `sel`) from instance inst's query and BLAS
        buffers; it is replayed after that instance's replay (and at most the other instance's), so those
        hold the batch's values."""
        fkey = ("fb", key, inst, nbp)
        if fkey not in self.graphs:
            sel = torch.zeros(nbp, dtype=torch.int64, device=qs.device)
            _, K, z, nprobe, k, _ = key

            def run():
                a = [t.index_select(0, sel) for t in (qs,) + tuple(blas)]
                return self._fallback_core(a[0], K, z, nprobe, k, *a[1:])

            g, outs = capture(run)
            self.graphs[fkey] = (g, sel, outs)
        return self.graphs[fkey]

    def _fallback(self, Qb, K, z, nprobe, k, zq=None, QM=None, Zq=None):
        """Flagged queries again with r = K, n1 over 1.5K blocks, M = 65,536, an fp32 LUT and every
        candidate scored (throughput/enginei8.py:112-120). zq / QM / Zq: the rows of the main pass's BLAS
        products for these queries (recomputed when not given)."""
        I, reads, ids, scores, ok = self._fallback_core(Qb, K, z, nprobe, k, zq, QM, Zq)
        self.nbad2 += int((~ok).sum())
        return I, reads, ids, scores

    def _fallback_core(self, Qb, K, z, nprobe, k, zq=None, QM=None, Zq=None):
        """The fallback without host synchronisation (capturable); also returns its own exactness flags."""
        qp = _lib.query_prep(Qb, self.Vr, self.s1["c"], zq)
        q8, qs, QC, Qh, _ = qp
        if QM is None:
            QM = self._plain_qm(Qh)
        # the reference's fallback routes without PROJ or ROUTE16 (throughput/enginei8.py:110-112)
        probe = _lib.route_topk(QM, nprobe) if self.NROUTE else _lib.route_topk_scaled(QM, self.s1["inv_mnorm"], nprobe)
        if Zq is None:
            Zq = s2lut.rotate(self.code, Qh)
        pos, ok = self.stage1_i8(Qb, QM, probe, K, rho_override=1.0, M_override=65536, qp=qp, delta=None)
        ok2, I, reads, ids, scores = self._finish(Qb, Zq, QC, pos, ok, K, z, k, half=False, ncnt=None)
        return I, reads, ids, scores, ok

    def trace(self, Qb, K, z, nprobe, k):
        """Eager run of one batch that returns every intermediate (for parity tests and profiling)."""
        self._check_knobs()
        Qb = Qb.float().contiguous()
        qp = _lib.query_prep(Qb, self.Vr, self.s1["c"], canonical=self.CANON_Z)
        q8, qs, QC, Qh, zq = qp
        QM, probe = self._route(Qh, QC, nprobe)
        pos, ok = self.stage1_i8(Qb, QM, probe, K, qp=qp, delta=self.DELTA, kd=k - 1)
        half = self.LUTF and self.LUTH
        ncnt = self._ncnt if self.DELTA is not None else None
        Zq = s2lut.rotate(self.code, Qh)
        tables = _lib.lut_build(Zq, self.code["TS"], half)  # returned for inspection; the scorer builds its own
        pre = _lib.ZqTables(Zq, half)
        pos1 = pos
        if self.K2 is not None and self.K2 < K:
            e_all, _ = s2lut.score_lut(self.code, QC, pos, pre, None, nt=min(self.NT, len(self.code["TS"])))
            cntK = torch.full((pos.shape[0],), K, dtype=torch.int32, device=pos.device)
            pos = _lib.select(e_all.contiguous(), pos.contiguous(), cntK, self.K2, 0, None)[0]
            if ncnt is not None:
                ncnt = ncnt.clamp(max=self.K2).contiguous()
        est, sd = s2lut.score_lut(self.code, QC, pos, pre, ncnt)
        ids, I, scores, reads = _lib.refine(est, sd, pos, self.s1["order"], self.H, Qb, z, k)
        return dict(q8=q8, qs=qs, QC=QC, Qh=Qh, z=zq, QM=QM, probe=probe, bm=self._bm, n1=self._n1, M=self._M,
                    t0=self._t0, cnt=self._cnt, bval=self._bval, bpos=self._bpos, pos=pos, pos1=pos1, est1=self._est1, ok=ok,
                    ncnt=self._ncnt, Zq=Zq, L=tables[0], qsum=tables[1], qn2=tables[2], est=est, sd=sd, ids=ids, I=I,
                    scores=scores, reads=reads)

    def gpu_bytes(self):
        """Bytes per vector kept on the GPU by the search tables (int8 code + scale, record, id), as the
        reference's memory accounting (throughput/enginei8.py:121-122)."""
        N = self.Z.shape[0]
        per = self.Z.shape[1] + 4 + self.code["RB"] + 4
        tables = (self.meansN.numel() * 2 + self.mnorm.numel() * 4 + self.Vr.numel() * 4 +
                  self.code["VP16"].numel() * 2)
        return per + tables / N
