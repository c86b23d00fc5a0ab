"""SpaceX on MI355X: the host-resident default engine (host_resident/space_x.py:13-78, benchmark config 5).

Every per-vector array lives in pinned host memory: the trellis words and scales, the packed stage-2
records, and the fp16 rows (kept in sorted order, so no id table is needed on the GPU; ids are mapped
on the host, as the reference's ids_host variant does). The GPU keeps only shared tables: the cell
means for routing and the pair constants, W1, the stage-2 rotation VP, the trellis table, the cell
offsets and the static work list (plus two stage-1 staging slots with copy staging). The reference's two
switches are kept (space_x.py:19-36):
  proj: the means projected on the stage-1 basis, meansR = fp16((m_c - c) @ W1) [NC, R], with
        QM = fp16(Qr) @ meansR.T and the pair term and routing key adding <q, c>. It is exact only when
        the cell means lie in the span of W1 (true of the reference's embeddings, not of isotropic
        cluster centres), so it is off by default;
  vp16: W1 and VP in fp16, with Qr = f32(fp16(Qb) @ W1h) and Zq = f32(fp16(Qb) @ VP16).
The default (proj off, vp16 on, zero-copy stage 1) stays under 8 B per vector at 1.28M vectors, and so
does copy staging with its 16,384-row chunks.

Stage 1 has two stagings of its trellis words and scales (the same results either way):
  "zero-copy" (the default, and the reference's placement: space_x.py:23 hands the pinned arrays to the
        scan): one fvs_tr_scan launch per pass over the whole work list reads the words and scales from
        pinned memory over PCIe, each item's rows once, with consecutive lanes on consecutive dwords;
  "copy": the index is cut into cell-aligned chunks of about CHUNK rows, each stored in pinned memory as
        one contiguous block (its rows' trellis words, then their scales, padded to 16 bytes); a side
        stream copies chunk i+1's block into the free one of two staging slots with one hipMemcpyAsync
        while the main stream scans chunk i (fvs_tr_scan_streamed).
Stage 2 and stage 3 read their records and rows zero-copy from pinned memory. Results equal EngineS's
with the projected-means routing.
"""
import numpy as np
import torch

from . import _lib, index, s2lut
from .engine_cell import EngineS


def _pin(t):
    out = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
    out.copy_(t.cpu())
    return out


class SpaceX(EngineS):
    CHUNK = 16384  # rows per staged stage-1 chunk

    def __init__(self, s1, code, H16, proj=False, vp16=True, staging="zero-copy"):
        if staging not in ("zero-copy", "copy"):
            raise ValueError("SpaceX: staging is 'zero-copy' or 'copy'")
        self.staging = staging
        s2lut.prepare_u(code)
        if "VP" not in code:
            raise ValueError("SpaceX needs a Lloyd-Max tiered code (s2lut.encode_lloyd)")
        dev = s1["words"].device
        self.order_np = s1["order"].cpu().numpy()
        order = s1["order"].long()
        self.Hs = _pin(H16[order.to(H16.device)])
        self.proj, self.vp16 = proj, vp16
        VP = code["VP"].to(dev)
        self.code = dict(TS=code["TS"], rec=_pin(code["rec"]), RB=code["RB"], soff=code["soff"], toff=code["toff"],
                         cb=code["cb"].to(dev), VP=VP.half().contiguous() if vp16 else VP, kind=code.get("kind"))
        W1 = s1["W1"].to(dev)
        means = (((s1["means16"].float() - s1["c"]) @ W1).half() if proj else s1["means16"]).contiguous()
        self.s1 = dict(off=np.asarray(s1["off"]), off_t=s1["off_t"].to(dev), c=s1["c"].to(dev),
                       W1=W1.half().contiguous() if vp16 else W1, tab=s1["tab"].to(dev), L=int(s1["L"]),
                       inv_mnorm=s1["inv_mnorm"].float().to(dev), means=means)
        self.W1, self.inv_mnorm, self.means = self.s1["W1"], self.s1["inv_mnorm"], means
        self.N = int(s1["words"].shape[0])
        self.Wd = int(s1["words"].shape[1])
        self.blocks, self.MB = index.static_blocks(self.s1["off_t"], self.BN)
        self.H = self.Hs
        self.graphs = {}
        self.nbad = 0
        if staging == "copy":
            self._chunks()
            self._stage_host(s1["words"], s1["scale1"])
            self.side = torch.cuda.Stream()
            self.slots = [torch.empty((self._block_bytes(self.chunk_rows),), dtype=torch.uint8, device=dev)
                          for _ in range(2)]
        else:
            self.chunks, self.slots = [], []
            self.words_h, self.scale1_h = _pin(s1["words"]), _pin(s1["scale1"])
        self.copied_bytes = 0
        self.copy_events = []
        self.phase_events = None  # when a list, _run records (name, event) at each stage boundary
        self._cus = torch.cuda.get_device_properties(dev).multi_processor_count
        self._np = 1  # n_p of the search in progress (sets the query-split of the chunk scans)

    def _block_bytes(self, rows):
        """Bytes of one chunk's block: rows x Wd int32 words, then rows fp16 scales, padded to 16 bytes."""
        return rows * 4 * self.Wd + -(-rows * 2 // 16) * 16

    def _stage_host(self, words, scale1):
        """The stage-1 arrays in pinned memory, one contiguous block per chunk (words, then scales)."""
        offs, at = [], 0
        for r0, r1, _, _ in self.chunks:
            offs.append(at)
            at += self._block_bytes(r1 - r0)
        self.block_off = offs
        self.chunk_tab = np.array([(r0, r1, i0, i1, o) for (r0, r1, i0, i1), o in zip(self.chunks, offs)], np.int64)
        self.stage_h = torch.empty((at,), dtype=torch.uint8, pin_memory=True)
        w, sc = words.cpu(), scale1.cpu()
        for (r0, r1, _, _), o in zip(self.chunks, offs):
            n = r1 - r0
            self.stage_h[o:o + 4 * self.Wd * n] = w[r0:r1].contiguous().view(torch.uint8).reshape(-1)
            self.stage_h[o + 4 * self.Wd * n:o + 4 * self.Wd * n + 2 * n] = sc[r0:r1].contiguous().view(torch.uint8)

    def _params(self, K, nprobe, rho_override=None, M_override=None):
        NC = len(self.s1["off"]) - 1
        # the reference's size: at batch 2000 a larger buffer (index.emit_buffer) avoids most overflow
        # fallbacks but measured no faster, the batch being bound by the zero-copy stage-2 reads
        M = M_override or self.M or index.emit_buffer(None, K)
        beta, rho = (1.1, 0.75) if K <= 400 else (0.7, 0.5)
        if rho_override:
            beta, rho = 1.5, rho_override
        n1 = min(max(int(np.ceil(beta * K / (self.N / NC / self.BN + 1))), 1), nprobe)
        return M, n1, int(np.ceil(rho * K))

    def _chunks(self):
        """Cell-aligned chunks [(row0, row1, item0, item1)] of at most chunk_rows rows."""
        off = self.s1["off"].astype(np.int64)
        sizes = np.diff(off)
        self.chunk_rows = int(max(self.CHUNK, sizes.max()))
        pcell = self.blocks[0].cpu().numpy()
        first_item = np.searchsorted(pcell, np.arange(len(off)))  # first item of each cell (items are cell-sorted)
        chunks, c0 = [], 0
        NC = len(off) - 1
        while c0 < NC:
            c1 = c0
            while c1 < NC and off[c1 + 1] - off[c0] <= self.chunk_rows:
                c1 += 1
            c1 = max(c1, c0 + 1)
            chunks.append((int(off[c0]), int(off[c1]), int(first_item[c0]), int(first_item[c1])))
            c0 = c1
        self.chunks = [c for c in chunks if c[3] > c[2]]

    timing = False  # when set, every chunk copy is bracketed by events (copy_events) for the PCIe rate

    def _nsplit(self, items, B, NC):
        """Waves per item of a chunk's scan: a chunk holds a few hundred items, so its launch would leave most
        of the GPU idle at one wave per item; its queries per cell (B x n_p / NC on average, at least 16 per
        part) are split over up to 8 waves instead (the same results)."""
        qpc = B * self._np / max(NC, 1)
        fill = -(-32 * self._cus // max(items, 1))  # parts for about eight workgroups per CU
        return int(max(1, min(8, fill, qpc // 16)))

    def _scan_streamed(self, mode, Qr, pr, **kw):
        """One stage-1 pass. Zero-copy staging: one scan over the whole work list reading pinned memory.
        Copy staging: every chunk copied on the side stream, overlapped with the scans; one library call
        (fvs_tr_scan_streamed) queues every chunk's copy and scan; with `timing` set, the same steps are
        queued from here with every copy bracketed by timing events."""
        if self.staging == "zero-copy":
            _lib.tr_scan(mode, self.blocks, Qr, pr, self.words_h, self.scale1_h, self.s1["tab"], self.s1["L"],
                         half=True, **kw)
            self.copied_bytes += self.N * (4 * self.Wd + 2)
            return
        nsplit = self._nsplit(max(i1 - i0 for _, _, i0, i1 in self.chunks), Qr.shape[0], pr[2].numel())
        if not self.timing:
            _lib.tr_scan_streamed(mode, self.chunk_tab, self.stage_h, self.slots, self.side, self.blocks, Qr, pr,
                                  self.s1["tab"], self.s1["L"], self.Wd, half=True, nsplit=nsplit, **kw)
            self.copied_bytes += int(sum(self._block_bytes(r1 - r0) for r0, r1, _, _ in self.chunks))
            return
        main = torch.cuda.current_stream()
        self.side.wait_stream(main)  # the slots' previous contents have been scanned
        done = [None, None]
        for i, (r0, r1, i0, i1) in enumerate(self.chunks):
            slot = i % 2
            n = r1 - r0
            nb = self._block_bytes(n)
            buf = self.slots[slot]
            with torch.cuda.stream(self.side):
                if done[slot] is not None:
                    self.side.wait_event(done[slot])
                if self.timing:
                    a = torch.cuda.Event(enable_timing=True)
                    a.record(self.side)
                o = self.block_off[i]
                buf[:nb].copy_(self.stage_h[o:o + nb], non_blocking=True)
                ready = torch.cuda.Event(enable_timing=self.timing)
                ready.record(self.side)
                if self.timing:
                    self.copy_events.append((a, ready, nb))
            self.copied_bytes += nb
            main.wait_event(ready)
            w = buf[:4 * self.Wd * n].view(torch.int32).view(n, self.Wd)
            s = buf[4 * self.Wd * n:4 * self.Wd * n + 2 * n].view(torch.float16)
            blocks = tuple(b[i0:i1] for b in self.blocks)
            # fp16 operands at every batch size: the reference's host-resident engine always runs
            # search_static (host_resident/space_x.py:15,42)
            _lib.tr_scan(mode, blocks, Qr, pr, w, s, self.s1["tab"], self.s1["L"], row0=r0, half=True, nsplit=nsplit,
                         **kw)
            ev = torch.cuda.Event()
            ev.record(main)
            done[slot] = ev

    def stage1(self, Qr, QM, probe, K, rho_override=None, M_override=None, QC=None):
        NC = len(self.s1["off"]) - 1
        B = Qr.shape[0]
        dev = Qr.device
        M, n1, r = self._params(K, probe.shape[1], rho_override, M_override)
        scratch = _lib.pairs_scratch(B, NC, dev)
        pr, prn = _lib.pairs2(probe, n1, NC, QM, None, scratch, qadd=QC)
        bm = torch.empty((B, n1, self.MB), dtype=torch.float32, device=dev)
        self._mark("pair lists")
        self._scan_streamed(0, Qr, pr, bm=bm, MB=self.MB, n1=n1)
        self._mark("first pass (streamed)")
        cnt = torch.empty((B,), dtype=torch.int32, device=dev)  # zeroed by the threshold kernel
        t0 = _lib.threshold(bm, probe, self.s1["off_t"], n1, self.MB, r, cnt)
        bval = torch.empty((B, M), dtype=torch.float32, device=dev)
        bpos = torch.empty((B, M), dtype=torch.int32, device=dev)
        pr = prn
        self._mark("threshold")
        self._scan_streamed(1, Qr, pr, t0=t0, cnt=cnt, bval=bval, bpos=bpos, CAP=M)
        self._mark("emit pass (streamed)")
        pos, est1, ok, _ = _lib.select(bval, bpos, cnt, K, 0, None)
        self._bm, self._t0, self._cnt, self._bval, self._bpos, self._n1, self._M = bm, t0, cnt, bval, bpos, n1, M
        return pos, ok.view(torch.bool)  # the kernel writes 0 / 1 bytes: a view, no conversion kernel

    def _dense(self, Qb):
        """The dense products (space_x.py:33-38): Qr = Qb @ W1 and Zq = Qb @ VP (f32, or f32 of the fp16
        products with vp16), QC = <Qb, c>, QM = fp16(Qb) @ means16.T (fp16), or fp16(Qr) @ meansR.T with proj
        (the pair term and routing key then add QC)."""
        Qh = Qb.half()
        if self.vp16:
            Qr = (Qh @ self.W1).float().contiguous()
            Zq = (Qh @ self.code["VP"]).float().contiguous()
        else:
            Qr = (Qb @ self.W1).contiguous()
            Zq = (Qb @ self.code["VP"]).contiguous()
        _, _, QC, _, _ = _lib.query_prep(Qb, None, self.s1["c"], Qr)
        QM = ((Qr.half() if self.proj else Qh) @ self.means.T).contiguous()
        return Qr, QC, QM, Zq

    def _finish(self, Qb, QC, Zq, pos, z, k):
        est, sd = _lib.tiered_score(pos, QC, Zq, self.code)
        self._est, self._sd = est, sd
        return _lib.refine(est, sd, pos, None, self.Hs, Qb, z, k)

    def _mark(self, name):
        if self.phase_events is not None:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record()
            self.phase_events.append((name, ev))

    def _run(self, Qb, K, z, nprobe, k, rho_override=None, M_override=None, dense=None):
        self._mark("start")
        Qr, QC, QM, Zq = dense if dense is not None else self._dense(Qb)
        qadd = QC if self.proj else None
        self._np = nprobe
        probe = _lib.route_topk_scaled(QM, self.inv_mnorm, nprobe, qadd=qadd)
        self._mark("dense products and routing")
        pos, ok = self.stage1(Qr, QM, probe, K, rho_override, M_override, QC=qadd)
        self._mark("stage 1 (streamed)")
        est, sd = _lib.tiered_score(pos, QC, Zq, self.code)
        self._est, self._sd = est, sd
        self._mark("stage 2 (records zero-copy)")
        ids, I, scores, reads = _lib.refine(est, sd, pos, None, self.Hs, Qb, z, k)
        self._mark("refine (rows zero-copy)")
        return ok, I, reads, ids, scores, (Qr, QC, QM, Zq)

    FALLBACK_M = 1 << 20  # emit buffer of the flagged queries' second pass (host_resident/space_x.py:65)

    def search(self, Qb, K, z, nprobe, k, ret_scores=False, sorted_ids=False):
        """(I, reads, cand_ids) (+ scores): ids mapped to the original ids on the host (numpy -> torch CPU
        tensors), as SpaceX.run does (host_resident/space_x.py:71-78); sorted_ids keeps sorted positions.
        Flagged queries run the same pass again with a 1 << 20-entry buffer (space_x.py:58-70), which holds
        every row above the threshold of a query whose count overflowed the main buffer: its top K no longer
        depends on the order the rows were emitted in."""
        Qb = Qb.float().contiguous()
        ok, I, nr, ids, sc, dense = self._run(Qb, K, z, nprobe, k)
        if not bool(ok.all()):
            bad = torch.nonzero(~ok).flatten()
            self.nbad += len(bad)
            sub = tuple(t[bad].contiguous() for t in dense)
            _, a, b, c, s, _ = self._run(Qb[bad], K, z, nprobe, k, M_override=self.FALLBACK_M, dense=sub)
            I, nr, ids, sc = I.clone(), nr.clone(), ids.clone(), sc.clone()
            I[bad], nr[bad], ids[bad], sc[bad] = a, b, c, s
        if not sorted_ids:
            I = torch.from_numpy(self.order_np[I.cpu().numpy()])
            ids = torch.from_numpy(self.order_np[ids.cpu().numpy()])
        return (I, nr, ids, sc) if ret_scores else (I, nr, ids)

    def trace(self, Qb, K, z, nprobe, k):
        Qb = Qb.float().contiguous()
        ok, I, reads, ids, scores, (Qr, QC, QM, Zq) = self._run(Qb, K, z, nprobe, k)
        return dict(Qr=Qr, QC=QC, QM=QM, Zq=Zq, pos=None, ok=ok, I=I, ids=ids, scores=scores, reads=reads,
                    cnt=self._cnt, t0=self._t0, est=self._est, sd=self._sd)

    def gpu_bytes(self):
        """Bytes per vector resident on the GPU (host_resident/space_x.py:80-88): every device tensor the
        engine holds (tables, work list, staging slots), divided by N."""
        seen, tot = set(), 0

        def walk(x):
            nonlocal tot
            if isinstance(x, torch.Tensor):
                if x.is_cuda and x.untyped_storage().data_ptr() not in seen:
                    seen.add(x.untyped_storage().data_ptr())
                    tot += x.untyped_storage().nbytes()
            elif isinstance(x, dict):
                for v in x.values():
                    walk(v)
            elif isinstance(x, (list, tuple)):
                for v in x:
                    walk(v)

        walk(self.s1)
        walk(self.code)
        walk(self.blocks)
        walk(self.slots)
        return tot / self.N
