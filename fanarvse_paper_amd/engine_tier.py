"""EngineS with its fp16 rows on an NVMe drive: the row tier of the reference's Engine12
(src/engine3.py:204-233, "lean + NVMe").

Stages 1 and 2 run on the GPU as in EngineS. Stage 3 is split: fvs_classify flags the ambiguous
candidates, their ids come back to the host in one synchronisation, a reader thread fetches those rows
from the tier file (tier.RowTier: io_uring or a pread pool, O_DIRECT) into pinned memory, and
fvs_refine_rows scores them and takes the final top-k. The results are those of EngineS with the same
rows in GPU memory, bit for bit. run() overlaps the reads of one batch with the GPU stages of the next,
as Engine12.run does.

    tier.write_tier(path, X16)                       # once: rows in id order, 4096-byte slots
    E = EngineSTier(s1, code, tier.RowTier(path, d))
    I, reads, cand_ids = E.search(Qb, K, z, nprobe, k)
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _lib
from .engine_cell import EngineS


class EngineSTier(EngineS):
    def __init__(self, s1, code, tier):
        super().__init__(s1, code, H=None)
        self.tier = tier
        self.pool = ThreadPoolExecutor(1)
        self.rows_read = 0

    def _gpu_part(self, Qb, K, z, nprobe, k):
        """Stages 1-2 and the classification on the GPU; starts the tier read of the ambiguous rows."""
        Qb = Qb.float().contiguous()
        Qr, QC, QM, Zq = self._dense(Qb)
        probe = _lib.route_topk_scaled(QM, self.inv_mnorm, nprobe)
        pos, ok = self.stage1(Qr, QM, probe, K, half=len(Qb) > self.TINY)
        okh = ok.cpu().numpy()
        if not okh.all():  # flagged queries: stage 1 again with the fallback's settings (src/engine_cell.py:98-101)
            bad = torch.from_numpy(np.nonzero(~okh)[0]).to(Qb.device)
            self.nbad += len(bad)
            pos[bad], _ = self.stage1(Qr[bad].contiguous(), QM[bad].contiguous(), probe[bad].contiguous(), K,
                                      rho_override=1.0, M_override=65536, half=True)
        est, sd = _lib.tiered_score(pos, QC, Zq, self.code)
        ids, flag, namb, aslot = _lib.classify(est, sd, pos, self.s1["order"], z, k)
        aid = ids.gather(1, aslot.long())
        nh, ah = namb.cpu().numpy(), aid.cpu().numpy()
        want = np.concatenate([ah[q, :nh[q]] for q in range(len(nh))]).astype(np.int64)
        roff = torch.from_numpy(np.concatenate([[0], np.cumsum(nh)[:-1]]).astype(np.int64)).to(Qb.device)
        buf = torch.empty((max(len(want), 1), Qb.shape[1]), dtype=torch.float16, pin_memory=True)
        fut = self.pool.submit(self.tier.read_into, want, buf[:len(want)])
        self.rows_read += len(want)
        return Qb, est, flag, aslot, namb, roff, ids, buf, fut

    def _finish_part(self, part, k):
        Qb, est, flag, aslot, namb, roff, ids, buf, fut = part
        fut.result()
        rows = buf.to(Qb.device, non_blocking=True)  # the caching host allocator keeps buf until the copy ends
        I, scores, reads = _lib.refine_rows(est, flag, aslot, namb, roff, ids, rows, Qb, k)
        return I, reads, ids, scores

    def search(self, Qb, K, z, nprobe, k, ret_scores=False):
        """(I [B,k], reads [B], cand_ids [B,K]) (+ scores), as EngineS.search."""
        I, reads, ids, sc = self._finish_part(self._gpu_part(Qb, K, z, nprobe, k), k)
        return (I, reads, ids, sc) if ret_scores else (I, reads, ids)

    def search_host(self, Qb, K, z, nprobe, k):
        return self.search(Qb, K, z, nprobe, k)[0].cpu().numpy().astype(np.int64)

    def run(self, Q, K, z, nprobe, k, B=500):
        """All queries in batches of B, the tier reads of batch i overlapping the GPU stages of batch
        i + 1 (src/engine3.py:225-233). Returns numpy (I, reads, cand_ids)."""
        out, prev = [], None
        for s in range(0, len(Q) + B, B):
            cur = self._gpu_part(Q[s:s + B], K, z, nprobe, k) if s < len(Q) else None
            if prev is not None:
                I, reads, ids, _ = self._finish_part(prev, k)
                out.append((I.cpu().numpy(), reads.cpu().numpy(), ids.cpu().numpy()))
            prev = cur
        return tuple(np.concatenate([o[j] for o in out]) for j in range(3))
