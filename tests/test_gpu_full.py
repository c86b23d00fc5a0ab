"""Every BASELINE configuration at its real workload on the GPU, against the CPU oracle.

For each configuration the index is built at full size and the HIP path runs at the configuration's
batch; then:
  * a sample of queries (spread over the batch) goes through the oracle's whole pipeline with the GPU's
    dense products as shared inputs, and the final ids, exact-read counts and candidate ids must be
    bit-identical (fallback included);
  * on every query of the batch (the trellis engines: a large sample), the emit count equals the
    oracle's #{probed rows : est >= t0} for the GPU's own threshold t0 -- the premise of Lemma 2
    (paper/main.tex:206-213), which then makes the top-K of the buffer the exact top-K of the probed rows
    -- and the first-pass block maxima and t0 are bit-exact;
  * recall against the exact ground truth.
Config 1 (the CPU path) has no GPU workload; its oracle run is a bench.py figure.
Sizes: config 2 and 3 = 1M x 1536 (NC 4096), config 4 = 2.25M x 768 (NC 8192, k = 100), config 5 =
1.28M x 768 host-resident (NC 4096)."""
import gc

import numpy as np
import pytest
import torch

from fanarvse_paper_amd import datagen, index, metrics, trellis
from fanarvse_paper_amd.engine_cell import EngineS
from fanarvse_paper_amd.engine_host import SpaceX
from fanarvse_paper_amd.enginei8 import EngineI8

pytestmark = pytest.mark.gpu
dev = "cuda"


def npy(t):
    return t.detach().cpu().numpy()


def u16(t):
    return npy(t).view(np.uint16)


def say(msg):
    print(f"\n[gpu full] {msg}", flush=True)


def free():
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def check_i8_config(E, idx, Q, GT, oracle_mod, K, z, nprobe, k, min_recall, nsample=32):
    """EngineI8 at a full-size batch against the oracle (see the module docstring)."""
    B = Q.shape[0]
    I, reads, ids = E.search(Q, K, z, nprobe, k)
    rec = metrics.recall(npy(I), GT, k)
    tr = E.trace(Q, K, z, nprobe, k)
    torch.cuda.synchronize()
    say(f"search done: recall@{k} {rec:.4f}, {E.nbad} flagged; oracle checks")
    q8, qs, probe, QM = npy(tr["q8"]), npy(tr["qs"]), npy(tr["probe"]), u16(tr["QM"])
    M, n1 = tr["M"], tr["n1"]
    MB = oracle_mod.static_blocks(idx["off"])[4]
    # first pass, threshold and the emit count on every query of the batch
    bm = oracle_mod.first_pass(q8, qs, probe[:, :n1], n1, idx["off"], idx["Z"], idx["zs"], QM, idx["mnorm"], MB)
    valid = bm > -1e29  # the entries of blocks each probed cell has (the kernel leaves the others unwritten)
    assert np.array_equal(npy(tr["bm"])[valid].view(np.uint32), bm[valid].view(np.uint32))
    r = E._params(K, nprobe)[2]
    t0 = oracle_mod.threshold(bm, probe, idx["off"], n1, MB, r)
    assert np.array_equal(npy(tr["t0"]).view(np.uint32), t0.view(np.uint32))
    cnt, _, _ = oracle_mod.emit(q8, qs, probe, idx["off"], idx["Z"], idx["zs"], QM, idx["mnorm"], t0, 1)
    assert np.array_equal(npy(tr["cnt"]), cnt)
    ok = npy(tr["ok"]).astype(bool)
    assert np.array_equal(ok, (cnt >= K) & (cnt <= M))
    # the whole pipeline on a sample, fallback included
    sample = np.linspace(0, B - 1, nsample).astype(np.int64)
    if (~ok).any():  # flagged queries first: they exercise the fallback
        sample = np.unique(np.concatenate([np.nonzero(~ok)[0][:8], sample]))
    knobs = dict(MSZ=E.MSZ, RHO=E.RHO, BETA=E.BETA, DELTA=E.DELTA, LUTF=E.LUTF, LUTH=E.LUTH)
    out = oracle_mod.pipeline(idx, npy(Q)[sample], K, z, nprobe, k, knobs=knobs, QM16=QM[sample],
                              Zq16=u16(tr["Zq"])[sample], zq=npy(tr["z"])[sample])
    assert np.array_equal(npy(I)[sample], out["I"])
    assert np.array_equal(npy(reads)[sample], out["reads"])
    assert np.array_equal(npy(ids)[sample], out["cand"])
    assert rec >= min_recall, rec
    return rec


def test_config2_throughput_1Mx1536(oracle_mod):
    """1M x 1536, batch 2000, k = 10, EngineI8 at the bench's operating point
    (n_p = 768, K = 400, M = 4096) and at the reference's final point (n_p = 352, K = 175, M = 3072)."""
    say("config 2: 1M x 1536 data, index (NC 4096), ground truth")
    X = datagen.gen(1_000_000, 1536, 1024, 0.7, seed=0, device=dev)
    Q = datagen.gen(2000, 1536, 1024, 0.7, seed=1, device=dev, dtype=torch.float32)
    GT = npy(datagen.ground_truth(X, Q, 10))
    s1, code, Z, zs, Vr = index.build_index(X, nlist=4096)
    E = EngineI8(s1, code, Z, zs, Vr, H=X)
    idx = oracle_mod.index_from_tables(s1, code, Z, zs, Vr, X)
    for nprobe, K, M, min_rec in ((768, 400, 4096, 0.985), (352, 175, 3072, 0.9)):
        say(f"config 2: n_p={nprobe} K={K} M={M}")
        E.MSZ = M
        E.nbad = 0
        check_i8_config(E, idx, Q, GT, oracle_mod, K, 1.25, nprobe, 10, min_rec)
    del E, idx, X, Q, s1, code, Z, zs, Vr
    free()


def test_config4_largek_2_25Mx768(oracle_mod):
    """2.25M x 768 (4,096 clusters, spectrum 0.5), NC 8192, batch 2000, k = 100,
    K = 1000, M = max(4096, 16 K), z = 2."""
    say("config 4: 2.25M x 768 data, index (NC 8192), ground truth")
    X = datagen.gen(2_250_000, 768, 4096, 0.5, seed=0, device=dev)
    Q = datagen.gen(2000, 768, 4096, 0.5, seed=1, device=dev, dtype=torch.float32)
    GT = npy(datagen.ground_truth(X, Q, 100))
    s1, code, Z, zs, Vr = index.build_index(X, nlist=8192)
    E = EngineI8(s1, code, Z, zs, Vr, H=X)
    E.MSZ = None
    idx = oracle_mod.index_from_tables(s1, code, Z, zs, Vr, X)
    check_i8_config(E, idx, Q, GT, oracle_mod, 1000, 2.0, 768, 100, 0.99, nsample=16)
    del E, idx, X, Q, s1, code, Z, zs, Vr
    free()


def check_trellis_batch(E, idx, Q, oracle_mod, K, z, nprobe, k, **kw):
    Qr, QC, QM, Zq = E._dense(Q)
    out = oracle_mod.tr_pipeline(idx, npy(Q), K, z, nprobe, k, Qr=npy(Qr), QM16=u16(QM), Zq=npy(Zq), **kw)
    return out


def test_config3_latency_1Mx1536(oracle_mod):
    """the trellis default engine on 1M x 1536 (NC 4096), n_p = 256, K = 200, z = 2, at
    batches 1, 16 and 64 (search and the lean search_host), each batch against the oracle; the emit count
    on 512 queries; recall@10 over the 2000 queries."""
    say("config 3: 1M x 1536 data, trellis index (NC 4096), ground truth")
    X = datagen.gen(1_000_000, 1536, 1024, 0.7, seed=0, device=dev)
    Q = datagen.gen(2000, 1536, 1024, 0.7, seed=1, device=dev, dtype=torch.float32)
    GT = npy(datagen.ground_truth(X, Q, 10))
    s1, code = trellis.build_index(X, nlist=4096)
    E = EngineS(s1, code, H=X)
    idx = oracle_mod.trellis_index_from_tables(s1, code, X)
    K, z, nprobe, k = 200, 2.0, 256, 10
    for B, starts in ((1, (0, 777, 1999)), (16, (0, 1000)), (64, (0, 1936))):
        for s in starts:
            say(f"config 3: batch {B} at query {s}")
            Qb = Q[s:s + B].contiguous()
            I, reads, ids = E.search(Qb, K, z, nprobe, k)
            h = E.search_host(Qb, K, z, nprobe, k)
            torch.cuda.synchronize()
            out = check_trellis_batch(E, idx, Qb, oracle_mod, K, z, nprobe, k, M=E._params(K, nprobe, B=B)[0])
            assert np.array_equal(npy(I), out["I"])
            assert np.array_equal(npy(reads), out["reads"])
            assert np.array_equal(npy(ids), out["cand"])
            if B == 1:  # the lean path: a large buffer, fp32 operands in the main pass and the fallback
                out = check_trellis_batch(E, idx, Qb, oracle_mod, K, z, nprobe, k,
                                          M=E._params(K, nprobe, B=1, lean=True)[0], fb_half=False)
            assert np.array_equal(h, out["I"])
    # the emit count against the oracle's estimates on 512 queries (batches of 64)
    for s in range(0, 512, 64):
        Qb = Q[s:s + 64].contiguous()
        tr = E.trace(Qb, K, z, nprobe, k)
        torch.cuda.synchronize()
        Qr, QM = npy(tr["Qr"]), u16(tr["QM"])
        probe = npy(tr["probe"])
        cnt, _, _ = oracle_mod.tr_emit(Qr, probe, idx["off"], idx["words"], idx["scale1"], idx["tab"], idx["L"], QM,
                                       npy(tr["t0"]), 1, half=True)
        assert np.array_equal(npy(tr["cnt"]), cnt)
    I = torch.cat([E.search(Q[i:i + 64], K, z, nprobe, k)[0] for i in range(0, 2000, 64)])
    rec = metrics.recall(npy(I), GT, k)
    say(f"config 3: recall@10 {rec:.4f}")
    assert rec >= 0.82, rec
    del E, idx, X, Q, s1, code
    free()


def test_config5_host_resident_1_28Mx768(oracle_mod):
    """1.28M x 768 with every per-vector array in pinned host memory (SpaceX), batch
    2000, k = 10, n_p = 256, K = 200, z = 2: a sample of 32 queries through the oracle's pipeline on the
    same dense products, the emit count on 256 queries, recall over the batch."""
    say("config 5: 1.28M x 768 data, trellis index (NC 4096), ground truth")
    X = datagen.gen(1_280_000, 768, 1024, 0.7, seed=0, device=dev)
    Q = datagen.gen(2000, 768, 1024, 0.7, seed=1, device=dev, dtype=torch.float32)
    GT = npy(datagen.ground_truth(X, Q, 10))
    s1, code = trellis.build_index(X, nlist=4096)
    idx = oracle_mod.trellis_index_from_tables(s1, code, X)
    idx["Hs"] = npy(X[s1["order"].long()]).view(np.uint16)
    E = SpaceX(s1, code, X)
    del s1, code
    free()
    K, z, nprobe, k = 200, 2.0, 256, 10
    I, reads, ids = E.search(Q, K, z, nprobe, k, sorted_ids=True)
    tr = E.trace(Q, K, z, nprobe, k)
    torch.cuda.synchronize()
    rec = metrics.recall(E.order_np[npy(I)], GT, k)
    say(f"config 5: recall@10 {rec:.4f}, {E.nbad} flagged; oracle checks")
    Qr, QC, QM, Zq = (npy(tr[n]) for n in ("Qr", "QC", "QM", "Zq"))
    sample = np.linspace(0, 1999, 32).astype(np.int64)
    out = oracle_mod.tr_pipeline(idx, npy(Q)[sample], K, z, nprobe, k, Qr=Qr[sample], QM16=QM.view(np.uint16)[sample],
                                 Zq=Zq[sample], proj=E.proj, order=False, half=True)
    assert np.array_equal(npy(I)[sample], out["I"])
    assert np.array_equal(npy(reads)[sample], out["reads"])
    assert np.array_equal(npy(ids)[sample], out["cand"])
    probe = oracle_mod.route_topk_scaled(QM.view(np.uint16)[:256], idx["inv_mnorm"], nprobe)
    cnt, _, _ = oracle_mod.tr_emit(Qr[:256], probe, idx["off"], idx["words"], idx["scale1"], idx["tab"], idx["L"],
                                   QM.view(np.uint16)[:256], npy(tr["t0"])[:256], 1, half=True)
    assert np.array_equal(npy(tr["cnt"])[:256], cnt)
    assert rec >= 0.82, rec
    del E, idx, X, Q
    free()
