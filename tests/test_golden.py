"""The committed fixture tests/golden/tiny_search.npz (written by tests/golden/make_golden.py from the CPU
oracle): the oracle must still reproduce it on the CPU, and the GPU kernels, called stage by stage
through the C ABI on the fixture's inputs, must reproduce it bit for bit."""
import os

import numpy as np
import pytest

from fanarvse_paper_amd import index as _index

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_search.npz")


@pytest.fixture(scope="module")
def G():
    with np.load(PATH, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _idx(G):
    TS = [tuple(int(v) for v in t) for t in G["TS"]]
    return dict(order=G["order"], off=G["off"], mnorm=G["mnorm"], c=G["c"], Vr=None, meansN=None, VP16=None,
                Z=G["Zc"], zs=G["zs"], TS=TS, deltas=G["deltas"], toff=G["toff"], soff=int(G["soff"]), rec=G["rec"],
                H=G["H"])


def _bits(a):
    a = np.asarray(a)
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_oracle_reproduces_golden(G, oracle_mod):
    K, nprobe, k, M = (int(v) for v in G["params"])
    rho, delta = (float(v) for v in G["knobs"])
    out = oracle_mod.pipeline(_idx(G), G["Q"], K, float(G["zval"]), nprobe, k,
                              knobs=dict(MSZ=M, RHO=rho, DELTA=delta, LUTF=True, LUTH=True),
                              QM16=G["QM"], Zq16=G["Zq"], zq=G["zq"], fallback=False)
    for name in ["q8", "qs", "qc", "probe", "bm", "t0", "cnt", "pos", "est1", "ok", "ncnt", "L", "qsum", "qn2", "est",
                 "sd", "ids", "I", "scores", "reads"]:
        assert np.array_equal(_bits(out[name]), _bits(G["out_" + name])), name


@pytest.mark.gpu
def test_gpu_reproduces_golden(G):
    import torch

    from fanarvse_paper_amd import _lib

    dev = "cuda"
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    K, nprobe, k, M = (int(v) for v in G["params"])
    rho, delta = (float(v) for v in G["knobs"])
    Q, z = t(G["Q"]), float(G["zval"])
    B, d = Q.shape
    Zc, zs = t(G["Zc"]), t(G["zs"])
    NC = len(G["off"]) - 1
    off_t = t(G["off"].astype(np.int32))
    QM = t(G["QM"]).view(torch.float16)
    Zq = t(G["Zq"]).view(torch.float16)
    mnorm = t(G["mnorm"])
    TS = [tuple(int(v) for v in tt) for tt in G["TS"]]
    code = dict(TS=TS, rec=t(G["rec"]), soff=int(G["soff"]), toff=[int(v) for v in G["toff"]],
                deltas={b: float(G["deltas"][i]) for i, (_, _, b) in enumerate(TS)})
    q8, qs, qc, qh, _ = _lib.query_prep(Q, torch.empty((d, Zc.shape[1]), device=dev), t(G["c"]), z=t(G["zq"]))
    probe = _lib.route_topk(QM, nprobe)
    n1, r = int(G["out_n1"]), int(G["out_r"])
    _, MB = _index.static_blocks(off_t)
    blocks = _index.static_chunks(off_t)
    pr = _lib.pairs(probe, n1, NC, QM, mnorm)
    bm = torch.full((B, n1, MB), -1e30, device=dev)
    _lib.i8_scan(0, blocks, q8, qs, pr, Zc, zs, bm=bm, MB=MB, n1=n1)
    t0 = _lib.threshold(bm, probe, off_t, n1, MB, r)
    cnt = torch.zeros((B,), dtype=torch.int32, device=dev)
    bval = torch.empty((B, M), device=dev)
    bpos = torch.empty((B, M), dtype=torch.int32, device=dev)
    pr = _lib.pairs(probe, nprobe, NC, QM, mnorm)
    # emit items of at most 128 rows on global blocks (four per item): any grouping gives the same sets
    _lib.i8_scan(1, _index.static_chunks(off_t, 32, 4), q8, qs, pr, Zc, zs, t0=t0, cnt=cnt, bval=bval, bpos=bpos,
                 CAP=M)
    pos, est1, ok, ncnt = _lib.select(bval, bpos, cnt, K, k - 1, delta)
    pre = _lib.lut_build(Zq, TS, True)
    est, sd = _lib.lut_score(pos, qc, pre, code, ncnt)
    ids, I, scores, reads = _lib.refine(est, sd, pos, t(G["order"]), t(G["H"]).view(torch.float16), Q, z, k)
    torch.cuda.synchronize()
    c = lambda x: x.cpu().numpy()
    got = dict(q8=c(q8), qs=c(qs), qc=c(qc), probe=c(probe), t0=c(t0), cnt=c(cnt), pos=c(pos), est1=c(est1),
               ok=c(ok), ncnt=c(ncnt), L=c(pre[0].view(torch.int16)).view(np.uint16), qsum=c(pre[1]), qn2=c(pre[2]),
               est=c(est), sd=c(sd), ids=c(ids), I=c(I), scores=c(scores), reads=c(reads))
    for name, v in got.items():
        assert np.array_equal(_bits(v), _bits(G["out_" + name])), name
    # block maxima: entries of blocks a cell does not have are left untouched (-1e30 fill)
    assert np.array_equal(_bits(c(bm)), _bits(G["out_bm"]))
    # emitted sets (order-free); the fixture is sized so that no query overflows its buffer (cnt <= M),
    # since past M the buffer keeps an arbitrary subset (the append order is atomic)
    cn = c(cnt)
    assert np.all(cn <= M)
    emitted = np.concatenate([np.sort(c(bpos)[q, :int(cn[q])]) for q in range(B)])
    assert np.array_equal(emitted, G["out_emitted"])
