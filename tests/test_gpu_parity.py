"""GPU parity: every stage of the gfx950 path against the CPU oracle on the same seeded inputs.

Integer and index results must be bit-exact; so must the floating-point stages, because the kernels
and oracle.c follow one canonical operation order (include/fvs.h). The three dense products (the
fp32 projection z = Q @ Vr, the fp16 routing scores QM and the fp16 rotated tier queries Zq) come from
the GPU's BLAS and are handed to the oracle as shared inputs; their own accuracy is checked against
float64 (one rounding of the output plus fp32 accumulation).
"""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import datagen, index, metrics
from fanarvse_paper_amd.enginei8 import EngineI8

pytestmark = pytest.mark.gpu

K, Z_, NPROBE, KK = 175, 1.25, 24, 10


def u16(t):
    return t.detach().cpu().numpy().view(np.uint16)


def npy(t):
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def env(oracle_mod):
    print("\n[gpu parity] building N=30000 d=768 NC=128 index on cuda:0", flush=True)
    dev = "cuda"
    X = datagen.gen(30000, 768, 64, 0.7, seed=0, device=dev)
    Q = datagen.gen(256, 768, 64, 0.7, seed=1, device=dev, dtype=torch.float32)
    s1, code, Z, zs, Vr = index.build_index(X, nlist=128)
    E = EngineI8(s1, code, Z, zs, Vr, H=X)
    idx = oracle_mod.index_from_tables(s1, code, Z, zs, Vr, X)
    GT = npy(datagen.ground_truth(X, Q, 10))
    return dict(X=X, Q=Q, s1=s1, code=code, Z=Z, zs=zs, Vr=Vr, E=E, idx=idx, GT=GT)


@pytest.fixture(scope="module")
def traced(env, oracle_mod):
    """The eager trace of one batch with the canonical projection (CANON_Z): the oracle computes z itself, so
    everything but the two fp16 library products (QM, Zq) is checked end to end."""
    E, Q = env["E"], env["Q"]
    E.CANON_Z = True
    try:
        tr = E.trace(Q, K, Z_, NPROBE, KK)
        torch.cuda.synchronize()
    finally:
        E.CANON_Z = False
    tr = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in tr.items()}
    out = oracle_mod.pipeline(env["idx"], npy(Q), K, Z_, NPROBE, KK, QM16=u16(tr["QM"]), Zq16=u16(tr["Zq"]),
                              fallback=False)
    return tr, out


def test_build_codes_bit_exact(env, oracle_mod):
    s1 = env["s1"]
    Z, zs = oracle_mod.build_codes(npy(env["X"]), npy(s1["order"]), npy(s1["cell"]), npy(s1["means16"]),
                                   npy(env["Vr"]))
    assert np.array_equal(npy(env["Z"]), Z)
    assert np.array_equal(npy(env["zs"]).view(np.uint32), zs.view(np.uint32))


def test_query_code_bit_exact(traced):
    tr, out = traced
    assert np.array_equal(npy(tr["q8"]), out["q8"])
    assert np.array_equal(npy(tr["qs"]).view(np.uint32), out["qs"].view(np.uint32))
    assert np.array_equal(npy(tr["QC"]).view(np.uint32), out["qc"].view(np.uint32))
    assert np.array_equal(u16(tr["Qh"]), out["qh"])


def test_projection_bit_exact(env, oracle_mod, traced):
    """With CANON_Z, z = Q @ Vr is a sequential fp32 fmaf chain over d (fvs_query_code): the oracle's
    or_project gives the same bits. The default library GEMM's z is within fp32 accumulation error of float64,
    and the query code derived from it matches the oracle's given that z."""
    tr, _ = traced
    Q, Vr = npy(env["Q"]), npy(env["Vr"])
    assert np.array_equal(npy(tr["z"]).view(np.uint32), oracle_mod.project(Q, Vr).view(np.uint32))
    z64 = Q.astype(np.float64) @ Vr.astype(np.float64)
    assert np.all(np.abs(npy(tr["z"]) - z64) <= 1e-5 * np.abs(z64).max(1, keepdims=True))
    from fanarvse_paper_amd import _lib

    q8, qs, qc, qh, zb = _lib.query_prep(env["Q"], env["Vr"], env["s1"]["c"])  # the engine's default path
    torch.cuda.synchronize()
    assert np.all(np.abs(npy(zb) - z64) <= 1e-5 * np.abs(z64).max(1, keepdims=True))
    o8, oqs, oqc, oqh = oracle_mod.query_prep(Q, Vr, npy(env["s1"]["c"]), npy(zb))
    assert np.array_equal(npy(q8), o8) and np.array_equal(npy(qs).view(np.uint32), oqs.view(np.uint32))
    assert np.array_equal(npy(qc).view(np.uint32), oqc.view(np.uint32)) and np.array_equal(u16(qh), oqh)


def test_blas_products_accuracy(env, traced):
    """QM and Zq: fp16 outputs of fp16 GEMMs, within one fp16 rounding (+ fp32 accumulation) of float64."""
    tr, _ = traced
    Qh = npy(tr["Qh"]).astype(np.float64)
    E = env["E"]
    QM64 = Qh @ npy(E.meansN).astype(np.float64).T
    Zq64 = Qh @ npy(env["code"]["VP16"]).astype(np.float64)
    for got, ref in ((npy(tr["QM"]).astype(np.float64), QM64), (npy(tr["Zq"]).astype(np.float64), Zq64)):
        err = np.abs(got - ref)
        assert np.all(err <= np.abs(ref) * 2.0 ** -10 + 2.0 ** -20), float(err.max())


def test_routing_and_threshold_bit_exact(traced):
    tr, out = traced
    assert np.array_equal(npy(tr["probe"]), out["probe"])
    assert tr["n1"] == out["n1"] and tr["M"] == out["M"]
    # first-pass block maxima: compare the entries of blocks each probed cell has
    bm_g = npy(tr["bm"])
    bm_o = out["bm"]
    valid = bm_o > -1e29
    assert np.array_equal(bm_g[valid].view(np.uint32), bm_o[valid].view(np.uint32))
    assert np.array_equal(npy(tr["t0"]).view(np.uint32), out["t0"].view(np.uint32))
    assert np.array_equal(npy(tr["cnt"]), out["cnt"])


def test_emitted_sets_bit_exact(traced):
    tr, out = traced
    cnt = npy(tr["cnt"])
    M = tr["M"]
    bval, bpos = npy(tr["bval"]), npy(tr["bpos"])
    checked = 0
    for q in range(len(cnt)):
        n = int(cnt[q])
        if n > M:
            continue
        g = sorted(zip((-bval[q, :n]).tolist(), bpos[q, :n].tolist()))
        o = list(zip((-out["bval"][q, :n]).tolist(), out["bpos"][q, :n].tolist()))
        assert g == o, f"query {q}"
        checked += 1
    assert checked > 0


def test_select_and_stage2_bit_exact(traced):
    tr, out = traced
    assert np.array_equal(npy(tr["ok"]).astype(np.uint8), out["ok"])
    ok = out["ok"] == 1
    assert np.array_equal(npy(tr["pos"])[ok], out["pos"][ok])
    assert np.array_equal(npy(tr["est1"])[ok].view(np.uint32), out["est1"][ok].view(np.uint32))
    assert np.array_equal(npy(tr["ncnt"])[ok], out["ncnt"][ok])
    assert np.array_equal(u16(tr["L"]), out["L"])
    assert np.array_equal(npy(tr["qsum"]).view(np.uint32), out["qsum"].view(np.uint32))
    assert np.array_equal(npy(tr["qn2"]).view(np.uint32), out["qn2"].view(np.uint32))
    assert np.array_equal(npy(tr["est"])[ok].view(np.uint32), out["est"][ok].view(np.uint32))
    assert np.array_equal(npy(tr["sd"])[ok].view(np.uint32), out["sd"][ok].view(np.uint32))


def test_fused_lut_scorer_matches_build_then_score(env, traced):
    """fvs_lut_score_zq (tables and tier sums formed inside the scorer from Zq) gives the bits of
    fvs_lut_build followed by fvs_lut_score: fp16 and fp32 tables, all tiers or the leading two, with and
    without the delta-rule counts."""
    from fanarvse_paper_amd import _lib

    tr, _ = traced
    code = env["code"]
    dev = "cuda"
    pos, QC, Zq = tr["pos"].to(dev), tr["QC"].to(dev), tr["Zq"].to(dev)
    ncnt = tr["ncnt"].to(dev)
    for half in (True, False):
        pre = _lib.lut_build(Zq, code["TS"], half)
        for nt in (None, 2):
            for nc in (ncnt, None):
                a = _lib.lut_score(pos, QC, pre, code, nc, nt)
                b = _lib.lut_score(pos, QC, _lib.ZqTables(Zq, half), code, nc, nt)
                torch.cuda.synchronize()
                for x, y in zip(a, b):
                    assert np.array_equal(npy(x).view(np.uint32), npy(y).view(np.uint32)), (half, nt, nc is None)


def test_refine_and_final_ids_bit_exact(traced):
    tr, out = traced
    ok = out["ok"] == 1
    assert np.array_equal(npy(tr["ids"])[ok], out["ids"][ok])
    assert np.array_equal(npy(tr["I"])[ok], out["I"][ok])
    assert np.array_equal(npy(tr["scores"])[ok].view(np.uint32), out["scores"][ok].view(np.uint32))
    assert np.array_equal(npy(tr["reads"])[ok], out["reads"][ok])


def test_search_graph_replays_match_eager(env, traced):
    """The captured search (with the trace's canonical projection) replayed three times gives the eager ids."""
    tr, _ = traced
    E, Q = env["E"], env["Q"]
    ok = npy(tr["ok"]).astype(bool)
    E.CANON_Z = True
    try:
        for rep in range(3):
            I, reads, ids = E.search(Q, K, Z_, NPROBE, KK)
            x = torch.randn(1000, device="cuda").sum()  # eager work between replays
            torch.cuda.synchronize()
            assert np.array_equal(npy(I)[ok], npy(tr["I"])[ok]), f"replay {rep}"
            assert np.array_equal(npy(reads)[ok], npy(tr["reads"])[ok])
            assert np.array_equal(npy(ids)[ok], npy(tr["ids"])[ok])
            del x
    finally:
        E.CANON_Z = False


def test_fallback_matches_oracle(env, oracle_mod):
    """A buffer of K+8 entries overflows for most queries: they take the fallback path, which must agree
    with the oracle's fallback on the same shared BLAS inputs."""
    E, Q = env["E"], env["Q"]
    Qs = Q[:64].contiguous()
    old = E.MSZ
    E.MSZ = K + 8
    try:
        tr = E.trace(Qs, K, Z_, NPROBE, KK)
        I, reads, ids, sc = E.search(Qs, K, Z_, NPROBE, KK, ret_scores=True)
        torch.cuda.synchronize()
        nbad = int((~tr["ok"]).sum())
        out = oracle_mod.pipeline(env["idx"], npy(Qs), K, Z_, NPROBE, KK, knobs=dict(MSZ=K + 8),
                                  QM16=u16(tr["QM"]), Zq16=u16(tr["Zq"]), zq=npy(tr["z"]))
    finally:
        E.MSZ = old
        E.graphs.clear()
    assert nbad > 0 and len(out["bad"]) == nbad
    assert np.array_equal(npy(I), out["I"])
    assert np.array_equal(npy(reads), out["reads"])
    assert np.array_equal(npy(ids), out["cand"])
    assert np.array_equal(npy(sc).view(np.uint32), out["scores"].view(np.uint32))


def test_pipelined_submit_collect_matches_search(env):
    """NINST batches in flight, each with flagged queries (so a batch's fallback runs while the later
    batches' graphs run), give the same results as one search at a time; so do NINST full batches whose
    graph instances run at the same time, each on its own stream. One more submit of the shape, or a
    second collect of a ticket, raises."""
    E, Q = env["E"], env["Q"]
    n = E.NINST
    assert 2 <= n <= 4
    batches = [Q[64 * i:64 * (i + 1)].contiguous() for i in range(n)]
    old = E.MSZ
    E.MSZ = K + 8
    try:
        ref = [E.search(x, K, Z_, NPROBE, KK, ret_scores=True) for x in batches]
        torch.cuda.synchronize()
        # one search at a time collects each batch before the next submit: only instance 0 is captured
        insts = {gk[1] for gk in E.graphs if gk[0] != "fb"} | {gk[2] for gk in E.graphs if gk[0] == "fb"}
        assert insts == {0}, insts
        nb0 = E.nbad
        for rep in range(2):
            tickets = [E.submit(x, K, Z_, NPROBE, KK) for x in batches]
            with pytest.raises(RuntimeError):
                E.submit(batches[0], K, Z_, NPROBE, KK)  # one more batch of the shape than instances
            res = [E.collect(t, ret_scores=True) for t in tickets]
            with pytest.raises(RuntimeError):
                E.collect(tickets[0])
            torch.cuda.synchronize()
            for got, want in zip(res, ref):
                for g, w in zip(got, want):
                    assert np.array_equal(npy(g), npy(w)), f"rep {rep}"
        assert E.nbad > nb0
    finally:
        E.MSZ = old
        E.graphs.clear()
    # the whole query set, n different batches in flight at once
    full = [torch.roll(Q, 37 * i, 0).contiguous() for i in range(n)]
    ref = [E.search(x, K, Z_, NPROBE, KK, ret_scores=True) for x in full]
    torch.cuda.synchronize()
    for rep in range(3):
        tickets = [E.submit(x, K, Z_, NPROBE, KK) for x in full]
        res = [E.collect(t, ret_scores=True) for t in tickets]
        torch.cuda.synchronize()
        for got, want in zip(res, ref):
            for g, w in zip(got, want):
                assert np.array_equal(npy(g), npy(w)), f"concurrent rep {rep}"


def test_recall_and_pinned_host_rows(env):
    E, Q = env["E"], env["Q"]
    I, reads, ids = E.search(Q, K, Z_, NPROBE, KK)
    rec = metrics.recall(npy(I), env["GT"])
    assert rec >= 0.95, rec
    Hh = torch.empty(env["X"].shape, dtype=torch.float16, pin_memory=True)
    Hh.copy_(env["X"].cpu())
    Hd = E.H
    try:
        E.H = Hh
        E.graphs.clear()
        I2, reads2, ids2 = E.search(Q, K, Z_, NPROBE, KK)
        torch.cuda.synchronize()
    finally:
        E.H = Hd
        E.graphs.clear()
    assert np.array_equal(npy(I), npy(I2)) and np.array_equal(npy(reads), npy(reads2))
