"""GPU parity of the trellis (default) engine against the CPU oracle on the same seeded inputs: the
Viterbi encoder, routing on fp32 keys, the trellis stage-1 scan (block maxima, threshold, emitted sets,
selection), the Lloyd-Max stage 2, refinement, and whole searches at the latency batch sizes 1, 16, 64.
Integer and index results are bit-exact; so are the floating-point stages (one canonical operation
order, include/fvs.h). The dense products (Qr = Q @ W1, QM, Zq = Q @ VP) come from the GPU's BLAS and
are shared inputs of the oracle."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import datagen, metrics, trellis
from fanarvse_paper_amd.engine_cell import EngineS

pytestmark = pytest.mark.gpu

K, Z_, NPROBE, KK = 100, 2.0, 12, 10


def npy(t):
    return t.detach().cpu().numpy()


def u16(t):
    return npy(t).view(np.uint16)


@pytest.fixture(scope="module")
def env(oracle_mod):
    print("\n[gpu trellis] building N=20000 d=768 NC=64 trellis index on cuda:0", flush=True)
    dev = "cuda"
    X = datagen.gen(20000, 768, 32, 0.7, seed=0, device=dev)
    Q = datagen.gen(64, 768, 32, 0.7, seed=1, device=dev, dtype=torch.float32)
    s1, code = trellis.build_index(X, nlist=64)
    E = EngineS(s1, code, H=X)
    idx = oracle_mod.trellis_index_from_tables(s1, code, X)
    GT = npy(datagen.ground_truth(X, Q, 10))
    return dict(X=X, Q=Q, s1=s1, code=code, E=E, idx=idx, GT=GT)


@pytest.fixture(scope="module")
def traced(env, oracle_mod):
    tr = env["E"].trace(env["Q"], K, Z_, NPROBE, KK)
    torch.cuda.synchronize()
    tr = {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in tr.items()}
    out = oracle_mod.tr_pipeline(env["idx"], npy(env["Q"]), K, Z_, NPROBE, KK, Qr=npy(tr["Qr"]), QM16=u16(tr["QM"]),
                                 Zq=npy(tr["Zq"]), fallback=False)
    return tr, out


def test_encoder_bit_exact(oracle_mod):
    rng = np.random.default_rng(11)
    for L in (8, 10):
        Zs = rng.standard_normal((300, 256)).astype(np.float32)
        Zs *= np.float32(16.0) / np.linalg.norm(Zs, axis=1, keepdims=True).astype(np.float32)
        nz = rng.uniform(0.2, 3.0, 300).astype(np.float32)
        tab = (0.93 * trellis.make_table(L)).astype(np.float32)
        w, s1, p = trellis.encode(torch.from_numpy(Zs).cuda(), torch.from_numpy(nz).cuda(),
                                  torch.from_numpy(tab).cuda(), L, paths=True)
        torch.cuda.synchronize()
        ow, os1, op = oracle_mod.trellis_encode(Zs, nz, tab, L)
        assert np.array_equal(npy(p), op)
        assert np.array_equal(npy(w).view(np.uint32), ow)
        assert np.array_equal(u16(s1), os1)


def test_routing_and_first_pass_bit_exact(env, traced):
    tr, out = traced
    assert np.array_equal(npy(tr["QC"]).view(np.uint32), out["qc"].view(np.uint32))
    assert np.array_equal(npy(tr["probe"]), out["probe"])
    assert tr["n1"] == out["n1"] and tr["M"] == out["M"]
    # block maxima of the blocks each probed cell has (the others are never read)
    off = env["idx"]["off"]
    bm, obm = npy(tr["bm"]), out["bm"]
    for q in range(bm.shape[0]):
        for j in range(tr["n1"]):
            c = out["probe"][q, j]
            nb = (off[c + 1] - 1) // 32 - off[c] // 32 + 1 if off[c + 1] > off[c] else 0
            assert np.array_equal(bm[q, j, :nb].view(np.uint32), obm[q, j, :nb].view(np.uint32)), (q, j)
    assert np.array_equal(npy(tr["t0"]).view(np.uint32), out["t0"].view(np.uint32))


def test_emit_and_select_bit_exact(traced):
    tr, out = traced
    cnt = npy(tr["cnt"])
    assert np.array_equal(cnt, out["cnt"])
    M = tr["M"]
    for q in range(len(cnt)):
        n = min(int(cnt[q]), M)
        if cnt[q] > M:
            continue
        got = sorted(zip(npy(tr["bpos"])[q, :n].tolist(), npy(tr["bval"])[q, :n].view(np.uint32).tolist()))
        want = sorted(zip(out["bpos"][q, :n].tolist(), out["bval"][q, :n].view(np.uint32).tolist()))
        assert got == want, q
    ok = npy(tr["ok"]).astype(bool)
    assert np.array_equal(ok, out["ok"].astype(bool))
    assert np.array_equal(npy(tr["pos"])[ok], out["pos"][ok])


def test_stage2_and_refine_bit_exact(traced):
    tr, out = traced
    ok = npy(tr["ok"]).astype(bool)
    assert np.array_equal(npy(tr["est"])[ok].view(np.uint32), out["est"][ok].view(np.uint32))
    assert np.array_equal(npy(tr["sd"])[ok].view(np.uint32), out["sd"][ok].view(np.uint32))
    assert np.array_equal(npy(tr["I"])[ok], out["I"][ok])
    assert np.array_equal(npy(tr["reads"])[ok], out["reads"][ok])
    assert np.allclose(npy(tr["scores"])[ok], out["scores"][ok], rtol=1e-3)


@pytest.mark.parametrize("B", [1, 16, 64])
def test_search_batch_sizes_match_oracle(env, oracle_mod, B):
    E = env["E"]
    Q = env["Q"][:B].contiguous()
    I, reads, ids, sc = E.search(Q, K, Z_, NPROBE, KK, ret_scores=True)
    I2, _, _, _ = E.search(Q, K, Z_, NPROBE, KK, ret_scores=True)  # a second replay of the graph
    torch.cuda.synchronize()
    assert torch.equal(I, I2)
    Qr, QC, QM, Zq = E._dense(Q)
    out = oracle_mod.tr_pipeline(env["idx"], npy(Q), K, Z_, NPROBE, KK, Qr=npy(Qr), QM16=u16(QM), Zq=npy(Zq))
    assert np.array_equal(npy(I), out["I"])
    assert np.array_equal(npy(reads), out["reads"])
    assert np.array_equal(npy(ids), out["cand"])
    if B >= 16:  # one query's recall is too coarse a statistic
        rec = metrics.recall(npy(I), env["GT"][:B], 10)
        assert rec >= 0.85, rec
