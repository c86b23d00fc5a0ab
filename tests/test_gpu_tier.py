"""The NVMe row tier on the GPU: the split stage 3 (fvs_classify + fvs_refine_rows over rows gathered
in the classification's order) equals fvs_refine bit for bit on adversarial interval sets, and
EngineSTier, reading its rows from a tier file through both reader backends, returns exactly what
EngineS returns with the same rows in GPU memory: plain searches at batches 1, 16, 64, searches whose
queries take the fallback, and the pipelined run()."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib, datagen, tier, trellis
from fanarvse_paper_amd.engine_cell import EngineS
from fanarvse_paper_amd.engine_tier import EngineSTier

pytestmark = pytest.mark.gpu

K, Z_, NPROBE, KK = 100, 2.0, 12, 10


def npy(t):
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def env(tmp_path_factory):
    print("\n[gpu tier] building N=20000 d=768 NC=64 trellis index and its tier file", flush=True)
    X = datagen.gen(20000, 768, 32, 0.7, seed=0, device="cuda")
    Q = datagen.gen(200, 768, 32, 0.7, seed=1, device="cuda", dtype=torch.float32)
    s1, code = trellis.build_index(X, nlist=64)
    path = str(tmp_path_factory.mktemp("tier") / "rows.bin")
    tier.write_tier(path, X)
    E = EngineS(s1, code, H=X)
    return dict(X=X, Q=Q, s1=s1, code=code, E=E, path=path)


@pytest.mark.parametrize("B,Kc,k", [(1, 100, 10), (37, 400, 10), (300, 1000, 100), (5, 64, 63)])
def test_split_refine_equals_refine(env, B, Kc, k):
    X = env["X"]
    g = torch.Generator(device="cuda").manual_seed(B + Kc)
    # coarse values: many equal estimates and interval ends
    est = (torch.randint(-40, 40, (B, Kc), device="cuda", generator=g).float() * 0.01).contiguous()
    sd = (torch.randint(0, 6, (B, Kc), device="cuda", generator=g).float() * 0.02).contiguous()
    pos = torch.randint(0, X.shape[0], (B, Kc), device="cuda", generator=g, dtype=torch.int32)
    order = env["s1"]["order"]
    Q = torch.randn(B, 768, device="cuda", generator=g)
    ids, I, scores, reads = _lib.refine(est, sd, pos, order, X, Q, 1.5, k)
    ids2, flag, namb, aslot = _lib.classify(est, sd, pos, order, 1.5, k)
    nh = npy(namb)
    aid = npy(ids2.gather(1, aslot.long()))
    want = np.concatenate([aid[q, :nh[q]] for q in range(B)]).astype(np.int64)
    rows = X[torch.from_numpy(want).cuda()].contiguous() if len(want) else torch.zeros((1, 768), dtype=X.dtype,
                                                                                        device="cuda")
    roff = torch.from_numpy(np.concatenate([[0], np.cumsum(nh)[:-1]]).astype(np.int64)).cuda()
    I2, scores2, reads2 = _lib.refine_rows(est, flag, aslot, namb, roff, ids2, rows, Q, k)
    torch.cuda.synchronize()
    assert np.array_equal(npy(ids), npy(ids2))
    assert np.array_equal(npy(reads), npy(reads2)) and np.array_equal(npy(reads), nh)
    assert np.array_equal(npy(I), npy(I2))
    assert np.array_equal(npy(scores).view(np.uint32), npy(scores2).view(np.uint32))
    # the ambiguous slots are listed in ascending order
    asl = npy(aslot)
    for q in range(B):
        assert np.all(np.diff(asl[q, :nh[q]]) > 0)


def same(a, b):
    for x, y in zip(a, b):
        x, y = npy(x), npy(y)
        assert np.array_equal(x.view(np.uint32) if x.dtype == np.float32 else x,
                              y.view(np.uint32) if y.dtype == np.float32 else y)


@pytest.mark.parametrize("backend", [None, "threads"])
@pytest.mark.parametrize("B", [1, 16, 64])
def test_tier_engine_equals_engine(env, backend, B):
    print(f"\n[gpu tier] engine B={B} backend={backend}", flush=True)
    with tier.RowTier(env["path"], 768, qd=64, backend=backend) as T:
        Et = EngineSTier(env["s1"], env["code"], T)
        Q = env["Q"][:B].contiguous()
        same(env["E"].search(Q, K, Z_, NPROBE, KK, ret_scores=True), Et.search(Q, K, Z_, NPROBE, KK, ret_scores=True))
        assert Et.rows_read > 0


def test_tier_engine_fallback_and_pipeline(env):
    """A K+8 buffer sends most queries through the fallback in both engines; then the pipelined run()
    over all 200 queries against EngineS batch by batch."""
    E = env["E"]
    with tier.RowTier(env["path"], 768) as T:
        Et = EngineSTier(env["s1"], env["code"], T)
        Q = env["Q"][:48].contiguous()
        E.M = Et.M = K + 8
        E.graphs.clear()
        try:
            a = E.search(Q, K, Z_, NPROBE, KK, ret_scores=True)
            b = Et.search(Q, K, Z_, NPROBE, KK, ret_scores=True)
        finally:
            E.M = Et.M = None
            E.graphs.clear()
        assert Et.nbad > 0
        same(a, b)
        I, reads, ids = Et.run(env["Q"], K, Z_, NPROBE, KK, B=64)
        for s in range(0, 200, 64):
            ref = E.search(env["Q"][s:s + 64].contiguous(), K, Z_, NPROBE, KK)
            assert np.array_equal(npy(ref[0]), I[s:s + 64])
            assert np.array_equal(npy(ref[1]), reads[s:s + 64])
            assert np.array_equal(npy(ref[2]), ids[s:s + 64])
