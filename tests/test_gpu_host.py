"""GPU parity of the host-resident engine (SpaceX): stage-1 codes read zero-copy from pinned host memory
(or streamed from it in chunks on a side stream), stage-2 records and fp16 rows read zero-copy,
projected-means routing. Same results as the CPU oracle on the same inputs (the dense products are
shared), bit for bit, and the GPU holds under 8 bytes per vector."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import datagen, trellis
from fanarvse_paper_amd.engine_host import SpaceX

pytestmark = pytest.mark.gpu


def npy(t):
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def env(oracle_mod):
    print("\n[gpu host] building N=20000 d=768 NC=64 trellis index, host-resident engine", flush=True)
    X = datagen.gen(20000, 768, 32, 0.7, seed=0, device="cuda")
    Q = datagen.gen(48, 768, 32, 0.7, seed=1, device="cuda", dtype=torch.float32)
    s1, code = trellis.build_index(X, nlist=64)
    SpaceX.CHUNK = 2048  # several chunks, so the streaming path is exercised
    E = SpaceX(s1, code, X)
    Ec = SpaceX(s1, code, X, staging="copy")
    Ep = SpaceX(s1, code, X, proj=True, vp16=False)
    Epc = SpaceX(s1, code, X, proj=True, vp16=False, staging="copy")
    idx = oracle_mod.trellis_index_from_tables(s1, code, X)
    idx["Hs"] = npy(X[s1["order"].long()]).view(np.uint16)
    return dict(X=X, Q=Q, s1=s1, E=E, Ec=Ec, Ep=Ep, Epc=Epc, idx=idx)


@pytest.mark.parametrize("variant", ["E", "Ec", "Ep", "Epc"])
def test_streamed_engine_matches_oracle(env, oracle_mod, variant):
    E, Q = env[variant], env["Q"]
    print(f"\n[gpu host] {variant}: staging {E.staging}, proj {E.proj}", flush=True)
    assert len(E.chunks) > 4 if E.staging == "copy" else not E.chunks
    K, z, nprobe, k = 100, 2.0, 12, 10
    I, reads, ids = E.search(Q, K, z, nprobe, k, sorted_ids=True)
    torch.cuda.synchronize()
    Qr, QC, QM, Zq = E._dense(Q)
    out = oracle_mod.tr_pipeline(env["idx"], npy(Q), K, z, nprobe, k, Qr=npy(Qr), QM16=npy(QM).view(np.uint16),
                                 Zq=npy(Zq), proj=E.proj, order=False, half=True,  # search_static: fp16 operands
                                 fb_rho=None, fb_M=E.FALLBACK_M)
    assert np.array_equal(npy(I), out["I"])
    assert np.array_equal(npy(reads), out["reads"])
    assert np.array_equal(npy(ids), out["cand"])
    # host id mapping
    I2, _, _ = E.search(Q, K, z, nprobe, k)
    assert np.array_equal(I2.numpy(), E.order_np[out["I"]])


@pytest.mark.parametrize("variant", ["E", "Ec"])
def test_gpu_bytes_per_vector(env, variant):
    """Only the static work list grows with N on the GPU (16 B per 32-row block: 0.5 B per vector); the rest are
    shared tables of fixed size (and, with copy staging, the two slots), so at the host-resident config's 1.28M
    vectors the total stays under 8 B."""
    E = env[variant]
    N = E.N
    fixed = sum(t.numel() * t.element_size() for t in (E.means, E.W1, E.code["VP"], E.code["cb"], E.s1["tab"],
                                                       E.s1["off_t"], E.s1["inv_mnorm"], E.s1["c"]))
    fixed += sum(b.numel() * b.element_size() for b in E.slots)
    per_vector = E.gpu_bytes() - fixed / N
    assert per_vector <= 0.6, per_vector
    host = [E.Hs, E.code["rec"]] + ([E.stage_h] if E.staging == "copy" else [E.words_h, E.scale1_h])
    assert all(t.is_pinned() and not t.is_cuda for t in host)
    if E.staging == "zero-copy":
        assert not E.slots


def test_overflow_fallback_matches_oracle(env, oracle_mod):
    """A main-pass buffer of K + 28 entries: most queries overflow it and are flagged, and their second pass
    (the same rho, a 1 << 20-entry buffer: host_resident/space_x.py:63-70) is checked against the oracle's,
    bit for bit, as are the final ids of the batch."""
    E, Q = env["E"], env["Q"]
    K, z, nprobe, k = 100, 2.0, 12, 10
    E.M, E.nbad = K + 28, 0
    try:
        I, reads, ids = E.search(Q, K, z, nprobe, k, sorted_ids=True)
        torch.cuda.synchronize()
    finally:
        E.M = None
    assert E.nbad > Q.shape[0] // 2, E.nbad
    Qr, QC, QM, Zq = E._dense(Q)
    out = oracle_mod.tr_pipeline(env["idx"], npy(Q), K, z, nprobe, k, Qr=npy(Qr), QM16=npy(QM).view(np.uint16),
                                 Zq=npy(Zq), proj=E.proj, order=False, half=True, M=K + 28, fb_rho=None,
                                 fb_M=E.FALLBACK_M)
    assert len(out["bad"]) == E.nbad
    assert np.array_equal(npy(I), out["I"])
    assert np.array_equal(npy(reads), out["reads"])
    assert np.array_equal(npy(ids), out["cand"])
