"""The index-build entry points with the reference's signatures, on the GPU:
build_codes(s1, X16, V, R) -> (Z, zs, Vr) (throughput/enginei8.py:19-27) with the rows on the device or in
host memory (chunked, as the reference reads rf.host16), and with or without a `cell` table; and
compact(cellify(s1)) (src/engine_cell.py:8-32) over a reference-shaped s1 (order int64, off numpy, W1, tab,
no cell tables), whose codes must equal the oracle's Viterbi encode of the residuals against the fp32 cell
means."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import datagen, index, trellis

pytestmark = pytest.mark.gpu
dev = "cuda"


def npy(t):
    return t.detach().cpu().numpy()


@pytest.fixture(scope="module")
def env():
    print("\n[gpu build api] N=12000 d=384 NC=48", flush=True)
    X = datagen.gen(12000, 384, 24, 0.7, seed=8, device=dev)
    s1 = index.build_stage1_cells(X, 48, seed=1)
    return dict(X=X, s1=s1)


def test_build_codes_host_rows_and_offsets(env, oracle_mod):
    X, s1 = env["X"], env["s1"]
    V = index.pca_int8_basis(X, R=320)  # a basis wider than R: the first R columns are used
    Z, zs, Vr = index.build_codes(s1, X, V, R=256)
    assert torch.equal(Vr, V[:, :256])
    Zo, zso = oracle_mod.build_codes(npy(X), npy(s1["order"]), npy(s1["cell"]), npy(s1["means16"]), npy(Vr))
    assert np.array_equal(npy(Z), Zo) and np.array_equal(npy(zs).view(np.uint32), zso.view(np.uint32))
    ref_s1 = {k: v for k, v in s1.items() if k != "cell"}
    ref_s1["order"] = s1["order"].long()
    Zh, zsh, _ = index.build_codes(ref_s1, X.cpu(), V, R=256, chunk=5000)
    assert torch.equal(Zh, Z) and torch.equal(zsh.view(torch.int32), zs.view(torch.int32))


def test_compact_cellify_of_a_reference_s1(env, oracle_mod):
    X, s1 = env["X"], env["s1"]
    L, R = 10, 256
    W1 = trellis.rotation_basis(X, s1["c"], R)
    T = trellis.make_table(L)
    tab = (0.95 * torch.from_numpy(T)).to(dev).contiguous()
    ref = dict(c=s1["c"], W1=W1, tab=tab, alpha=0.95, off=s1["off"], order=s1["order"].long())
    out = trellis.compact(trellis.cellify(ref, X.cpu(), L))
    assert "cell" not in ref and ref["order"].dtype == torch.int64      # the input dict is not modified
    assert out["order"].dtype == torch.int32 and torch.equal(out["order"], s1["order"])
    assert torch.equal(out["cell"], s1["cell"]) and torch.equal(out["off_t"], s1["off_t"])
    assert torch.equal(out["means16"], s1["means16"])                    # the same member means
    assert torch.equal(out["inv_mnorm"], s1["inv_mnorm"]) and out["cen"] is out["inv_mnorm"]
    # the codes: Viterbi paths of the residuals against the fp32 cell means
    order, cell = s1["order"].long(), s1["cell"].long()
    means = index.cell_means(X, s1["order"], s1["cell"], torch.as_tensor(s1["off"], device=dev), 48)
    rows = slice(0, 600)
    Zr = (X[order].float() - means[cell]) @ W1  # one product over all rows, as encode_cells forms it
    nz = Zr.norm(dim=1).clamp(min=1e-6)
    Zs = Zr / nz[:, None] * R ** 0.5
    w, s, _ = oracle_mod.trellis_encode(npy(Zs[rows]), npy(nz[rows]), npy(tab), L)
    assert np.array_equal(npy(out["words"][rows]).view(np.uint32), w)
    assert np.array_equal(npy(out["scale1"][rows]).view(np.uint16), s)
