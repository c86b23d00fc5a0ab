"""A saved and reloaded index searches exactly like the one that was built: the int8 throughput tables
(s1, code, Z, zs, Vr) and the trellis tables (s1, code) go through the versioned index file, every table
comes back bit-exact and on the device it was saved from, and EngineI8, EngineS and SpaceX built on the
loaded tables return the same ids, reads and candidate sets as on the built ones."""
import pytest
import torch

from fanarvse_paper_amd import datagen, index, store, trellis
from fanarvse_paper_amd.engine_cell import EngineS
from fanarvse_paper_amd.engine_host import SpaceX
from fanarvse_paper_amd.enginei8 import EngineI8

from test_store import same

pytestmark = pytest.mark.gpu


def equal_outputs(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert torch.equal(x.cpu(), y.cpu())


def test_i8_index_round_trip(tmp_path):
    print("\n[gpu store] int8 index N=20000 d=768 NC=64: build, save, load, search", flush=True)
    X = datagen.gen(20000, 768, 32, 0.7, seed=0, device="cuda")
    Q = datagen.gen(64, 768, 32, 0.7, seed=1, device="cuda", dtype=torch.float32)
    s1, code, Z, zs, Vr = index.build_index(X, nlist=64)
    p = str(tmp_path / "i8.fvs")
    store.save(p, s1=s1, code=code, Z=Z, zs=zs, Vr=Vr)
    r = store.load(p)
    same(dict(s1=s1, code=code, Z=Z, zs=zs, Vr=Vr), r)
    a = EngineI8(s1, code, Z, zs, Vr, H=X).search(Q, 150, 1.25, 12, 10)
    b = EngineI8(r["s1"], r["code"], r["Z"], r["zs"], r["Vr"], H=X).search(Q, 150, 1.25, 12, 10)
    torch.cuda.synchronize()
    equal_outputs(a, b)


def test_trellis_index_round_trip(tmp_path):
    print("\n[gpu store] trellis index N=20000 d=768 NC=64: build, save, load, search", flush=True)
    X = datagen.gen(20000, 768, 32, 0.7, seed=0, device="cuda")
    Q = datagen.gen(16, 768, 32, 0.7, seed=1, device="cuda", dtype=torch.float32)
    s1, code = trellis.build_index(X, nlist=64)
    p = str(tmp_path / "tr.fvs")
    store.save(p, s1=s1, code=code)
    r = store.load(p)
    same(dict(s1=s1, code=code), r)
    equal_outputs(EngineS(s1, code, H=X).search(Q, 100, 2.0, 12, 10),
                  EngineS(r["s1"], r["code"], H=X).search(Q, 100, 2.0, 12, 10))
    equal_outputs(SpaceX(s1, code, X).search(Q, 100, 2.0, 12, 10),
                  SpaceX(r["s1"], r["code"], X).search(Q, 100, 2.0, 12, 10))
