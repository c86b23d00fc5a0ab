"""The versioned index file (fanarvse_paper_amd/store.py), on the CPU: every object the engines keep
(nested dicts with int keys, lists of tier tuples, tensors of every dtype, numpy arrays, empty arrays,
scalars) survives save -> load bit-exactly, arrays sit at 4096-byte offsets, and damaged or foreign files
are refused with IndexFormatError instead of being read."""
import os
import struct

import numpy as np
import pytest
import torch

from fanarvse_paper_amd import s2lut, store


def same(a, b, path="root"):
    """Deep equality that also compares types, dtypes, shapes and bits (NaN included)."""
    assert type(a) is type(b), f"{path}: {type(a)} vs {type(b)}"
    if isinstance(a, torch.Tensor):
        assert a.dtype == b.dtype and a.shape == b.shape, path
        assert a.device.type == b.device.type, path
        assert torch.equal(a.cpu().contiguous().view(-1).view(torch.uint8) if a.numel() else a.cpu(),
                           b.cpu().contiguous().view(-1).view(torch.uint8) if b.numel() else b.cpu()), path
    elif isinstance(a, np.ndarray):
        assert a.dtype == b.dtype and a.shape == b.shape, path
        assert a.tobytes() == b.tobytes(), path
    elif isinstance(a, dict):
        assert list(a.keys()) == list(b.keys()), path
        for k in a:
            same(a[k], b[k], f"{path}.{k}")
    elif isinstance(a, (list, tuple)):
        assert len(a) == len(b), path
        for i, (x, y) in enumerate(zip(a, b)):
            same(x, y, f"{path}.{i}")
    elif isinstance(a, float) and a != a:
        assert b != b, path
    else:
        assert a == b, path


def sample():
    g = torch.Generator().manual_seed(0)
    tensors = {str(dt).split(".")[-1]: (torch.randn(7, 5, generator=g) * 100).to(dt)
               for dt in (torch.float32, torch.float16, torch.float64, torch.int8, torch.uint8, torch.int16,
                          torch.int32, torch.int64, torch.bool)}
    tensors["nan"] = torch.tensor([float("nan"), -0.0, float("inf")])
    tensors["empty"] = torch.empty(0, 3, dtype=torch.int32)
    tensors["scalar"] = torch.tensor(3.5)
    tensors["strided"] = torch.arange(24, dtype=torch.int64).reshape(4, 6).t()   # saved contiguous
    return dict(t=tensors, TS=[(0, 32, 4), (32, 96, 2)], off=np.array([0, 3, 9], dtype=np.int64),
                bits={2: np.float32(0.5), 3: np.array([1.0, 2.0], dtype=np.float32)}, kind="lloyd",
                n=np.int64(7), alpha=0.875, none=None, flag=True, nested=[[torch.ones(2)], ()])


def test_round_trip_bit_exact(tmp_path):
    obj = sample()
    p = str(tmp_path / "a.fvs")
    store.save(p, s1=obj, Z=torch.arange(256, dtype=torch.int8).reshape(2, 128))
    r = store.load(p)
    want = dict(obj)
    want["n"] = 7                                   # numpy scalars come back as Python numbers
    want["bits"] = {2: 0.5, 3: obj["bits"][3]}
    want["t"] = dict(obj["t"], strided=obj["t"]["strided"].contiguous())
    same(want, r["s1"])
    same(torch.arange(256, dtype=torch.int8).reshape(2, 128), r["Z"])


def test_stage2_code_round_trip(tmp_path):
    """The Lloyd-Max and uniform tiered codes (int-keyed level and step tables, CPU rotations)."""
    X = (torch.randn(1500, 64, generator=torch.Generator().manual_seed(1))).half()
    c = X.float().mean(0)
    lam, V = s2lut.pca_basis(X, c)
    TS = s2lut.allocate(lam, int(2.5 * 64))
    order = torch.randperm(1500, generator=torch.Generator().manual_seed(2)).to(torch.int32)
    codes = dict(lloyd=s2lut.encode_lloyd(X, order, c, V, TS, seed=0), uniform=s2lut.encode_uniform_tiers(X, order, c, V, TS))
    p = str(tmp_path / "c.fvs")
    store.save(p, **codes)
    same(codes, store.load(p))


def test_layout_is_aligned_and_versioned(tmp_path):
    p = str(tmp_path / "b.fvs")
    store.save(p, x=torch.arange(1000, dtype=torch.int32), y=np.zeros(3, np.uint8))
    raw = open(p, "rb").read()
    assert raw[:8] == store.MAGIC
    version, n = struct.unpack("<II", raw[8:16])
    assert version == store.VERSION == 1
    import json
    man = json.loads(raw[16:16 + n])
    base = (16 + n + 4095) // 4096 * 4096
    for e in man["arrays"].values():
        assert (base + e["offset"]) % 4096 == 0
    assert np.frombuffer(raw[base:base + 4000], np.int32).tolist() == list(range(1000))
    assert len(raw) % 4096 == 0


def _write(p, raw):
    with open(p, "wb") as f:
        f.write(raw)


def test_damaged_files_are_refused(tmp_path):
    p = str(tmp_path / "d.fvs")
    store.save(p, x=torch.arange(5000, dtype=torch.int32))
    raw = bytearray(open(p, "rb").read())
    bad = str(tmp_path / "bad.fvs")

    flipped = bytearray(raw)
    flipped[-4096 - 100] ^= 1                        # one bit in the array payload
    _write(bad, flipped)
    with pytest.raises(store.IndexFormatError, match="checksum"):
        store.load(bad)
    store.load(bad, verify=False)                   # verify=False skips the check by request only

    _write(bad, raw[: len(raw) - 8192])              # truncated payload
    with pytest.raises(store.IndexFormatError, match="truncated"):
        store.load(bad)

    _write(bad, b"PK\x03\x04" + raw[4:])              # a zip (torch.save) file is not read
    with pytest.raises(store.IndexFormatError, match="magic"):
        store.load(bad)

    newer = bytearray(raw)
    newer[8:12] = struct.pack("<I", 2)
    _write(bad, newer)
    with pytest.raises(store.IndexFormatError, match="version 2"):
        store.load(bad)

    _write(bad, raw[:20])
    with pytest.raises(store.IndexFormatError):
        store.load(bad)


def test_unstorable_objects_are_rejected(tmp_path):
    p = str(tmp_path / "e.fvs")
    with pytest.raises(TypeError):
        store.save(p, x=object())
    with pytest.raises(TypeError):
        store.save(p, x=torch.zeros(2, dtype=torch.complex64))
    assert not os.path.exists(p)
    tricky = {"__array__": 1, "__tuple__": [2]}      # keys that look like markers are stored as pairs
    store.save(p, x=tricky)
    same(tricky, store.load(p)["x"])


def test_colliding_keys_are_rejected(tmp_path):
    """Array keys are '.'-joined paths: a key containing '.', two objects on one path, or an array used as a
    dict key (which would be dropped) are refused instead of silently overwriting or losing an array."""
    p = str(tmp_path / "k.fvs")
    t = torch.arange(4, dtype=torch.int32)
    with pytest.raises(ValueError):
        store.save(p, x={"a.b": t})
    with pytest.raises(ValueError):
        store.save(p, **{"x.0": t, "x": [t]})
    with pytest.raises(TypeError):
        store.save(p, x={1: t, torch.tensor(3): t})
    with pytest.raises(TypeError):
        store.save(p, x={np.int64(1): t, (1, 2): t})
    assert not os.path.exists(p)
    ok = {1: t, "1": t + 1}                            # an int and a str key stay distinct (stored as pairs)
    store.save(p, x=ok)
    same(ok, store.load(p)["x"])
