"""The row tier reader (libfvs_tier.so) on the CPU: rows written by tier.write_tier come back bit-exact
through both backends (io_uring where the kernel allows it, the pread() thread pool always), for row
sizes below, at and above one sector, unsorted and repeated ids, queue depths from 1 up, a last row
shorter than its slot, and every exported function of include/fvs_tier.h; bad ids and arguments are
refused before anything is read."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from fanarvse_paper_amd import tier

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module", autouse=True)
def built():
    from fanarvse_paper_amd import build

    if not os.path.exists(tier.LIB_PATH):
        build.build_tier()


def rows(N, d, seed):
    x = np.random.default_rng(seed).standard_normal((N, d)).astype(np.float16)
    x[0, 0] = np.float16(-0.0)
    x[1, :3] = [np.inf, -np.inf, np.nan]
    return x


def test_every_declared_symbol_is_exported():
    text = open(os.path.join(ROOT, "include", "fvs_tier.h")).read()
    names = sorted(set(re.findall(r"^\S.*?\b(fvs_tier_\w+)\s*\(", text, re.M)))
    assert len(names) == 5, names
    L = ctypes.CDLL(tier.LIB_PATH)
    for n in names:
        assert hasattr(L, n), n


@pytest.mark.parametrize("d", [100, 768, 2048, 3000])
@pytest.mark.parametrize("backend", [None, "threads"])
def test_rows_round_trip(tmp_path, d, backend):
    X = rows(3001, d, d)
    p = str(tmp_path / "t.bin")
    stride = tier.write_tier(p, X)
    assert stride == -(-2 * d // 4096) * 4096 and os.path.getsize(p) == 3001 * stride
    rng = np.random.default_rng(7)
    ids = np.concatenate([rng.integers(0, 3001, 5000), [3000, 0, 3000, 17, 17]])
    for qd in (1, 7, 128):
        with tier.RowTier(p, d, qd=qd, backend=backend) as T:
            assert T.rows == 3001
            if backend == "threads":
                assert T.backend == "threads"
            got = T.read(ids)
            assert got.view(np.uint16).tobytes() == X[ids].view(np.uint16).tobytes()
            # into a pinned-or-not CPU tensor, and an empty batch
            out = torch.empty((len(ids), d), dtype=torch.float16)
            T.read_into(ids, out)
            assert np.array_equal(out.numpy().view(np.uint16), X[ids].view(np.uint16))
            assert T.read(np.zeros(0, np.int64)).shape == (0, d)


def test_uring_backend_where_available(tmp_path):
    """Where the kernel allows io_uring the default handle uses it (this container's does)."""
    p = str(tmp_path / "u.bin")
    tier.write_tier(p, rows(64, 768, 1))
    with tier.RowTier(p, 768) as T:
        assert T.backend in ("io_uring", "threads")
        if T.backend == "io_uring":
            assert np.array_equal(T.read(np.arange(64)[::-1]).view(np.uint16), rows(64, 768, 1)[::-1].view(np.uint16))


def test_short_last_row_and_buffered(tmp_path):
    """A file whose last row is not padded to its slot still reads that row; O_DIRECT can be declined."""
    X = rows(10, 768, 3)
    p = str(tmp_path / "s.bin")
    tier.write_tier(p, X)
    with open(p, "r+b") as f:
        f.truncate(9 * 4096 + 2 * 768)
    for backend in (None, "threads"):
        with tier.RowTier(p, 768, backend=backend, buffered=backend is None) as T:
            assert T.rows == 10
            assert np.array_equal(T.read([9, 0, 9]).view(np.uint16), X[[9, 0, 9]].view(np.uint16))


def test_refusals(tmp_path):
    X = rows(20, 768, 4)
    p = str(tmp_path / "r.bin")
    tier.write_tier(p, X)
    T = tier.RowTier(p, 768)
    with pytest.raises(IndexError):
        T.read([0, 20])
    with pytest.raises(IndexError):
        T.read([-1])
    with pytest.raises(ValueError):
        T.read_into([0, 1], np.empty((3, 768), np.float16))
    with pytest.raises(ValueError):
        T.read_into([0], np.empty((1, 768), np.float32))
    assert np.array_equal(T.read([5]).view(np.uint16), X[[5]].view(np.uint16))  # still usable
    T.close()
    with pytest.raises(ValueError):
        T.read([0])
    with pytest.raises(OSError):
        tier.RowTier(str(tmp_path / "missing.bin"), 768)
    with pytest.raises(OSError):
        tier.RowTier(p, 768, stride=1000)             # not a multiple of 4096
    with pytest.raises(OSError):
        tier.RowTier(p, 768, qd=0)
    L = tier.lib()
    assert L.fvs_tier_read_rows(None, None, 0, None, 16) < 0
    with pytest.raises(ValueError):
        tier.write_tier(str(tmp_path / "x.bin"), X, stride=4096 + 1)
