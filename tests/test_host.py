"""Host-side logic of the product package that needs no GPU: work lists, knobs, record layout, the
scalar-quantiser tables behind the bit allocation, and the synthetic generator."""
import math

import numpy as np
import pytest
import torch
from scipy import integrate
from scipy.stats import norm

from fanarvse_paper_amd import datagen, index, s2lut


def test_static_chunks_cover_every_static_block_once(oracle_mod):
    rng = np.random.default_rng(2)
    sizes = rng.integers(0, 300, 40)
    sizes[[3, 17]] = 0
    sizes[5] = 1000
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    cell, blk, ps, pe, MB = oracle_mod.static_blocks(off)
    want = sorted(zip(cell.tolist(), blk.tolist()))
    c, r0, s, e = (t.numpy() for t in index.static_chunks(torch.from_numpy(off), 32, 8))
    assert (r0 % 32 == 0).all()
    got = []
    for i in range(len(c)):
        last = (e[i] - 1) // 32
        assert s[i] == off[c[i]] and e[i] == off[c[i] + 1]
        got += [(int(c[i]), int(bb)) for bb in range(r0[i] // 32, min(r0[i] // 32 + 8, last + 1))]
    assert sorted(got) == want and len(got) == len(set(got))
    _, MBt = index.static_blocks(torch.from_numpy(off), 32)
    assert MBt == MB


def test_row_chunks_cover_every_row_once():
    """Emit items: each row of each cell in exactly one item of at most 256 rows, the first item of a
    cell at its first row, and a cell of up to 256 rows in one item."""
    rng = np.random.default_rng(3)
    sizes = rng.integers(0, 700, 60)
    sizes[[2, 9]] = 0
    sizes[[4, 5, 6]] = [256, 257, 512]
    off = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int32)
    c, r0, s, e = (t.numpy() for t in index.row_chunks(torch.from_numpy(off), 256))
    seen = np.zeros(off[-1], np.int32)
    for i in range(len(c)):
        assert s[i] == off[c[i]] and e[i] == off[c[i] + 1] and s[i] <= r0[i] < e[i]
        seen[r0[i]:min(r0[i] + 256, e[i])] += 1
    assert (seen == 1).all()
    items = np.bincount(c, minlength=len(sizes))
    assert (items == (sizes + 255) // 256).all()
    assert items[4] == 1 and items[5] == 2 and items[6] == 2


def test_proj_knob_needs_stage1_basis():
    """PROJ routing (NROUTE off) projects through s1["W1"]: without it the engine refuses before any work;
    the other knobs need no extra table."""
    from fanarvse_paper_amd.enginei8 import EngineI8

    E = EngineI8.__new__(EngineI8)
    E.s1 = {}
    E.NROUTE, E.PROJ = False, True
    with pytest.raises(ValueError):
        E._check_knobs()
    E.s1 = {"W1": None}
    E._check_knobs()
    for attr, val in (("K2", 100), ("NROUTE", False), ("UNSORTED", True), ("SORTROUTE", True)):
        E2 = EngineI8.__new__(EngineI8)
        E2.s1 = {}
        setattr(E2, attr, val)
        E2._check_knobs()


def test_record_layout_of_the_paper_tiers():
    """The OpenAI tiering of paper/main.tex:219: 3,840 bits of planes = 480 B, then 6 fp16 pairs = 504 B,
    rounded to a 512-byte record."""
    TS = [(0, 32, 7), (32, 128, 5), (128, 384, 4), (384, 704, 3), (704, 1024, 2), (1024, 1536, 1)]
    toff, soff, RB = s2lut.record_layout(TS)
    assert toff == [0, 28, 88, 216, 336, 416] and soff == 480 and RB == 512


def test_pack_bits_msb_first():
    bits = torch.tensor([[1, 0, 0, 0, 0, 0, 0, 1, 0, 1, 0, 0, 0, 0, 0, 0]], dtype=torch.bool)
    assert s2lut._pack_bits(bits).tolist() == [[0x81, 0x40]]


def test_gaussian_mse_against_quadrature():
    for levels in ([-0.7979, 0.7979], [-1.5, -0.45, 0.45, 1.5], list(np.linspace(-2, 2, 7))):
        y = np.asarray(levels)
        t = np.concatenate([[-np.inf], (y[1:] + y[:-1]) / 2, [np.inf]])
        q = sum(integrate.quad(lambda x, yy=yy: (x - yy) ** 2 * norm.pdf(x), a, b)[0]
                for a, b, yy in zip(t[:-1], t[1:], y))
        assert abs(s2lut.gaussian_mse(levels) - q) < 1e-9


def test_lloyd_max_matches_max_1960():
    """Max (1960), Table I: optimal Gaussian quantiser output levels and mean-square error."""
    table = {1: ([0.7979], 0.3634), 2: ([0.4528, 1.510], 0.1175), 3: ([0.2451, 0.7560, 1.344, 2.152], 0.03454),
             4: ([0.1284, 0.3881, 0.6568, 0.9424, 1.256, 1.618, 2.069, 2.733], 0.009497)}
    for b, (pos_levels, mse) in table.items():
        y, m = s2lut.lloyd_max(b)
        assert np.allclose(y[len(y) // 2:], pos_levels, atol=6e-4), b
        assert abs(m - mse) < 2e-4 * max(1, mse * 100), b
        assert np.allclose(y, -y[::-1])
    D = s2lut.dist_table()
    assert all(D[b + 1] < D[b] for b in range(8))
    # high-rate limit: D_b * 4^b -> sqrt(3) pi / 2 (Panter-Dite)
    assert abs(D[8] * 4 ** 8 - math.sqrt(3) * math.pi / 2) < 0.1


def test_uniform_codebook_steps():
    """Optimal uniform Gaussian quantiser steps (Max 1960, Table II) to the grid resolution."""
    grid_step = (2.5 - 0.02) / 599
    for b, step in {1: 1.596, 2: 0.9957, 3: 0.5860, 4: 0.3352}.items():
        _, delta, lv, th = s2lut.uniform_cb(b)
        assert abs(delta - step) <= grid_step, (b, delta)
        assert len(lv) == 2 ** b and np.allclose(lv, -lv[::-1]) and np.allclose(th, (lv[1:] + lv[:-1]) / 2)


def test_allocate_is_optimal_on_small_cases():
    """Greedy water-filling (src/tiered.py:145-153) against brute force over every allocation."""
    import itertools

    D = s2lut.dist_table()
    rng = np.random.default_rng(0)
    for _ in range(5):
        lam = np.sort(rng.exponential(1.0, 4 * 32))[::-1]
        lamg = lam.reshape(4, 32).sum(1)
        B = 128 + 32 * int(rng.integers(1, 6))
        T = s2lut.allocate(torch.from_numpy(lam.copy()), B)
        bits = np.concatenate([[b] * ((e - s) // 32) for s, e, b in T])
        assert bits.sum() * 32 == B
        best = min(sum(lamg[i] * D[c[i]] for i in range(4))
                   for c in itertools.product(range(1, 9), repeat=4) if sum(c) * 32 == B)
        assert abs(sum(lamg[i] * D[bits[i]] for i in range(4)) - best) < 1e-12


def test_generator_properties():
    X = datagen.gen(3000, 64, 8, 0.7, seed=0)
    assert X.dtype == torch.float16 and X.shape == (3000, 64)
    n = X.float().norm(dim=1)
    assert torch.allclose(n, torch.ones_like(n), atol=2e-3)
    assert torch.equal(X, datagen.gen(3000, 64, 8, 0.7, seed=0))                       # deterministic
    assert not torch.equal(X[:100], datagen.gen(100, 64, 8, 0.7, seed=1))              # queries differ
    assert torch.equal(datagen.gen(3000, 64, 8, 0.7, seed=0, chunk=1000)[:1000],
                       datagen.gen(1000, 64, 8, 0.7, seed=0, chunk=1000))
    lam = datagen.spectrum(64, 0.7)
    assert abs(lam.mean() - 1) < 1e-6 and np.all(np.diff(lam) < 0)
    Rm = datagen.rotation(64)
    assert np.allclose(Rm @ Rm.T, np.eye(64), atol=1e-5)
    GT = datagen.ground_truth(X, X[:5].float(), 3)
    assert GT[:, 0].tolist() == list(range(5))


def test_emit_buffer_rule():
    """The trellis engines' emit buffer: the reference's max(4096, 16 K) without a batch size, raised
    towards 65,536 entries while the batch's buffers stay within 512 MB."""
    from fanarvse_paper_amd.index import emit_buffer

    assert emit_buffer(None, 200) == 4096 and emit_buffer(None, 400) == 6400
    assert emit_buffer(1, 200) == emit_buffer(1024, 200) == 65536
    assert emit_buffer(2000, 200) == (1 << 29) // 16000
    assert emit_buffer(1 << 20, 400) == 6400            # never below the reference's size
    assert emit_buffer(2000, 5000) == 80000             # nor capped below it for large K


def test_encode_uniform_reference_signature():
    """s2lut.encode_uniform(code, host16, order, c, seed) re-encodes `code`'s tiers with uniform codebooks
    (throughput/s2lut.py:18-29): the records equal those of the table-level encoder on the same inputs, the
    other entries of `code` are kept, and `code` itself is not modified."""
    X = datagen.gen(1200, 128, 8, 0.7, seed=3)
    c = X[:500].float().mean(0)
    lam, V = s2lut.pca_basis(X, c)
    TS = s2lut.allocate(lam, int(2.5 * X.shape[1]))
    order = torch.randperm(X.shape[0], generator=torch.Generator().manual_seed(0)).to(torch.int32)
    lloyd = s2lut.encode_lloyd(X, order, c, V, TS, seed=0)
    lloyd["extra"] = 7
    keys = set(lloyd)
    u = s2lut.encode_uniform(lloyd, X, order, c, seed=0)
    want = s2lut.encode_uniform_tiers(X, order, c, V, TS, seed=0)
    assert torch.equal(u["rec"], want["rec"]) and u["deltas"] == want["deltas"]
    assert u["extra"] == 7 and u["kind"] == "uniform" and u["TS"] == TS
    assert set(lloyd) == keys and lloyd["kind"] == "lloyd"


def test_sorted_cells_from_offsets():
    """build_codes derives each sorted position's cell from the offsets when s1 has no `cell` table, as
    the reference does (throughput/enginei8.py:21)."""
    off = np.array([0, 3, 3, 7, 10], np.int64)
    s1 = dict(off=off, means16=torch.zeros(4, 8, dtype=torch.float16))
    assert index.sorted_cells(s1).tolist() == [0, 0, 0, 2, 2, 2, 2, 3, 3, 3]
    s1["cell"] = torch.arange(10)
    assert index.sorted_cells(s1).tolist() == list(range(10))
