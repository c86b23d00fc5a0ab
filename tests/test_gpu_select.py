"""GPU stage-1 selection (top-K of each query's emit buffer by (est desc, pos asc), the exactness flag
and the delta-rule count) against the CPU oracle on adversarial buffers: runs of equal estimates at
the K-th value (ties broken by the smaller position), buffers shorter than K, overfull buffers
(cnt > M), buffers staged in LDS (M <= 4096) and read from global memory (the fallback's M = 65,536),
K from 1 to 4096. Results are bit-exact."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib

pytestmark = pytest.mark.gpu

CASES = [(1, 4096), (12, 4096), (64, 4096), (100, 3072), (256, 4096), (400, 4096), (512, 4096), (1000, 4096),
         (1500, 4096), (2048, 4096), (400, 4100), (400, 4094), (4096, 8192), (400, 65536)]


def buffers(B, M, K, seed):
    rng = np.random.default_rng(seed)
    cnt = rng.integers(0, M + M // 4, B).astype(np.int32)
    cnt[:4] = [0, K - 1, K, M + 7]
    bval = np.full((B, M), np.nan, np.float32)  # never read past min(cnt, M)
    bpos = np.full((B, M), -5, np.int32)
    for q in range(B):
        n = min(int(cnt[q]), M)
        if q % 2:  # few distinct values: long runs of ties
            v = rng.integers(-3, 4, n).astype(np.float32) * np.float32(0.25)
        else:
            v = rng.standard_normal(n).astype(np.float32)
        bval[q, :n] = v
        bpos[q, :n] = rng.permutation(10 * M)[:n]
    return bval, bpos, cnt


@pytest.mark.parametrize("B", [37, 80])     # 1024-thread blocks (batches <= 64), 256-thread blocks
@pytest.mark.parametrize("K,M", CASES)
def test_select_matches_oracle(oracle_mod, K, M, B):
    print(f"\n[gpu select] B={B} K={K} M={M}", flush=True)
    bval, bpos, cnt = buffers(B, M, K, K * 13 + M)
    for kd, delta in ((0, None), (min(9, K - 1), 0.07)):
        got = _lib.select(torch.from_numpy(bval).cuda(), torch.from_numpy(bpos).cuda(), torch.from_numpy(cnt).cuda(),
                          K, kd, delta)
        torch.cuda.synchronize()
        want = oracle_mod.select(bval, bpos, cnt, K, kd, delta)
        names = ("pos", "est1", "ok", "ncnt")
        for name, g, w in zip(names, got, want):
            g = g.cpu().numpy()
            if g.dtype == np.float32:
                g, w = g.view(np.uint32), w.view(np.uint32)
            assert np.array_equal(g, w), (name, kd, delta)


@pytest.mark.parametrize("B", [37, 80])          # 1024-thread blocks (batches <= 64), 256-thread blocks
@pytest.mark.parametrize("n1,MB", [(51, 35), (300, 40)])  # n1 x MB = 1,785 (keys staged in LDS), 12,000 (read per pass)
def test_threshold_matches_oracle(oracle_mod, n1, MB, B):
    """t0 from the first-pass block maxima, against the oracle, with the keys staged in LDS and with them
    read from global memory in each radix pass (more than 8,192 keys per query); runs of tied maxima and
    cells shorter than MB blocks, including empty ones."""
    print(f"\n[gpu threshold] B={B} n1={n1} MB={MB}", flush=True)
    rng = np.random.default_rng(n1 * 7 + B)
    NC = 700
    rows = rng.integers(0, 32 * (MB - 2), NC)
    rows[:5] = 0  # empty cells
    off = np.concatenate([[0], np.cumsum(rows)]).astype(np.int32)
    npr = n1 + 3
    probe = np.stack([rng.permutation(NC)[:npr] for _ in range(B)]).astype(np.int32)
    bm = rng.standard_normal((B, n1, MB)).astype(np.float32)
    bm[::2] = np.round(bm[::2] * 4) / 4  # ties
    for r in (1, 240, 3000):
        got = _lib.threshold(torch.from_numpy(bm).cuda(), torch.from_numpy(probe).cuda(), torch.from_numpy(off).cuda(),
                             n1, MB, r)
        torch.cuda.synchronize()
        want = oracle_mod.threshold(bm, probe, off, n1, MB, r)
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32)), r
