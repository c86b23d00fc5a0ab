"""End-to-end properties of the oracle pipeline on the tiny index (throughput/enginei8.py:61-120):
recall against the exact ground truth, the standardised error of the stage-2 estimates (the paper's
error-bar calibration, paper/main.tex:219-226; the reference measured std 0.91, results/v19_z.json), and
the fallback of queries whose exactness flag is off."""
import numpy as np
import pytest


@pytest.fixture(scope="module")
def run(tiny, oracle_mod):
    K, z, nprobe, k = 120, 2.0, 12, 10
    out = oracle_mod.pipeline(tiny["idx"], tiny["Qn"], K, z, nprobe, k, knobs=dict(MSZ=3072))
    return dict(out=out, K=K, z=z, k=k, nprobe=nprobe)


def test_recall_against_exact_ground_truth(tiny, oracle_mod, run):
    rec = oracle_mod.recall(run["out"]["I"], tiny["GT"], 10)
    assert rec >= 0.95, rec


def test_standardised_error_of_stage2(tiny, run):
    out = run["out"]
    H = tiny["X"].numpy().astype(np.float64)
    Q = tiny["Qn"].astype(np.float64)
    m = out["ncnt"]
    errs = []
    for q in range(len(Q)):
        n = int(m[q])
        ids = out["ids"][q, :n]
        exact = H[ids] @ Q[q]
        errs.append((exact - out["est"][q, :n]) / out["sd"][q, :n])
    e = np.concatenate(errs)
    assert len(e) > 1000
    assert abs(e.mean()) < 0.3 and 0.3 < e.std() < 1.3, (e.mean(), e.std())
    # tail bound of the paper's corollary: P(|e| > z) <= 2 exp(-z^2 / 2)
    for zz in (1.5, 2.0, 3.0):
        assert np.mean(np.abs(e) > zz) <= 2 * np.exp(-zz * zz / 2) + 0.01


def test_fallback_recomputes_flagged_queries(tiny, oracle_mod, run):
    """A buffer smaller than the emitted count flags queries (cnt > M); the fallback (rho = 1, beta = 1.5,
    M = 65,536, fp32 LUT, no delta rule) must clear the flag and give at least the same recall."""
    idx = tiny["idx"]
    out = oracle_mod.pipeline(idx, tiny["Qn"], run["K"], run["z"], run["nprobe"], run["k"],
                              knobs=dict(MSZ=run["K"] + 5))
    assert len(out["bad"]) > 0
    assert np.all(out["fallback_ok"] == 1)
    assert oracle_mod.recall(out["I"], tiny["GT"], 10) >= oracle_mod.recall(run["out"]["I"], tiny["GT"], 10) - 0.02
    # unflagged queries are untouched by the fallback
    good = np.setdiff1d(np.arange(len(out["I"])), out["bad"])
    base = oracle_mod.pipeline(idx, tiny["Qn"][good], run["K"], run["z"], run["nprobe"], run["k"],
                               knobs=dict(MSZ=run["K"] + 5), fallback=False)
    assert np.array_equal(out["I"][good], base["I"])
