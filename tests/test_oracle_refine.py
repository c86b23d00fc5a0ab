"""Pins of the oracle's error-bar classification, exact reads and final top-k (or_refine), following
throughput/enginei8.py:92-95 and src/stage3_zc.py:11-27.

* The exact scores are fp32 dot products of fp16 rows: checked against float64.
* Lemma 3 of the paper (paper/main.tex:230-237): when every interval [est - z*sd, est + z*sd] covers
  the exact score, the final ids are the exact top-k of the candidate set. Checked on random
  instances; a planted mistake (the sure rule using the (k+2)-th instead of the (k+1)-th largest
  upper bound) breaks it on a constructed instance.
* reads = number of ambiguous candidates, brute-forced from the definition.
"""
import numpy as np

from tests.conftest import fp16_bits


def _instance(rng, B=8, K=40, d=64, N=500):
    H = rng.standard_normal((N, d)).astype(np.float16)
    Q = rng.standard_normal((B, d)).astype(np.float32)
    pos = np.stack([rng.choice(N, K, replace=False) for _ in range(B)]).astype(np.int32)
    order = rng.permutation(N).astype(np.int32)
    ids = order[pos]
    exact = np.einsum("bkd,bd->bk", H[ids].astype(np.float64), Q.astype(np.float64))
    sd = rng.uniform(0.05, 0.5, (B, K)).astype(np.float32)
    return H, Q, pos, order, ids, exact, sd


def _brute(est, sd, z, k):
    """Sure / ambiguous sets of throughput/enginei8.py:92-93 in float32 arithmetic."""
    est, sd = est.astype(np.float32), sd.astype(np.float32)
    t = (np.float32(z) * sd).astype(np.float32)
    lo, hi = (est - t).astype(np.float32), (est + t).astype(np.float32)
    hk1 = -np.sort(-hi, 1)[:, k:k + 1]
    lk = -np.sort(-lo, 1)[:, k - 1:k]
    sure = lo > hk1
    amb = (hi >= lk) & ~sure
    return sure, amb


def test_exact_dot_and_reads(oracle_mod):
    rng = np.random.default_rng(3)
    H, Q, pos, order, ids, exact, sd = _instance(rng)
    z, k = 1.5, 5
    est = (exact + rng.uniform(-1, 1, exact.shape) * 1.4 * sd).astype(np.float32)
    oids, I, scores, reads = oracle_mod.refine(est, sd, pos, order, fp16_bits(H), Q, z, k)
    assert np.array_equal(oids, ids)
    sure, amb = _brute(est, sd, z, k)
    assert np.array_equal(reads, amb.sum(1))
    slot = {(b, int(i)): j for b in range(len(ids)) for j, i in enumerate(ids[b])}
    for b in range(len(I)):
        for j in range(k):
            s = slot[(b, int(I[b, j]))]
            if amb[b, s]:
                assert abs(scores[b, j] - exact[b, s]) <= 1e-5 * (1 + abs(exact[b, s]))
            else:
                assert sure[b, s] and scores[b, j] == est[b, s]


def test_lemma3_coverage_implies_exact_topk(oracle_mod):
    rng = np.random.default_rng(9)
    z, k = 2.0, 10
    for trial in range(6):
        H, Q, pos, order, ids, exact, sd = _instance(rng, B=6, K=60, d=96)
        # errors strictly inside the interval: every interval covers the exact score
        est = (exact + rng.uniform(-0.9, 0.9, exact.shape) * z * sd).astype(np.float32)
        _, I, _, _ = oracle_mod.refine(est, sd, pos, order, fp16_bits(H), Q, z, k)
        want = np.take_along_axis(ids, np.argsort(-exact, 1, kind="stable")[:, :k], 1)
        assert np.array_equal(np.sort(I, 1), np.sort(want, 1)), trial


def test_lemma3_planted_sure_rule_mistake(oracle_mod):
    """Planted mistake: `sure = lo > (k+2)-th largest hi` (one rank too lenient). On this covered instance
    it declares both leading candidates sure and returns the wrong top-1; the oracle's rule reads both
    and returns the exact top-1."""
    k, z = 1, 1.0
    d = 8
    H = np.zeros((3, d), np.float16)
    H[:, 0] = [1.0, 1.2, 0.0]
    Q = np.zeros((1, d), np.float32)
    Q[0, 0] = 1.0
    exact = H[:, 0].astype(np.float64)[None]
    est = np.array([[1.1, 1.0, 0.0]], np.float32)
    sd = np.array([[0.1, 0.25, 0.01]], np.float32)
    lo, hi = est - z * sd, est + z * sd
    assert np.all((lo <= exact) & (exact <= hi))            # every interval covers the exact score
    pos = np.array([[0, 1, 2]], np.int32)
    order = np.arange(3, dtype=np.int32)
    _, I, _, reads = oracle_mod.refine(est, sd, pos, order, fp16_bits(H), Q, z, k)
    assert I[0, 0] == 1 and reads[0] == 2
    wrong_sure = lo > -np.sort(-hi, 1)[:, k + 1:k + 2]
    score_wrong = np.where(wrong_sure, est + 10, -1e9)
    assert wrong_sure[0, 0] and wrong_sure[0, 1] and np.argmax(score_wrong) != np.argmax(exact)
