"""The oracle of the routing-free dense scan (throughput/brute.py:41-63), pinned independently of its own
code: the codes against a numpy restatement of the quantizer and its closed-form properties, the scores
against an exact int64 product, the threshold against torch.topk, the emitted set against a full sort of
the dense scores, and the search's top K against Lemma 2 (when K <= cnt <= M, the top K of the buffer is
the top K of the full scan). A planted mistake in the oracle's order of products is caught."""
import numpy as np
import pytest
import torch

from oracle import oracle as o


def rng(seed=0):
    return np.random.default_rng(seed)


def test_quantize_matches_closed_form():
    z = rng().standard_normal((64, 160)).astype(np.float32)
    z[3] = 0.0                       # an all-zero row: scale 1e-12 / 127, codes 0
    z[5, 7] = -40.0                  # a dominant negative entry becomes -127
    q, a = o.quantize_rows(z)
    a2 = (np.maximum(np.abs(z).max(1), np.float32(1e-12)) / np.float32(127)).astype(np.float32)
    assert np.array_equal(a, a2)
    assert np.array_equal(q, np.clip(np.rint(z / a2[:, None]), -127, 127).astype(np.int8))
    assert np.all(np.abs(q).max(1)[np.arange(64) != 3] == 127)   # the largest entry of a row maps to +-127
    assert q[5, 7] == -127 and not q[3].any() and a[3] == np.float32(1e-12) / np.float32(127)


def test_scores_equal_exact_integer_product():
    r = rng(1)
    Q = r.integers(-127, 128, (33, 256), dtype=np.int8)
    Z = r.integers(-127, 128, (301, 256), dtype=np.int8)
    qs = r.random(33).astype(np.float32) * 0.02
    zs = (r.random(301) * 0.02).astype(np.float16)
    S = o.dense_scores(Q, qs, Z, zs)
    acc = Q.astype(np.int64) @ Z.astype(np.int64).T
    assert np.abs(acc).max() < 2 ** 24                       # exact in float32, so the cast is exact too
    ref = (acc.astype(np.float32) * qs[:, None]).astype(np.float32) * zs.astype(np.float32)[None, :]
    assert np.array_equal(S.view(np.uint32), ref.astype(np.float32).view(np.uint32))


def test_planted_product_order_is_caught():
    """A restatement that multiplies the two scales first gives different bits on some entries."""
    r = rng(2)
    Q = r.integers(-127, 128, (16, 128), dtype=np.int8)
    Z = r.integers(-127, 128, (512, 128), dtype=np.int8)
    qs = r.random(16).astype(np.float32) * 0.02
    zs = (r.random(512) * 0.02).astype(np.float16)
    S = o.dense_scores(Q, qs, Z, zs)
    acc = (Q.astype(np.int64) @ Z.astype(np.int64).T).astype(np.float32)
    wrong = acc * (qs[:, None] * zs.astype(np.float32)[None, :]).astype(np.float32)
    assert not np.array_equal(S, wrong.astype(np.float32))


def test_threshold_is_torch_topk():
    S = rng(3).standard_normal((20, 1000)).astype(np.float32)
    S[4, :10] = S[4, 10]             # ties at the threshold
    for r in (1, 7, 40, 1000):
        t = o.row_kth(S, r)
        assert np.array_equal(t, torch.from_numpy(S).topk(r, 1).values[:, -1].numpy())


def test_emit_is_the_set_above_threshold():
    r = rng(4)
    Q = r.integers(-127, 128, (12, 128), dtype=np.int8)
    Z = r.integers(-127, 128, (2000, 128), dtype=np.int8)
    qs = r.random(12).astype(np.float32) * 0.02
    zs = (r.random(2000) * 0.02).astype(np.float16)
    S = o.dense_scores(Q, qs, Z, zs)
    t0 = np.sort(S, 1)[:, -50].copy()
    t0[2] = 1e30                      # nothing passes
    cnt, bval, bpos = o.dense_emit(Q, qs, Z, zs, t0, 40)
    for q in range(12):
        keep = np.nonzero(S[q] >= t0[q])[0]
        assert cnt[q] == len(keep)
        order = keep[np.lexsort((keep, -S[q, keep]))][:40]
        assert np.array_equal(bpos[q, :len(order)], order)
        assert np.array_equal(bval[q, :len(order)], S[q, order])
        assert np.all(bval[q, len(order):] == np.float32(-1e30))


@pytest.mark.parametrize("K", [5, 60])
def test_search_top_k_is_the_full_scan_top_k(K):
    """Lemma 2 for the routing-free scan: a query with K <= cnt <= M gets the top K of all N scores."""
    r = rng(5)
    X = r.standard_normal((3000, 96)).astype(np.float32)
    Z, zs = o.quantize_rows(X)
    zs16 = zs.astype(np.float16)
    q, qs = o.quantize_rows(r.standard_normal((10, 96)).astype(np.float32))
    pos, est, ok, cnt = o.brute_search(q, qs, Z, zs16, K, over=2.0, M=400)
    S = o.dense_scores(q, qs, Z, zs16)
    assert ok.any()
    for i in range(10):
        assert ok[i] == (K <= cnt[i] <= 400)
        if ok[i]:
            top = np.lexsort((np.arange(3000), -S[i]))[:K]
            assert np.array_equal(pos[i], top) and np.array_equal(est[i], S[i, top])
