"""Pins of the oracle's stage-1 functions (query code, int8 estimate, first pass, threshold, emit,
selection, pairs, static blocks, routing) against closed forms, brute force and Lemma 2 of the paper
(paper/main.tex:206-213), with planted mistakes showing each check can fail."""
from fractions import Fraction

import numpy as np
import pytest

from tests.conftest import fp16_bits


def f32_round(fr):
    """Correctly rounded (ties to even) float32 of an exact Fraction."""
    x = np.float32(float(fr))  # float() is correctly rounded to float64; fix the double rounding below
    best = x
    for y in (np.nextafter(x, np.float32(-np.inf)), np.nextafter(x, np.float32(np.inf))):
        dy, db = abs(Fraction(float(y)) - fr), abs(Fraction(float(best)) - fr)
        if dy < db or (dy == db and (int(np.float32(y).view(np.uint32)) & 1) == 0):
            best = y
    return np.float32(best)


def exact_fma32(a, b, c):
    return f32_round(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def est_closed_form(q8, qs, Z, zs, qcp):
    """est = fma(f32(acc) * qs, zs, qcp) with acc the exact int8 dot product (throughput/ivf8c_kern.py:14)."""
    acc = int(np.dot(q8.astype(np.int64), Z.astype(np.int64)))
    t = np.float32(np.float32(acc) * np.float32(qs))
    return exact_fma32(t, zs, qcp)


# ------------------------------------------------------------------------------------------ query code
def test_query_code_matches_float64_projection(tiny, oracle_mod):
    Qn, Vr, c = tiny["Qn"], tiny["idx"]["Vr"], tiny["idx"]["c"]
    q8, qs, qc, qh = oracle_mod.query_prep(Qn, Vr, c)
    z64 = Qn.astype(np.float64) @ Vr.astype(np.float64)
    assert np.allclose(oracle_mod.project(Qn, Vr), z64, atol=1e-5)
    amax = np.abs(z64).max(1)
    assert np.allclose(qs, amax / 127, rtol=1e-5)
    assert np.all(np.abs(q8).max(1) == 127), "the largest coordinate must map to +-127"
    err = np.abs(q8 * qs[:, None].astype(np.float64) - z64)
    assert np.all(err <= qs[:, None] * 0.5 * (1 + 1e-4) + 1e-6)
    assert np.allclose(qc, Qn.astype(np.float64) @ c.astype(np.float64), atol=1e-6)
    assert np.array_equal(qh, fp16_bits(Qn))
    # planted mistake: scale by 128 instead of 127 -> the +-127 property fails
    q_bad = np.clip(np.rint(z64 / (amax[:, None] / 128)), -127, 127)
    assert not np.all(np.abs(q_bad).max(1) == 127) or not np.all(np.abs(q_bad * (amax / 128)[:, None] - z64) <= qs[:, None] * 0.5)


def test_build_codes_quantisation(tiny, oracle_mod):
    idx, s1, X = tiny["idx"], tiny["s1"], tiny["X"].numpy()
    order, cell = s1["order"].numpy(), s1["cell"].numpy()
    means = s1["means16"].numpy().astype(np.float64)
    sel = np.arange(0, len(order), 97)
    x = X[order[sel]].astype(np.float64) - means[cell[sel]]
    z64 = x @ idx["Vr"].astype(np.float64)
    Zs, zss = idx["Z"][sel].astype(np.float64), idx["zs"][sel].astype(np.float64)
    assert np.allclose(zss, np.abs(z64).max(1) / 127, rtol=1e-5)
    assert np.all(np.abs(Zs).max(1) == 127)
    assert np.all(np.abs(Zs * zss[:, None] - z64) <= zss[:, None] * 0.5 * (1 + 1e-4) + 1e-6)


# ------------------------------------------------------------------------------------------ stage 1
@pytest.fixture(scope="module")
def s1run(tiny, oracle_mod):
    idx = tiny["idx"]
    Qn = tiny["Qn"]
    q8, qs, qc, qh = oracle_mod.query_prep(Qn, idx["Vr"], idx["c"])
    QM = oracle_mod.fp16_gemm_nt(qh, idx["meansN"])
    K, nprobe = 60, 8
    probe = oracle_mod.route_topk(QM, nprobe)
    st = oracle_mod.stage1(idx, q8, qs, QM, probe, K, dict(MSZ=4096, RHO=0.6), delta=0.07, kd=9)
    return dict(q8=q8, qs=qs, QM=QM, probe=probe, K=K, st=st)


def _probed_rows(idx, probe_row, QM_row, q8, qs):
    """(est, row) of every row of the probed cells, closed form."""
    out = []
    for c in probe_row:
        qcp = np.float32(np.float32(QM_row.view(np.float16)[c]) * idx["mnorm"][c])
        for r in range(idx["off"][c], idx["off"][c + 1]):
            out.append((est_closed_form(q8, qs, idx["Z"][r], idx["zs"][r], qcp), r))
    return out


def test_int8_estimates_and_block_maxima(tiny, s1run):
    idx, st = tiny["idx"], s1run["st"]
    for q in (0, 7, 31):
        n1 = st["n1"]
        for j in range(n1):
            c = s1run["probe"][q, j]
            qcp = np.float32(np.float32(s1run["QM"][q].view(np.float16)[c]) * idx["mnorm"][c])
            cs, ce = idx["off"][c], idx["off"][c + 1]
            for b in range((ce - 1) // 32 - cs // 32 + 1 if ce > cs else 0):
                blk = cs // 32 + b
                rows = [r for r in range(blk * 32, blk * 32 + 32) if cs <= r < ce]
                m = max(est_closed_form(s1run["q8"][q], s1run["qs"][q], idx["Z"][r], idx["zs"][r], qcp) for r in rows)
                assert st["bm"][q, j, b].view(np.uint32) == np.float32(m).view(np.uint32)


def test_threshold_rule_cases(oracle_mod):
    off = np.array([0, 70, 70, 100], np.int32)  # cell 0: blocks 0,1,2; cell 1 empty; cell 2: rows 70..99 -> blocks 2,3
    MB = 4
    probe = np.array([[0, 2, 1], [1, 2, 0], [1, 1, 1]], np.int32)
    bm = np.full((3, 3, MB), -1e30, np.float32)
    bm[0, 0, :3] = [0.5, 0.9, 0.1]
    bm[0, 1, :2] = [0.7, 0.3]
    bm[1, 1, :2] = [0.2, 0.4]
    bm[1, 2, :3] = [0.6, 0.0, 0.8]
    n1 = 2
    t0 = oracle_mod.threshold(bm[:, :n1].copy(), probe, off, n1, MB, 3)
    assert t0[0] == np.float32(0.5)  # 3rd largest of {0.5,0.9,0.1,0.7,0.3}
    assert t0[1] == np.float32(0.2)  # only 2 valid values (cell 1 empty): the smaller valid one
    assert t0[2] == np.float32(1e30)  # no valid value
    t0b = oracle_mod.threshold(bm[:, :n1].copy(), probe, off, n1, MB, 100)
    assert t0b[0] == np.float32(0.1)  # r capped by the valid count
    # planted mistake: "t0 = 1e30 whenever fewer than r maxima are valid" differs on query 1
    wrong = np.float32(1e30)
    assert t0[1] != wrong


def test_threshold_out_of_range_probe_ids(oracle_mod):
    """A probe id outside [0, NC) (a stale or foreign list) reads no cell offsets: the query gets t0 = 1e30,
    so it emits nothing and is flagged; the other queries keep their thresholds."""
    off = np.array([0, 70, 70, 100], np.int32)
    MB = 4
    bm = np.full((4, 2, MB), -1e30, np.float32)
    bm[:, 0, :3] = [0.5, 0.9, 0.1]
    bm[:, 1, :2] = [0.7, 0.3]
    good = np.array([[0, 2, 1]] * 4, np.int32)
    t_good = oracle_mod.threshold(bm, good, off, 2, MB, 3)
    bad = good.copy()
    bad[1, 1] = 3          # == NC
    bad[2, 0] = -1
    bad[3, 2] = 1 << 20    # past n1: not read by the threshold
    t_bad = oracle_mod.threshold(bm, bad, off, 2, MB, 3)
    assert t_bad[0] == t_good[0] == np.float32(0.5)
    assert t_bad[1] == t_bad[2] == np.float32(1e30)
    assert t_bad[3] == t_good[3]


def test_emit_is_threshold_set_and_lemma2(tiny, s1run):
    """cnt = #{probed rows: est >= t0}; for ok queries the top K of the buffer equals the brute-force top K
    of all probed rows (Lemma 2)."""
    idx, st, K = tiny["idx"], s1run["st"], s1run["K"]
    nok = 0
    for q in range(0, len(s1run["probe"]), 5):
        allrows = _probed_rows(idx, s1run["probe"][q], s1run["QM"][q], s1run["q8"][q], s1run["qs"][q])
        t0 = st["t0"][q]
        assert st["cnt"][q] == sum(1 for e, _ in allrows if e >= t0)
        ranked = sorted(allrows, key=lambda x: (-float(x[0]), x[1]))
        if st["ok"][q]:
            nok += 1
            assert [r for _, r in ranked[:K]] == st["pos"][q].tolist()
            assert np.array_equal(np.array([e for e, _ in ranked[:K]], np.float32).view(np.uint32),
                                  st["est1"][q].view(np.uint32))
    assert nok > 0


def test_select_canonical_order_fillers_and_delta(oracle_mod):
    bval = np.array([[0.5, 0.9, 0.5, 0.2, -1e30, -1e30], [0.3, 0.1, 0.0, 0.0, 0.0, 0.0]], np.float32)
    bpos = np.array([[7, 3, 2, 9, 0, 0], [5, 6, 0, 0, 0, 0]], np.int32)
    cnt = np.array([4, 2], np.int32)  # row 0 is not in canonical order: select sorts
    pos, est1, ok, ncnt = oracle_mod.select(bval, bpos, cnt, 3, 1, 0.3)
    assert pos[0].tolist() == [3, 2, 7] and est1[0].tolist() == [np.float32(0.9), np.float32(0.5), np.float32(0.5)]
    assert pos[1].tolist() == [5, 6, 0] and est1[1, 2] == np.float32(-1e30)
    assert ok.tolist() == [1, 0]
    assert ncnt.tolist() == [3, 2]  # row 0: >= 0.5-0.3 -> 3; row 1: >= 0.1-0.3 -> 2 (filler excluded)
    _, _, ok2, ncnt2 = oracle_mod.select(bval, bpos, cnt, 3, 1, None)
    assert ncnt2.tolist() == [3, 3] and ok2.tolist() == [1, 0]
    _, _, ok3, _ = oracle_mod.select(bval, bpos, np.array([7, 2], np.int32), 3, 1, None)
    assert ok3[0] == 0  # cnt > M overflows


def test_select_is_sorted_topk_bruteforce(oracle_mod):
    """Top-K of the first min(cnt, M) entries of unsorted buffers by (est desc, pos asc), against a numpy
    lexsort; rows with long runs of equal estimates, short rows and overfull rows (cnt > M)."""
    rng = np.random.default_rng(4)
    B, M, K = 40, 64, 10
    cnt = rng.integers(0, M + 20, B).astype(np.int32)
    bval = np.where(np.arange(B)[:, None] % 2 == 1, rng.integers(-2, 3, (B, M)) * np.float32(0.5),
                    rng.standard_normal((B, M))).astype(np.float32)
    bpos = np.stack([rng.permutation(1000)[:M] for _ in range(B)]).astype(np.int32)
    pos, est1, ok, _ = oracle_mod.select(bval, bpos, cnt, K, 0, None)
    for q in range(B):
        n = min(int(cnt[q]), M)
        o = np.lexsort((bpos[q, :n], -bval[q, :n].astype(np.float64)))[:K]
        want_p = np.concatenate([bpos[q, o], np.zeros(K - len(o), np.int32)])
        want_e = np.concatenate([bval[q, o], np.full(K - len(o), -1e30, np.float32)])
        assert np.array_equal(pos[q], want_p) and np.array_equal(est1[q], want_e), q
    assert np.array_equal(ok, ((cnt >= K) & (cnt <= M)).astype(np.uint8))
    # a planted mistake (ties broken by the larger position) fails the same check
    q = next(q for q in range(1, B, 2) if min(cnt[q], M) > K)
    n = min(int(cnt[q]), M)
    bad = np.lexsort((-bpos[q, :n], -bval[q, :n].astype(np.float64)))[:K]
    assert not np.array_equal(pos[q], bpos[q, bad])


def test_pairs_against_bruteforce(oracle_mod):
    rng = np.random.default_rng(5)
    NC, B, n = 11, 9, 4
    probe = np.stack([rng.permutation(NC)[:n] for _ in range(B)]).astype(np.int32)
    QM = fp16_bits(rng.standard_normal((B, NC)).astype(np.float32))
    mnorm = rng.random(NC).astype(np.float32) + 0.5
    qid, coff, ccnt, qcp, o = oracle_mod.pairs(probe, NC, QM, mnorm)
    for c in range(NC):
        qs = sorted(q for q in range(B) if c in probe[q])
        assert ccnt[c] == len(qs)
        assert qid[coff[c]:coff[c] + ccnt[c]].tolist() == qs
        for i, q in enumerate(qs):
            want = np.float32(np.float32(QM[q].view(np.float16)[c]) * mnorm[c])
            assert qcp[coff[c] + i] == want


def test_static_blocks_enumeration(oracle_mod):
    off = np.array([0, 5, 5, 40, 41, 100, 131], np.int64)
    cell, blk, ps, pe, MB = oracle_mod.static_blocks(off)
    want = sorted({(c, r // 32) for c in range(len(off) - 1) for r in range(off[c], off[c + 1])})
    assert list(zip(cell.tolist(), blk.tolist())) == want
    assert all(ps[i] == off[cell[i]] and pe[i] == off[cell[i] + 1] for i in range(len(cell)))
    assert MB == (59 + 31) // 32 + 1


def test_route_topk_ties_and_signed_zero(oracle_mod):
    vals = np.array([[0.5, -0.0, 0.5, 0.25, 0.0, -1.0, 0.5, 0.25]], np.float32)
    probe = oracle_mod.route_topk(fp16_bits(vals), 6)
    want = sorted(range(8), key=lambda c: (-float(vals[0, c]), c))[:6]
    assert probe[0].tolist() == want == [0, 2, 6, 3, 7, 1]


def test_routing_variants_brute_force(oracle_mod):
    """The oracle's routing variants (throughput/enginei8.py:66-76) against a numpy sort by (key desc,
    cell asc): fp16 keys of (float)QM * inv_mnorm (ROUTE16), fp32 keys, and the cell-ordered UNSORTED list."""
    rng = np.random.default_rng(11)
    B, NC, npr = 40, 96, 17
    QM = (rng.standard_normal((B, NC)) * 0.3).astype(np.float16)
    QM[3, :20] = QM[3, 20]                       # ties
    inv = (1.0 / (0.5 + rng.random(NC))).astype(np.float32)
    inv[5] = inv[6]
    idx = dict(inv_mnorm=inv)

    def brute(keys):
        return np.stack([np.lexsort((np.arange(NC), -keys[b]))[:npr] for b in range(B)]).astype(np.int32)

    k16 = (QM.astype(np.float32) * inv[None, :]).astype(np.float16).astype(np.float32)
    k32 = QM.astype(np.float32) * inv[None, :]
    p16 = oracle_mod.route(idx, QM.view(np.uint16), npr, dict(NROUTE=False, ROUTE16=True))
    p32 = oracle_mod.route(idx, QM.view(np.uint16), npr, dict(NROUTE=False, ROUTE16=False))
    pu = oracle_mod.route(idx, QM.view(np.uint16), npr, dict(NROUTE=False, ROUTE16=False, UNSORTED=True))
    assert np.array_equal(p16, brute(k16)) and np.array_equal(p32, brute(k32))
    assert np.array_equal(pu, np.sort(brute(k32), axis=1))
    assert not np.array_equal(p16, p32)          # the fp16 rounding changes some lists
