"""Pins of the oracle's trellis engine: the trellis table (src/trellis.py:12-15), the word format
(src/trellis_scan.py:10-18, 36-44), the Viterbi encoder (src/viterbi_fused.py:7-46) against brute force
over every bit stream of short segments, the trellis estimate against float64, routing on fp32 keys, and
the Lloyd-Max tiered score (src/tiered_fused.py:47-72) against the direct codeword sum."""
import itertools

import numpy as np
import pytest
from scipy.stats import norm

from fanarvse_paper_amd import trellis
from tests.conftest import fp16_bits


def test_table_is_a_permuted_gaussian_grid():
    T = trellis.make_table(10)
    assert T.dtype == np.float32 and T.shape == (1024,)
    grid = norm.ppf((np.arange(1024) + 0.5) / 1024).astype(np.float32)
    assert np.array_equal(np.sort(T), grid)
    perm = np.random.default_rng(0).permutation(1024)
    assert np.array_equal(T, grid[perm])
    assert abs(float(T.mean())) < 1e-6


def _stream_paths(bits, L):
    n, nb = bits.shape
    R = nb - L + 1
    wts = 1 << np.arange(L - 1, -1, -1)
    return np.stack([(bits[:, j:j + L] * wts).sum(1) for j in range(R)], 1)


def test_words_round_trip(oracle_mod):
    rng = np.random.default_rng(3)
    for L in (8, 10):
        bits = rng.integers(0, 2, (5, 256 + L - 1))
        path = _stream_paths(bits, L)
        w = trellis.paths_to_words(path, L)
        assert w.shape == (5, trellis.n_words(256, L))
        # word bits are the stream, first bit most significant
        flat = np.unpackbits(w.astype(">u4").view(np.uint8), axis=1, bitorder="big")[:, :256 + L - 1]
        assert np.array_equal(flat, bits)
        assert np.array_equal(oracle_mod.trellis_decode(w, 256, L), path)
        assert np.array_equal(trellis.decode_states(w, 256, L), path)


def _viterbi_brute(x, tab, L):
    """min over every stream of sum_j (x_j - tab[state_j])^2, accumulated in f32 like the encoder, ties broken
    as the encoder does; returns the cost of the optimum."""
    n = len(x)
    best = None
    for bits in itertools.product((0, 1), repeat=n + L - 1):
        path = _stream_paths(np.array([bits]), L)[0]
        c = np.float32(0)
        for j in range(n):
            d = np.float32(x[j] - tab[path[j]])
            c = np.float32(c + d * d)
        if best is None or c < best[0]:
            best = (c, path)
    return best


def test_viterbi_matches_brute_force_on_short_segments(oracle_mod):
    """The C encoder (any R) on n = 6 coordinates, L = 3, against brute force over all 2^8 streams: the same
    minimum cost (f32, accumulated in coordinate order) and a path of that cost. Planted mistake: states that
    take the new bit at the top (s' = (s >> 1) | b << (L-1)) describe a different trellis, and the encoder's
    cost is not reachable by it on some instance."""
    rng = np.random.default_rng(5)
    L, n = 3, 6
    S = 2 ** L
    differs = 0
    for trial in range(20):
        tab = rng.standard_normal(S).astype(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        _, _, path = oracle_mod.trellis_encode(x[None], np.ones(1, np.float32), tab, L)
        path = path[0]
        assert np.all((path[1:] >> 1) == (path[:-1] & (S // 2 - 1)))
        c = np.float32(0)
        for j in range(n):
            d = np.float32(x[j] - tab[path[j]])
            c = np.float32(c + d * d)
        bc, _ = _viterbi_brute(x, tab, L)
        assert c == bc, trial
        # planted: the mirrored trellis (new bit enters at the top)
        best = None
        for bits in itertools.product((0, 1), repeat=n + L - 1):
            st = [int("".join(map(str, bits[j:j + L][::-1])), 2) for j in range(n)]
            cc = np.float32(0)
            for j in range(n):
                d = np.float32(x[j] - tab[st[j]])
                cc = np.float32(cc + d * d)
            best = cc if best is None or cc < best else best
        differs += best != bc
    assert differs > 0


def test_oracle_encoder_is_optimal_and_consistent(oracle_mod):
    """The C encoder's path cost is never above the cost of perturbed paths, its words decode to its path,
    and the scale makes scale * <Zs, Y> / sqrt(R) reproduce |z| * fip-weighted norm (engine_cell.py:21-22)."""
    rng = np.random.default_rng(7)
    L, R = 8, 256
    tab = (0.9 * trellis.make_table(L)).astype(np.float32)
    Zs = rng.standard_normal((4, R)).astype(np.float32)
    Zs *= np.sqrt(R) / np.linalg.norm(Zs, axis=1, keepdims=True)
    nz = rng.uniform(0.5, 2, 4).astype(np.float32)
    w, s1, paths = oracle_mod.trellis_encode(Zs, nz, tab, L)
    assert np.array_equal(trellis.decode_states(w, R, L), paths)
    # valid trellis paths: consecutive states overlap in L-1 bits
    assert np.all((paths[:, 1:] >> 1) == (paths[:, :-1] & ((1 << (L - 1)) - 1)))
    cost = ((Zs - tab[paths]) ** 2).sum(1)
    for v in range(4):
        for _ in range(20):   # flip one stream bit: never cheaper
            bits = np.unpackbits(w[v:v + 1].astype(">u4").view(np.uint8), axis=1, bitorder="big")[0, :R + L - 1].copy()
            bits[rng.integers(0, R + L - 1)] ^= 1
            p2 = _stream_paths(bits[None], L)[0]
            assert ((Zs[v] - tab[p2]) ** 2).sum() >= cost[v] - 1e-3
    Y = tab[paths].astype(np.float64)
    yn = np.linalg.norm(Y, axis=1)
    fip = (Zs * Y).sum(1) / (yn * np.sqrt(R))
    assert np.allclose(s1.view(np.float16).astype(np.float64), nz / (fip * yn), rtol=1e-3)


def test_trellis_estimate_matches_float64(oracle_mod):
    rng = np.random.default_rng(9)
    L, R = 10, 256
    tab = (0.95 * trellis.make_table(L)).astype(np.float32)
    N = 64
    bits = rng.integers(0, 2, (N, R + L - 1))
    words = trellis.paths_to_words(_stream_paths(bits, L), L)
    scale1 = fp16_bits(rng.uniform(0.05, 0.2, N).astype(np.float32))
    off = np.array([0, 30, 64], np.int32)
    Qr = rng.standard_normal((3, R)).astype(np.float32)
    QM = fp16_bits(rng.standard_normal((3, 2)).astype(np.float32))
    probe = np.array([[0, 1], [1, 0], [0, 1]], np.int32)
    MB = 3
    bm = oracle_mod.tr_first_pass(Qr, probe, 2, off, words, scale1, tab, L, QM, MB)
    v = tab[trellis.decode_states(words, R, L)].astype(np.float64)
    est = (v @ Qr.astype(np.float64).T).T * scale1.view(np.float16).astype(np.float64)[None]
    for q in range(3):
        for j in range(2):
            c = probe[q, j]
            cs, ce = off[c], off[c + 1]
            qcp = float(QM[q].view(np.float16)[c])
            for b in range((ce - 1) // 32 - cs // 32 + 1):
                rows = [r for r in range((cs // 32 + b) * 32, (cs // 32 + b) * 32 + 32) if cs <= r < ce]
                want = max(est[q, r] + qcp for r in rows)
                assert abs(bm[q, j, b] - want) < 1e-4 * (1 + abs(want))
    # the emitted set is exactly {rows of probed cells with est >= t0}
    t0 = np.array([bm[0, 0, 0], -1e30, 1e30], np.float32)
    cnt, bval, bpos = oracle_mod.tr_emit(Qr, probe, off, words, scale1, tab, L, QM, t0, 128)
    assert cnt[1] == 64 and cnt[2] == 0
    assert cnt[0] >= 1 and np.all(bval[0, :cnt[0]] >= t0[0])


def test_trellis_fp16_operands(oracle_mod):
    """half=True rounds both operands of every product to fp16 (the reference's `.to(tl.float16)` before
    tl.dot, src/s1cell.py:127,131-132): the estimates then match the float64 dot of the rounded operands to
    fp32 accumulation error, and differ from the fp32-operand estimate by far more. Rounding only one of
    the two operands (a planted mistake) fails the first check."""
    rng = np.random.default_rng(19)
    L, R = 10, 256
    tab = (0.95 * trellis.make_table(L)).astype(np.float32)
    N = 96
    bits = rng.integers(0, 2, (N, R + L - 1))
    words = trellis.paths_to_words(_stream_paths(bits, L), L)
    scale1 = fp16_bits(rng.uniform(0.05, 0.2, N).astype(np.float32))
    off = np.array([0, N], np.int32)
    Qr = rng.standard_normal((2, R)).astype(np.float32)
    QM = fp16_bits(np.zeros((2, 1), np.float32))
    probe = np.zeros((2, 1), np.int32)
    t0 = np.full(2, -1e30, np.float32)
    v = tab[trellis.decode_states(words, R, L)]
    s = scale1.view(np.float16).astype(np.float64)
    r16 = lambda x: x.astype(np.float16).astype(np.float64)
    want16 = (r16(v) @ r16(Qr).T).T * s[None]
    want32 = (v.astype(np.float64) @ Qr.astype(np.float64).T).T * s[None]
    one_side = (r16(v) @ Qr.astype(np.float64).T).T * s[None]
    for half, want in ((True, want16), (False, want32)):
        cnt, bval, bpos = oracle_mod.tr_emit(Qr, probe, off, words, scale1, tab, L, QM, t0, N, half=half)
        assert np.all(cnt == N)
        got = np.empty((2, N))
        for q in range(2):
            got[q, bpos[q]] = bval[q]
        err = np.abs(got - want) / (1 + np.abs(want))
        assert err.max() < 2e-6
        if half:
            assert (np.abs(want16 - want32) / (1 + np.abs(want32))).mean() > 20 * err.max()
            assert (np.abs(got - one_side) / (1 + np.abs(one_side))).max() > 10 * err.max()


def test_route_scaled_orders_by_fp32_key(oracle_mod):
    rng = np.random.default_rng(2)
    QM = fp16_bits(rng.standard_normal((4, 50)).astype(np.float32))
    QM[0, 7] = QM[0, 9]  # a tie
    sc = rng.uniform(0.5, 2, 50).astype(np.float32)
    sc[7] = sc[9]
    probe = oracle_mod.route_topk_scaled(QM, sc, 12)
    for q in range(4):
        key = QM[q].view(np.float16).astype(np.float32) * sc
        want = sorted(range(50), key=lambda c: (-float(key[c]), c))[:12]
        assert probe[q].tolist() == want


def test_lloyd_tiered_score_matches_direct_sum(oracle_mod):
    from fanarvse_paper_amd import s2lut

    rng = np.random.default_rng(4)
    TS = [(0, 32, 4), (32, 96, 2), (96, 128, 1)]
    toff, soff, RB = s2lut.record_layout(TS)
    N, B, K = 200, 3, 20
    codes = np.concatenate([rng.integers(0, 2 ** b, (N, e - s)) for s, e, b in TS], 1)
    rec = np.zeros((N, RB), np.uint8)
    for t, (s, e, b) in enumerate(TS):
        kb = (e - s) // 8
        for p in range(b):
            bit = (codes[:, s:e] >> (b - 1 - p)) & 1
            rec[:, toff[t] + p * kb: toff[t] + (p + 1) * kb] = np.packbits(bit.astype(np.uint8), axis=1, bitorder="big")
    ss = np.stack([rng.uniform(0.5, 1.5, (N, 3)), rng.uniform(0, 0.1, (N, 3))], 2).astype(np.float16)
    rec[:, soff:soff + 12] = ss.reshape(N, -1).view(np.uint8)
    cb = np.zeros((3, 256), np.float32)
    for t, (_, _, b) in enumerate(TS):
        cb[t, :2 ** b] = s2lut.lloyd_cb(b)[0]
    Zq = rng.standard_normal((B, 128)).astype(np.float32)
    qc = rng.standard_normal(B).astype(np.float32)
    pos = np.stack([rng.choice(N, K, replace=False) for _ in range(B)]).astype(np.int32)
    est, sd = oracle_mod.tiered_score(pos, qc, Zq, rec, soff, TS, toff, cb)
    s64 = ss.astype(np.float64)
    for q in range(B):
        for m in range(K):
            r = pos[q, m]
            want = float(qc[q])
            var = 0.0
            for t, (s, e, b) in enumerate(TS):
                want += s64[r, t, 0] * float((cb[t, codes[r, s:e]].astype(np.float64) * Zq[q, s:e]).sum())
                var += float((Zq[q, s:e].astype(np.float64) ** 2).sum()) * s64[r, t, 1] ** 2
            assert abs(est[q, m] - want) < 1e-4 * (1 + abs(want))
            assert abs(sd[q, m] - np.sqrt(var)) < 1e-4 * (1 + np.sqrt(var))
    # planted mistake: LSB-first planes break the identity
    rec2 = rec.copy()
    for t, (s, e, b) in enumerate(TS):
        kb = (e - s) // 8
        if b > 1:
            blk = rec2[:, toff[t]:toff[t] + b * kb].reshape(N, b, kb)[:, ::-1].reshape(N, -1)
            rec2[:, toff[t]:toff[t] + b * kb] = blk
    est2, _ = oracle_mod.tiered_score(pos, qc, Zq, rec2, soff, TS, toff, cb)
    assert np.abs(est2 - est).max() > 0.1
