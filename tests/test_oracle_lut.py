"""Pins of the oracle's LUT stage 2 (or_lut_build, or_lut_score) and of the product's record encoder.

The closed-form identity of throughput/s2lut.py:1-4 (paper/main.tex:250),
    <q_t, level(code)> = Delta_b * (sum_p 2^(b-1-p) <q_t, beta_p> - mid_b * sum(q_t)),
is checked by comparing the LUT score with the direct codeword sum in float64 over hand-packed records
(planes MSB first, src/tiered.py:11-12; nibble bit i of v is (v >> (3-i)) & 1, throughput/s2lut.py:36).
Planted mistakes (LSB-first planes, reversed nibble bits) show that the comparison fails on them.
"""
import numpy as np
import pytest
import torch

from tests.conftest import fp16_bits

TS = [(0, 32, 3), (32, 96, 2), (96, 128, 1)]
DELTAS = {1: 1.596, 2: 0.9957, 3: 0.5860}


def _layout(TS):
    from fanarvse_paper_amd import s2lut

    return s2lut.record_layout(TS)


def _pack(codes, TS, msb_first=True):
    """Records [N, RB] of per-coordinate codes [N, D] (tier by tier, plane by plane, 8 coords per byte)."""
    toff, soff, RB = _layout(TS)
    N = codes.shape[0]
    rec = np.zeros((N, RB), np.uint8)
    for t, (s, e, b) in enumerate(TS):
        kb = (e - s) // 8
        for p in range(b):
            bit = (codes[:, s:e] >> ((b - 1 - p) if msb_first else p)) & 1
            byte = np.zeros((N, kb), np.uint32)
            for j in range(8):
                byte |= bit[:, j::8].astype(np.uint32) << (7 - j)
            rec[:, toff[t] + p * kb: toff[t] + (p + 1) * kb] = byte.astype(np.uint8)
    return rec, soff


def _direct(Zq, codes, scale, qc):
    """qc + sum_t scale_t * <Zq_t, Delta_b (code - mid_b)> in float64."""
    out = np.zeros(codes.shape[:2]) + np.asarray(qc, np.float64)
    for t, (s, e, b) in enumerate(TS):
        lv = DELTAS[b] * (codes[:, :, s:e].astype(np.float64) - (2 ** b - 1) / 2)
        out += scale[:, :, t] * np.einsum("qkd,qd->qk", lv, Zq[:, s:e].astype(np.float64))
    return out


@pytest.fixture(scope="module")
def case():
    rng = np.random.default_rng(11)
    B, N, K, D = 5, 300, 24, 128
    Zq = rng.standard_normal((B, D)).astype(np.float16)
    codes = np.concatenate([rng.integers(0, 2 ** b, size=(N, e - s)) for s, e, b in TS], 1).astype(np.int64)
    ss = np.stack([rng.uniform(0.5, 1.5, (N, len(TS))), rng.uniform(0.0, 0.1, (N, len(TS)))], 2).astype(np.float16)
    pos = np.stack([rng.choice(N, K, replace=False) for _ in range(B)]).astype(np.int32)
    qc = rng.standard_normal(B).astype(np.float32)
    return dict(Zq=Zq, codes=codes, ss=ss, pos=pos, qc=qc, B=B, K=K, D=D)


def _records(case, msb_first=True):
    rec, soff = _pack(case["codes"], TS, msb_first)
    rec[:, soff:soff + 4 * len(TS)] = case["ss"].reshape(len(rec), -1).view(np.uint8)
    return rec, soff


def _score(oracle_mod, case, L, half, rec, soff, ncnt=None):
    _, qsum, qn2 = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, half)
    deltas = np.array([DELTAS[b] for _, _, b in TS], np.float32)
    toff = np.array(_layout(TS)[0], np.int32)
    return oracle_mod.lut_score(case["pos"], case["qc"], L, half, qsum, qn2, rec, soff, TS, deltas, toff, ncnt)


def test_lut_entries_and_tier_sums(oracle_mod, case):
    Zq = case["Zq"]
    L, qsum, qn2 = oracle_mod.lut_build(fp16_bits(Zq), TS, False)
    z = Zq.astype(np.float64).reshape(case["B"], -1, 4)
    bits = np.array([[(v >> (3 - i)) & 1 for i in range(4)] for v in range(16)], np.float64)  # [16, 4]
    want = np.einsum("qni,vi->qnv", z, bits).reshape(case["B"], -1)
    assert np.allclose(L, want, rtol=1e-6, atol=1e-6)
    L16, _, _ = oracle_mod.lut_build(fp16_bits(Zq), TS, True)
    assert np.array_equal(L16, fp16_bits(L))  # the fp16 table is the rounded f32 table
    for t, (s, e, _) in enumerate(TS):
        zt = Zq[:, s:e].astype(np.float64)
        assert np.allclose(qsum[t], zt.sum(1), rtol=1e-6, atol=1e-6)
        assert np.allclose(qn2[t], (zt * zt).sum(1), rtol=1e-6)
    # planted mistake: LSB-first nibble bits give a different table
    wrong = np.einsum("qni,vi->qnv", z, bits[:, ::-1]).reshape(case["B"], -1)
    assert not np.allclose(L, wrong, rtol=1e-3)


def test_lut_score_matches_direct_codeword_sum(oracle_mod, case):
    rec, soff = _records(case)
    L, qsum, qn2 = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, False)
    est, sd = _score(oracle_mod, case, L, False, rec, soff)
    codes = case["codes"][case["pos"]]                               # [B, K, D]
    ss = case["ss"].astype(np.float64)[case["pos"]]                   # [B, K, T, 2]
    want = _direct(case["Zq"], codes, ss[..., 0], case["qc"][:, None])
    mag = 1 + np.abs(want)
    assert np.all(np.abs(est - want) <= 2e-5 * mag), np.abs(est - want).max()
    sd_want = np.sqrt(np.einsum("tq,qkt->qk", qn2.astype(np.float64), ss[..., 1] ** 2))
    assert np.allclose(sd, sd_want, rtol=1e-5, atol=1e-7)
    # the fp16 table only adds the fp16 rounding of each entry
    L16, _, _ = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, True)
    est16, _ = _score(oracle_mod, case, L16, True, rec, soff)
    assert np.all(np.abs(est16 - want) <= 5e-3 * mag)


def test_lut_score_planted_plane_and_nibble_mistakes(oracle_mod, case):
    codes = case["codes"][case["pos"]]
    ss = case["ss"].astype(np.float64)[case["pos"]]
    want = _direct(case["Zq"], codes, ss[..., 0], case["qc"][:, None])
    L, _, _ = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, False)
    rec_lsb, soff = _records(case, msb_first=False)
    est, _ = _score(oracle_mod, case, L, False, rec_lsb, soff)
    assert np.abs(est - want).max() > 0.1, "LSB-first planes must not pass the identity"
    rec, soff = _records(case)
    z = case["Zq"].astype(np.float32).reshape(case["B"], -1, 4)
    bits_rev = np.array([[(v >> i) & 1 for i in range(4)] for v in range(16)], np.float32)
    L_rev = np.einsum("qni,vi->qnv", z, bits_rev).reshape(case["B"], -1).astype(np.float32)
    est, _ = _score(oracle_mod, case, L_rev, False, rec, soff)
    assert np.abs(est - want).max() > 0.1, "reversed nibble bits must not pass the identity"


def test_lut_score_delta_rule_slots(oracle_mod, case):
    rec, soff = _records(case)
    L, _, _ = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, False)
    ncnt = np.array([0, 1, 7, case["K"], 3], np.int32)
    est, sd = _score(oracle_mod, case, L, False, rec, soff, ncnt)
    full, fsd = _score(oracle_mod, case, L, False, rec, soff)
    for q, n in enumerate(ncnt):
        assert np.array_equal(est[q, :n], full[q, :n]) and np.array_equal(sd[q, :n], fsd[q, :n])
        assert np.all(est[q, n:] == np.float32(-1e30)) and np.all(sd[q, n:] == 0)


def test_encoder_records_decode_to_the_uniform_code():
    """The product's packer (s2lut.encode_uniform, CPU tensors) writes exactly the bucketized codes, MSB
    plane first, and the reference's scale/sigma formulas (src/tiered.py:161-166)."""
    from fanarvse_paper_amd import datagen, s2lut

    X = datagen.gen(512, 128, 8, 0.7, seed=4)
    c = X.float().mean(0)
    lam, V = s2lut.pca_basis(X, c, n=512)
    order = torch.arange(512, dtype=torch.int32)
    code = s2lut.encode_uniform_tiers(X, order, c, V, TS)
    rec = code["rec"].numpy()
    toff, soff = code["toff"], code["soff"]
    Zc = ((X.float() - c) @ V).numpy().astype(np.float64)
    for t, ((s, e, b), P) in enumerate(zip(TS, code["rots"])):
        F = Zc[:, s:e] @ P.numpy().astype(np.float64)
        Fu = F / np.linalg.norm(F, axis=1, keepdims=True) * np.sqrt(e - s)
        delta = code["deltas"][b]
        th = (np.arange(1, 2 ** b) - 2 ** (b - 1)) * delta        # midpoints of the uniform levels
        q = np.searchsorted(th, Fu, side="left")
        kb = (e - s) // 8
        got = np.zeros_like(q)
        for p in range(b):
            plane = np.unpackbits(rec[:, toff[t] + p * kb: toff[t] + (p + 1) * kb], axis=1, bitorder="big")
            got |= plane.astype(np.int64) << (b - 1 - p)
        agree = (got == q).mean()
        assert agree > 0.999, (t, agree)  # float32 vs float64 rounding at bucket edges only
        sc = rec[:, soff + 4 * t: soff + 4 * t + 4].copy().view(np.float16).astype(np.float64)
        Y = (got - (2 ** b - 1) / 2) * delta
        ct = (Fu * Y).sum(1) / (np.linalg.norm(Y, axis=1) * np.sqrt(e - s))
        nf = np.linalg.norm(F, axis=1)
        assert np.allclose(sc[:, 0], nf / (ct * np.linalg.norm(Y, axis=1)), rtol=2e-3)
        assert np.allclose(sc[:, 1], nf * np.sqrt(np.clip(1 - ct ** 2, 0, None)) / (ct * np.sqrt(e - s - 1)),
                           rtol=5e-3, atol=1e-4)


def test_partial_estimate_over_leading_tiers(oracle_mod, case):
    """score_lut(..., nt) (throughput/s2lut.py:92-93) scores TS[:nt] with the full tables: the oracle's
    estimate over the first two tiers equals the direct codeword sum over those tiers; the all-tiers
    estimate (the planted mistake) does not."""
    rec, soff = _records(case)
    L, qsum, qn2 = oracle_mod.lut_build(fp16_bits(case["Zq"]), TS, False)
    deltas = np.array([DELTAS[b] for _, _, b in TS], np.float32)
    toff = np.array(_layout(TS)[0], np.int32)
    nt = 2
    est, sd = oracle_mod.lut_score(case["pos"], case["qc"], L, False, qsum[:nt], qn2[:nt], rec, soff, TS[:nt],
                                   deltas[:nt], toff[:nt])
    codes = case["codes"][case["pos"]]
    ss = case["ss"].astype(np.float64)[case["pos"]]
    want = np.zeros(codes.shape[:2]) + case["qc"][:, None].astype(np.float64)
    for t, (s, e, b) in enumerate(TS[:nt]):
        lv = DELTAS[b] * (codes[:, :, s:e].astype(np.float64) - (2 ** b - 1) / 2)
        want += ss[..., t, 0] * np.einsum("qkd,qd->qk", lv, case["Zq"][:, s:e].astype(np.float64))
    mag = 1 + np.abs(want)
    assert np.all(np.abs(est - want) <= 2e-5 * mag), np.abs(est - want).max()
    sd_want = np.sqrt(np.einsum("tq,qkt->qk", qn2[:nt].astype(np.float64), ss[..., :nt, 1] ** 2))
    assert np.allclose(sd, sd_want, rtol=1e-5, atol=1e-7)
    full, _ = _score(oracle_mod, case, L, False, rec, soff)
    assert np.abs(full - want).max() > 0.1, "the all-tiers estimate must not pass as the partial one"


def _decode_tiers(rec, pos, TS, toff, soff, deltas, Zq, qc, nt):
    """float64 direct estimate over the first nt tiers of the candidates pos [B, K], decoded from the records
    (planes MSB first, src/tiered.py:11-12; levels Delta_b (code - mid_b), throughput/s2lut.py:9-16)."""
    R = rec[pos]                                                     # [B, K, RB]
    est = np.zeros(pos.shape) + np.asarray(qc, np.float64)[:, None]
    for t, (s, e, b) in enumerate(TS[:nt]):
        kb = (e - s) // 8
        code = np.zeros(pos.shape + (e - s,), np.int64)
        for p in range(b):
            plane = np.unpackbits(R[:, :, toff[t] + p * kb: toff[t] + (p + 1) * kb], axis=2, bitorder="big")
            code |= plane.astype(np.int64) << (b - 1 - p)
        lv = float(deltas[t]) * (code - (2 ** b - 1) / 2)
        sc = R[:, :, soff + 4 * t: soff + 4 * t + 2].copy().view(np.float16)[..., 0].astype(np.float64)
        est += sc * np.einsum("qkd,qd->qk", lv, Zq[:, s:e])
    return est


def test_progressive_stage_ranks_by_leading_tiers(oracle_mod, tiny):
    """K2 < K (throughput/enginei8.py:82-85): the K2 candidates kept are the best of the K by the estimate over
    the first NT tiers. Checked against a float64 direct codeword sum of those tiers (every candidate clearly
    above the K2-th value is kept, every one clearly below is dropped); the planted all-tiers ranking fails
    the same check."""
    idx = tiny["idx"]
    TS = idx["TS"]
    assert len(TS) == 3
    K, K2, NT = 120, 40, 2
    knobs = dict(K2=K2, NT=NT, LUTF=True, LUTH=False)
    out = oracle_mod.pipeline(idx, tiny["Qn"], K, 1.25, 16, 10, knobs=knobs, fallback=False)
    pos1, pos2 = out["pos"], out["pos2"]
    assert pos2.shape == (len(pos1), K2)
    Zq = np.asarray(out["Zq"]).view(np.float16).astype(np.float64)
    args = (idx["rec"], pos1, TS, idx["toff"], idx["soff"], idx["deltas"], Zq, out["qc"])

    def consistent(keep, v):
        ok = []
        for q in range(len(v)):
            th = np.sort(v[q])[::-1][K2 - 1]
            eps = 1e-4 * (1 + abs(th))
            kept = np.isin(pos1[q], keep[q])
            ok.append(kept[v[q] > th + eps].all() and not kept[v[q] < th - eps].any())
        return np.array(ok)

    part = _decode_tiers(*args, NT)
    assert consistent(pos2, part).all()
    allt = _decode_tiers(*args, len(TS))
    wrong = np.take_along_axis(pos1, np.argsort(-allt, axis=1, kind="stable")[:, :K2], 1)
    assert not consistent(wrong, part).all(), "ranking by all tiers must not pass"
