"""The LUT stage-2 scorer over record layouts other than the index's, bit for bit against the CPU oracle.

The layouts give planes of 1, 2, 3, 4, 5, 7 and 16 dwords (tiers 32 to 512 coordinates wide), 1 to 8 bits
per coordinate, one to eight tiers (the most a record may hold) and records of one to four 128-byte units,
so the scorer's tier sums meet every case of their per-dword schedule: plane ends, tier ends, the dword
pairs whose entry sums are added together, the pairs that straddle a plane end, and the (scale, sigma)
dwords after the planes. Each layout runs with fp16 and fp32 tables (fvs_lut_build then fvs_lut_score)
and with the tables formed inside the scorer (fvs_lut_score_zq), over all tiers and the leading ones, with
delta-rule counts that leave some queries no candidate and others all of them. The records are random
bytes with finite (scale, sigma) pairs; K = 300 takes two rounds of the scorer's 256 lanes, and a second test
runs K = 1, 63, 257 and 1000 (one to four rounds) with a delta-rule count above K."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib, s2lut

pytestmark = pytest.mark.gpu

LAYOUTS = {
    "planes_1_2_4_1": [(0, 32, 8), (32, 96, 1), (96, 224, 3), (224, 256, 2)],
    "planes_3": [(0, 96, 5), (96, 192, 7), (192, 288, 4)],
    "one_tier_4_units": [(0, 512, 6)],
    "eight_tiers": [(32 * i, 32 * i + 32, 1 + i) for i in range(8)],
    "planes_5_1_7": [(0, 160, 2), (160, 192, 8), (192, 416, 1)],
}


def npy(t):
    return t.detach().cpu().numpy()


def make_case(TS, seed, N=4000, B=48, K=300):
    rng = np.random.default_rng(seed)
    D = TS[-1][1]
    toff, soff, RB = s2lut.record_layout(TS)
    rec = rng.integers(0, 256, size=(N, RB), dtype=np.uint8)
    T = len(TS)
    pairs = np.empty((N, 2 * T), np.float16)
    pairs[:, 0::2] = rng.uniform(0.5, 2.0, size=(N, T))   # scale
    pairs[:, 1::2] = rng.uniform(0.0, 0.1, size=(N, T))   # sigma
    rec[:, soff:soff + 4 * T] = pairs.view(np.uint8)
    deltas_by_bits = [0.0] + [2.0 / (1 << b) for b in range(1, 9)]
    Zq = rng.standard_normal((B, D)).astype(np.float16)
    pos = rng.integers(0, N, size=(B, K), dtype=np.int32)
    qc = rng.standard_normal(B).astype(np.float32)
    ncnt = rng.integers(0, K + 1, size=B).astype(np.int32)
    ncnt[0], ncnt[1] = 0, K
    return dict(TS=TS, D=D, toff=toff, soff=soff, rec=rec, deltas_by_bits=deltas_by_bits, Zq=Zq, pos=pos, qc=qc,
                ncnt=ncnt)


@pytest.mark.parametrize("name", sorted(LAYOUTS))
def test_lut_scorer_layouts_match_oracle(name, oracle_mod):
    c = make_case(LAYOUTS[name], seed=sorted(LAYOUTS).index(name))
    TS, T = c["TS"], len(c["TS"])
    print(f"layout {name}: TS {TS}, record {c['rec'].shape[1]} bytes", flush=True)
    dev = "cuda"
    code = {"TS": TS, "rec": torch.from_numpy(c["rec"]).to(dev), "soff": c["soff"], "toff": c["toff"],
            "deltas": c["deltas_by_bits"]}
    deltas = np.asarray([c["deltas_by_bits"][b] for _, _, b in TS], np.float32)
    toff = np.asarray(c["toff"], np.int32)
    Zq = torch.from_numpy(c["Zq"]).to(dev)
    pos = torch.from_numpy(c["pos"]).to(dev)
    qc = torch.from_numpy(c["qc"]).to(dev)
    for half in (True, False):
        L, qsum, qn2 = oracle_mod.lut_build(c["Zq"].view(np.uint16), TS, half)
        pre = _lib.lut_build(Zq, TS, half)
        for nt in (None, max(1, T - 1)):
            n = T if nt is None else nt
            for nc in (c["ncnt"], None):
                want_e, want_s = oracle_mod.lut_score(c["pos"], c["qc"], L, half, qsum[:n], qn2[:n], c["rec"],
                                                      c["soff"], TS[:n], deltas[:n], toff[:n], nc)
                ncd = None if nc is None else torch.from_numpy(nc).to(dev)
                for form, p in (("build-then-score", pre), ("fused", _lib.ZqTables(Zq, half))):
                    e, s = _lib.lut_score(pos, qc, p, code, ncd, nt)
                    torch.cuda.synchronize()
                    tag = (name, form, half, nt, nc is None)
                    assert np.array_equal(npy(e).view(np.uint32), want_e.view(np.uint32)), tag
                    assert np.array_equal(npy(s).view(np.uint32), want_s.view(np.uint32)), tag


@pytest.mark.parametrize("K", [1, 63, 257, 1000])
def test_lut_scorer_candidate_counts_match_oracle(K, oracle_mod):
    """Candidate counts that leave one lane, part of a wave, one lane of a second round and four rounds per
    query, with delta-rule counts above K (clamped to K) among them: fused fp16 tables as the engine runs them."""
    TS = LAYOUTS["planes_1_2_4_1"]
    c = make_case(TS, seed=100 + K, N=3000, B=24, K=K)
    c["ncnt"][2] = K + 5
    dev = "cuda"
    code = {"TS": TS, "rec": torch.from_numpy(c["rec"]).to(dev), "soff": c["soff"], "toff": c["toff"],
            "deltas": c["deltas_by_bits"]}
    deltas = np.asarray([c["deltas_by_bits"][b] for _, _, b in TS], np.float32)
    L, qsum, qn2 = oracle_mod.lut_build(c["Zq"].view(np.uint16), TS, True)
    want_e, want_s = oracle_mod.lut_score(c["pos"], c["qc"], L, True, qsum, qn2, c["rec"], c["soff"], TS, deltas,
                                          np.asarray(c["toff"], np.int32), c["ncnt"])
    e, s = _lib.lut_score(torch.from_numpy(c["pos"]).to(dev), torch.from_numpy(c["qc"]).to(dev),
                          _lib.ZqTables(torch.from_numpy(c["Zq"]).to(dev), True), code,
                          torch.from_numpy(c["ncnt"]).to(dev))
    torch.cuda.synchronize()
    assert np.array_equal(npy(e).view(np.uint32), want_e.view(np.uint32)), K
    assert np.array_equal(npy(s).view(np.uint32), want_s.view(np.uint32)), K
