"""GPU routing (top-n_p cells per query) against the CPU oracle on adversarial fp16 score rows: heavy
ties at the n_p-th value (taken lowest cells first), +-0 (equal), +-inf, and every shape class of the
launcher: the wave-per-query kernel for each (cells per lane, sorted keys per lane) instantiation and
the block-per-query kernel for rows it does not take (NC not a multiple of 8, NC > 8192, n_p > 2048).
Routing on fp32 keys (QM * scale, or (QM + qadd) * scale: the trellis engines) is checked the same way
over its three kernels: 1024 threads per query (small batches), one wave per query, and the block
kernel for the rows neither takes. Results are bit-exact: the probe lists are
sorted by (score desc, cell asc)."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib

pytestmark = pytest.mark.gpu

SHAPES = [(64, 1), (64, 12), (64, 64), (520, 65), (1024, 128), (4096, 256), (4096, 300), (4096, 512),
          (4096, 768), (4096, 1024), (4096, 1025), (4096, 2048), (8192, 1), (8192, 768), (8192, 1536),
          (8192, 2048), (100, 37), (16384, 768), (4096, 4096)]


def rows(B, NC, seed):
    rng = np.random.default_rng(seed)
    levels = np.array([-np.inf, -2.0, -0.0, 0.0, 0.5, 1.0, 1.5, 3.0, np.inf], np.float16)
    few = levels[rng.integers(0, len(levels), (B // 2, NC))]              # ties everywhere
    many = rng.standard_normal((B - B // 2, NC)).astype(np.float16)      # fp16 rounding ties only
    return np.concatenate([few, many]).view(np.uint16)


@pytest.mark.parametrize("NC,npr", SHAPES)
def test_route_topk_matches_oracle(oracle_mod, NC, npr):
    print(f"\n[gpu route] NC={NC} nprobe={npr}", flush=True)
    QM = rows(8, NC, NC * 7 + npr)
    got = _lib.route_topk(torch.from_numpy(QM.view(np.float16)).cuda(), npr)
    torch.cuda.synchronize()
    want = oracle_mod.route_topk(QM, npr)
    assert np.array_equal(got.cpu().numpy(), want)


def test_route_topk_many_queries(oracle_mod):
    """A batch that is not a multiple of the 4 queries per block, at the headline shape."""
    QM = rows(1001, 4096, 5)
    got = _lib.route_topk(torch.from_numpy(QM.view(np.float16)).cuda(), 768)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle_mod.route_topk(QM, 768))


SCALED = [(64, 1), (64, 12), (104, 64), (520, 65), (1024, 128), (4096, 256), (4096, 384), (4096, 512),
          (4096, 1024), (4096, 1025), (8192, 1), (8192, 768), (8192, 1024), (100, 37), (4100, 300)]


@pytest.mark.parametrize("B", [9, 300])    # the block-per-query kernel (small batches), the wave kernel
@pytest.mark.parametrize("add", [False, True])
@pytest.mark.parametrize("NC,npr", SCALED)
def test_route_topk_scaled_matches_oracle(oracle_mod, NC, npr, add, B):
    print(f"\n[gpu route scaled] B={B} NC={NC} nprobe={npr} qadd={add}", flush=True)
    QM = rows(B, NC, NC * 5 + npr)
    rng = np.random.default_rng(npr)
    # repeated scales keep exact key ties; some zeros and negatives
    scale = rng.choice(np.array([0.0, 0.5, 1.0, 1.0, 2.0, -1.0, 3.0], np.float32), NC)
    qadd = rng.choice(np.array([0.0, -1.5, 2.0], np.float32), B) if add else None
    QMd = torch.from_numpy(QM.view(np.float16)).cuda()
    got = _lib.route_topk_scaled(QMd, torch.from_numpy(scale).cuda(), npr,
                                 None if qadd is None else torch.from_numpy(qadd).cuda())
    torch.cuda.synchronize()
    want = oracle_mod.route_topk_scaled(QM, scale, npr, qadd)
    assert np.array_equal(got.cpu().numpy(), want)


def test_route_topk_scaled_batches(oracle_mod):
    """Batch 1 and a batch that is not a multiple of the 4 queries per block, at the latency shape; a
    misaligned scale vector takes the block kernel."""
    for B in (1, 1001):
        QM = rows(B, 4096, B)
        scale = np.random.default_rng(B).uniform(0.5, 2.0, 4096).astype(np.float32)
        QMd = torch.from_numpy(QM.view(np.float16)).cuda()
        got = _lib.route_topk_scaled(QMd, torch.from_numpy(scale).cuda(), 384)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle_mod.route_topk_scaled(QM, scale, 384))
    buf = torch.from_numpy(np.concatenate([np.zeros(1, np.float32), scale])).cuda()  # 4-byte offset
    got = _lib.route_topk_scaled(QMd, buf[1:], 384)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle_mod.route_topk_scaled(QM, scale, 384))


@pytest.mark.parametrize("B,NC,npr,n", [(1, 64, 12, 12), (7, 64, 24, 5), (2000, 4096, 768, 768), (2001, 4096, 768, 90),
                                        (333, 5000, 300, 300), (129, 9000, 1024, 1000), (64, 16384, 64, 64),
                                        (16, 4096, 768, 768), (17, 4096, 256, 256), (16, 4097, 1536, 1200)])
def test_pairs_match_oracle(oracle_mod, B, NC, npr, n):
    """Cell-major (query, cell) pairs of the first n probe columns: counts, offsets, queries ascending
    inside a cell (the stable-sort order), probe ranks and the pair constants, bit-exact; through the
    one-workgroup builder (B <= 16, NC <= 4096) and the matrix builder."""
    print(f"\n[gpu pairs] B={B} NC={NC} npr={npr} n={n}", flush=True)
    rng = np.random.default_rng(B + NC + n)
    probe = np.stack([rng.permutation(NC)[:npr] for _ in range(B)]).astype(np.int32)
    QM = rng.standard_normal((B, NC)).astype(np.float16)
    mnorm = rng.uniform(0.5, 2.0, NC).astype(np.float32)
    qadd = rng.standard_normal(B).astype(np.float32)
    for qa in (None, qadd):
        qid, qrank, coff, ccnt, qcp = _lib.pairs(torch.from_numpy(probe).cuda(), n, NC, torch.from_numpy(QM).cuda(),
                                                 torch.from_numpy(mnorm).cuda(),
                                                 qadd=None if qa is None else torch.from_numpy(qa).cuda())
        torch.cuda.synchronize()
        oq, oc, on, oqcp, o = oracle_mod.pairs(np.ascontiguousarray(probe[:, :n]), NC, QM.view(np.uint16), mnorm, qa)
        assert np.array_equal(ccnt.cpu().numpy(), on)
        assert np.array_equal(coff.cpu().numpy(), oc)
        assert np.array_equal(qid.cpu().numpy(), oq)
        assert np.array_equal(qrank.cpu().numpy(), (o % n).astype(np.int32))
        assert np.array_equal(qcp.cpu().numpy().view(np.uint32), oqcp.view(np.uint32))


@pytest.mark.parametrize("B,NC,npr,n1", [(1, 64, 12, 3), (2001, 4096, 768, 52), (129, 9000, 1024, 1024),
                                         (16, 4096, 384, 51), (5, 4096, 1536, 100), (17, 4096, 1536, 100)])
def test_pairs2_is_two_pairs_calls(oracle_mod, B, NC, npr, n1):
    """The fused first-pass and emit lists equal the oracle's pairs of the first n1 and of all columns."""
    print(f"\n[gpu pairs2] B={B} NC={NC} npr={npr} n1={n1}", flush=True)
    rng = np.random.default_rng(3 * B + n1)
    probe = np.stack([rng.permutation(NC)[:npr] for _ in range(B)]).astype(np.int32)
    QM = rng.standard_normal((B, NC)).astype(np.float16)
    mnorm = rng.uniform(0.5, 2.0, NC).astype(np.float32)
    lists = _lib.pairs2(torch.from_numpy(probe).cuda(), n1, NC, torch.from_numpy(QM).cuda(),
                        torch.from_numpy(mnorm).cuda())
    torch.cuda.synchronize()
    for n, (qid, qrank, coff, ccnt, qcp) in zip((n1, npr), lists):
        oq, oc, on, oqcp, o = oracle_mod.pairs(np.ascontiguousarray(probe[:, :n]), NC, QM.view(np.uint16), mnorm)
        assert np.array_equal(ccnt.cpu().numpy(), on)
        assert np.array_equal(coff.cpu().numpy(), oc)
        assert np.array_equal(qid.cpu().numpy(), oq)
        assert np.array_equal(qrank.cpu().numpy(), (o % n).astype(np.int32))
        assert np.array_equal(qcp.cpu().numpy().view(np.uint32), oqcp.view(np.uint32))
