"""The routing-free dense int8 scan (throughput/brute.py:41-63) on the GPU against the oracle, bit for bit:
the row quantizer, the fragment-tiled layout, the dense scores (mode 0) and the threshold-and-emit pass
(mode 1) at several widths R (zero-padded to a multiple of 128), batch sizes and row counts that are not
multiples of the tiles, the sample threshold, and Brute.search end to end. At the literal config-2 width
R = 1536 with a full 2000-query batch, the two modes are checked against each other (every emitted pair is
a mode-0 score at or above t0, and cnt is the number of such scores) and the oracle on a subset."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib, brute

pytestmark = pytest.mark.gpu
dev = "cuda"


def npy(t):
    return t.detach().cpu().numpy()


def codes(B, N, R, seed):
    g = torch.Generator().manual_seed(seed)
    zq = torch.randn(B, R, generator=g)
    zx = torch.randn(N, R, generator=g) * (1 + torch.rand(N, 1, generator=g))
    q, qs = _lib.quantize_i8(zq.to(dev))
    Z, zs = _lib.quantize_i8(zx.to(dev), half=True)
    return q, qs, Z, zs


def packed(q, qs, Z, zs, t0=None):
    B, R = q.shape
    N = len(Z)
    Rp = _lib.round_up(R, 128)
    Bpad, Npad = _lib.round_up(B, 128), _lib.round_up(N, 256)
    Qt, Zt = _lib.dense_pack(q, Bpad, Rp), _lib.dense_pack(Z, Npad, Rp)
    qsp = torch.zeros(Bpad, device=dev)
    qsp[:B] = qs
    zsp = torch.zeros(Npad, dtype=torch.float16, device=dev)
    zsp[:N] = zs
    t0p = None
    if t0 is not None:
        t0p = torch.full((Bpad,), 1e30, device=dev)
        t0p[:B] = t0
    return Qt, qsp, Zt, zsp, t0p, Rp


def test_quantize_matches_oracle(oracle_mod):
    print("\n[gpu dense] quantize n=3001 R=200", flush=True)
    g = torch.Generator().manual_seed(3)
    z = torch.randn(3001, 200, generator=g) * torch.rand(3001, 1, generator=g) * 5
    z[7] = 0
    q, a = _lib.quantize_i8(z.to(dev))
    q16, a16 = _lib.quantize_i8(z.to(dev), half=True)
    qo, ao = oracle_mod.quantize_rows(z.numpy())
    assert np.array_equal(npy(q), qo) and np.array_equal(npy(q16), qo)
    assert np.array_equal(npy(a).view(np.uint32), ao.view(np.uint32))
    assert np.array_equal(npy(a16).view(np.uint16), ao.astype(np.float16).view(np.uint16))


def test_pack_layout():
    print("\n[gpu dense] pack n=70 R=80 -> npad=96 Rp=128", flush=True)
    X = torch.randint(-127, 128, (70, 80), dtype=torch.int8, device=dev)
    T = npy(_lib.dense_pack(X, 96, 128)).reshape(3, 4, 2, 32, 16)  # (rb, s, h, li, byte)
    Xp = np.zeros((96, 128), np.int8)
    Xp[:70, :80] = npy(X)
    ref = Xp.reshape(3, 32, 4, 2, 16).transpose(0, 2, 3, 1, 4)  # (rb, li, s, h, byte) -> (rb, s, h, li, byte)
    assert np.array_equal(T, ref)


@pytest.mark.parametrize("B,N,R", [(1, 1, 128), (5, 1000, 64), (130, 3000, 256), (300, 4100, 1536), (128, 512, 384)])
def test_scores_match_oracle(B, N, R, oracle_mod):
    print(f"\n[gpu dense] mode 0 B={B} N={N} R={R}", flush=True)
    q, qs, Z, zs = codes(B, N, R, seed=B + N + R)
    Qt, qsp, Zt, zsp, _, Rp = packed(q, qs, Z, zs)
    out = torch.empty(B, N, device=dev)
    _lib.dense_scan(0, Qt, qsp, B, Zt, zsp, N, Rp, out=out)
    ref = oracle_mod.dense_scores(npy(q), npy(qs), npy(Z), npy(zs))
    assert np.array_equal(npy(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("B,N,R,keep", [(7, 2000, 128, 30), (200, 5000, 1536, 40), (129, 777, 256, 777)])
def test_emit_matches_oracle(B, N, R, keep, oracle_mod):
    """cnt exact; the emitted (est, position) set equals the oracle's when cnt <= CAP. keep = N: every row
    passes (t0 = the smallest score)."""
    print(f"\n[gpu dense] mode 1 B={B} N={N} R={R} keep={keep}", flush=True)
    q, qs, Z, zs = codes(B, N, R, seed=7 * B + N)
    S = oracle_mod.dense_scores(npy(q), npy(qs), npy(Z), npy(zs))
    t0 = np.sort(S, 1)[:, N - keep].copy()
    t0[1] = 1e30                    # a query with nothing above its threshold
    Qt, qsp, Zt, zsp, t0p, Rp = packed(q, qs, Z, zs, torch.from_numpy(t0).to(dev))
    CAP = keep + 8
    cnt = torch.zeros(B, dtype=torch.int32, device=dev)
    bval = torch.full((B, CAP), -1e30, device=dev)
    bpos = torch.zeros((B, CAP), dtype=torch.int32, device=dev)
    _lib.dense_scan(1, Qt, qsp, B, Zt, zsp, N, Rp, t0=t0p, cnt=cnt, bval=bval, bpos=bpos, CAP=CAP)
    cnto, bvo, bpo = oracle_mod.dense_emit(npy(q), npy(qs), npy(Z), npy(zs), t0, CAP)
    assert np.array_equal(npy(cnt), cnto)
    bv, bp = npy(bval), npy(bpos)
    for i in range(B):
        c = cnto[i]
        assert c <= CAP
        got = sorted(zip(bp[i, :c].tolist(), bv[i, :c].view(np.uint32).tolist()))
        exp = sorted(zip(bpo[i, :c].tolist(), bvo[i, :c].view(np.uint32).tolist()))
        assert got == exp, i


def test_emit_overflow_keeps_cap_valid_pairs(oracle_mod):
    """cnt > CAP: cnt is still the full count, and the CAP stored pairs are distinct rows that pass, with
    their exact scores."""
    print("\n[gpu dense] mode 1 overflow B=64 N=3000 R=128", flush=True)
    B, N, R, CAP = 64, 3000, 128, 50
    q, qs, Z, zs = codes(B, N, R, seed=11)
    S = oracle_mod.dense_scores(npy(q), npy(qs), npy(Z), npy(zs))
    t0 = np.sort(S, 1)[:, N - 400].copy()
    Qt, qsp, Zt, zsp, t0p, Rp = packed(q, qs, Z, zs, torch.from_numpy(t0).to(dev))
    cnt = torch.zeros(B, dtype=torch.int32, device=dev)
    bval = torch.empty((B, CAP), device=dev)
    bpos = torch.empty((B, CAP), dtype=torch.int32, device=dev)
    _lib.dense_scan(1, Qt, qsp, B, Zt, zsp, N, Rp, t0=t0p, cnt=cnt, bval=bval, bpos=bpos, CAP=CAP)
    assert np.array_equal(npy(cnt), (S >= t0[:, None]).sum(1))
    bv, bp = npy(bval), npy(bpos)
    for i in range(B):
        assert len(set(bp[i].tolist())) == CAP
        assert np.array_equal(bv[i], S[i, bp[i]]) and np.all(bv[i] >= t0[i])


@pytest.mark.parametrize("B,n", [(300, 5000), (40, 65536), (20, 70000)])
def test_threshold_matches_oracle(B, n, oracle_mod):
    """Rows of up to 64 K values take the register-resident selection, longer ones the streaming one."""
    print(f"\n[gpu dense] threshold B={B} n={n}", flush=True)
    S = torch.randn(B, n, generator=torch.Generator().manual_seed(5))
    S[3, :100] = S[3, 100]          # ties
    S[4] = 0.25                     # a constant row
    S[5, ::2] = -S[5, 1::2]         # +-x pairs, -0 and +0 included below
    S[6, :10] = -0.0
    S[6, 10:20] = 0.0
    cnt = torch.full((B,), 9, dtype=torch.int32, device=dev)
    for r in (1, 40, n):
        t0 = _lib.dense_threshold(S.to(dev), r, cnt)
        assert np.array_equal(npy(t0), oracle_mod.row_kth(S.numpy(), r))
        assert not cnt.any()


@pytest.mark.parametrize("R,K,over", [(128, 40, 2.0), (192, 100, 3.0)])
def test_brute_search_matches_oracle(R, K, over, oracle_mod):
    """Brute (throughput/brute.py:41-63) end to end: codes, sample threshold, emit and top K."""
    print(f"\n[gpu dense] Brute.search N=20000 d=192 R={R} K={K}", flush=True)
    g = torch.Generator().manual_seed(R)
    d, N, B = 192, 20000, 150
    C = torch.randn(40, d, generator=g)
    X16 = (C[torch.randint(0, 40, (N,), generator=g)] + 0.6 * torch.randn(N, d, generator=g)).half()
    mu = X16[:5000].float().mean(0).to(dev)
    V = torch.linalg.qr(torch.randn(d, d, generator=g))[0].to(dev)
    Qb = (C[torch.randint(0, 40, (B,), generator=g)] + 0.6 * torch.randn(B, d, generator=g)).to(dev)
    b = brute.Brute(X16, mu, V, R=R, chunk=7000)
    pos, est, ok, cnt = b.search(Qb, K, over=over, M=2000)
    q, qs = b.qcode(Qb)
    po, eo, oko, cnto = oracle_mod.brute_search(npy(q), npy(qs), npy(b.Z), npy(b.zs), K, over=over, M=2000)
    assert np.array_equal(npy(cnt), cnto) and np.array_equal(npy(ok), oko)
    assert oko.mean() > 0.5
    assert np.array_equal(npy(pos), po) and np.array_equal(npy(est).view(np.uint32), eo.view(np.uint32))
    # the stored codes: the quantizer over the same projection, chunk by chunk
    z = (X16[:7000].to(dev).float() - mu) @ V[:, :R].contiguous()
    Zo, zso = oracle_mod.quantize_rows(npy(z))
    assert np.array_equal(npy(b.Z[:7000]), Zo) and np.array_equal(npy(b.zs[:7000]), zso.astype(np.float16))
    # the dense scores method against the oracle
    S = b.scores(q[:10], qs[:10])
    assert np.array_equal(npy(S), oracle_mod.dense_scores(npy(q[:10]), npy(qs[:10]), npy(b.Z), npy(b.zs)))


def test_full_batch_at_config2_width(oracle_mod):
    """2000 queries x 60,000 rows x R = 1536: emit against the GPU's own dense scores (every emitted pair has
    its mode-0 score, cnt = #{score >= t0}) and both modes against the oracle on 24 queries."""
    print("\n[gpu dense] B=2000 N=60000 R=1536", flush=True)
    B, N, R = 2000, 60000, 1536
    q, qs, Z, zs = codes(B, N, R, seed=2000)
    Qt, qsp, Zt, zsp, _, Rp = packed(q, qs, Z, zs)
    S = torch.empty(B, N, device=dev)
    _lib.dense_scan(0, Qt, qsp, B, Zt, zsp, N, Rp, out=S)
    cnt = torch.empty(B, dtype=torch.int32, device=dev)
    t0 = _lib.dense_threshold(S[:, ::20].contiguous(), 6, cnt)   # the reference's sample rule, about 120 pass
    t0p = torch.full((_lib.round_up(B, 128),), 1e30, device=dev)
    t0p[:B] = t0
    M = 4096
    bval = torch.empty(B, M, device=dev)
    bpos = torch.empty(B, M, dtype=torch.int32, device=dev)
    _lib.dense_scan(1, Qt, qsp, B, Zt, zsp, N, Rp, t0=t0p, cnt=cnt, bval=bval, bpos=bpos, CAP=M)
    assert torch.equal(cnt, (S >= t0[:, None]).sum(1).int())
    c = cnt.clamp(max=M).long()
    valid = torch.arange(M, device=dev)[None, :] < c[:, None]
    assert int(cnt.max()) <= M
    assert torch.equal(torch.gather(S, 1, bpos.long().clamp(min=0) * valid)[valid], bval[valid])
    sel = np.r_[0:8, 997:1005, 1992:2000]
    So = oracle_mod.dense_scores(npy(q[sel]), npy(qs[sel]), npy(Z), npy(zs))
    assert np.array_equal(npy(S[sel]).view(np.uint32), So.view(np.uint32))
