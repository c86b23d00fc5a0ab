"""fvs_pairs_noalloc (the pair builder that allocates nothing: its scratch is a static device array of
the library) against fvs_pairs with a caller scratch buffer, through the C ABI: bit-identical pair lists
on consecutive calls that reuse the array with smaller inputs (the second call's matrices lie inside what
the first one wrote), on the one-workgroup path of small batches, and a refusal of sizes beyond the array.
"""
import ctypes

import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib

pytestmark = pytest.mark.gpu
dev = "cuda"


def case(B, NC, npr, n, seed, qadd=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    probe = torch.stack([torch.randperm(NC, generator=g)[:npr] for _ in range(B)]).to(torch.int32).to(dev)
    QM = torch.randn((B, NC), generator=g).half().to(dev)
    mnorm = torch.rand(NC, generator=g).to(dev) + 0.5
    qa = torch.randn(B, generator=g).to(dev) if qadd else None
    return probe, QM, mnorm, qa


def outputs(B, NC, n):
    return (torch.full((B * n,), -7, dtype=torch.int32, device=dev), torch.full((B * n,), -7, dtype=torch.int32, device=dev),
            torch.full((NC,), -7, dtype=torch.int32, device=dev), torch.full((NC,), -7, dtype=torch.int32, device=dev),
            torch.full((B * n,), -7.0, dtype=torch.float32, device=dev))


@pytest.mark.parametrize("order", ["large_then_small", "small_batch_path"])
def test_noalloc_pairs_equal_scratch_pairs(order):
    shapes = {"large_then_small": [(2000, 4096, 768, 768, False), (300, 1024, 64, 40, True)],
              "small_batch_path": [(16, 4096, 256, 256, False), (9, 512, 32, 20, True)]}[order]
    for i, (B, NC, npr, n, qadd) in enumerate(shapes):
        print(f"\n[no-alloc] call {i}: B={B} NC={NC} npr={npr} n={n}", flush=True)
        probe, QM, mnorm, qa = case(B, NC, npr, n, seed=10 * i + B, qadd=qadd)
        want = _lib.pairs(probe, n, NC, QM, mnorm, qadd=qa)             # (qid, qrank, coff, ccnt, qcp)
        got = _lib.pairs_noalloc(probe, n, NC, QM, mnorm, outputs(B, NC, n), qadd=qa)
        torch.cuda.synchronize()
        for w, o in zip(want, got):
            assert torch.equal(w.view(torch.int32), o.view(torch.int32))


def test_noalloc_refuses_sizes_beyond_the_array():
    L = _lib.lib()
    limit = L.fvs_pairs_scratch_bytes(2048, 4096)
    assert limit <= (32 << 20) < L.fvs_pairs_scratch_bytes(2049, 4096)
    probe, QM, mnorm, _ = case(4, 64, 8, 8, seed=1)
    out = outputs(4, 64, 8)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    # B beyond the array at NC = 4096: refused before anything is launched (the buffers are never touched)
    rc = L.fvs_pairs_noalloc(p(probe), 4096, 8, 8, 4096, p(QM), None, None, p(out[3]), p(out[2]), p(out[0]),
                             p(out[1]), p(out[4]), _lib._stream())
    assert rc == -3
    assert bool((out[0] == -7).all())
