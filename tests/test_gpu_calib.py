"""The matrix-core calibration kernel (fvs_calib_mfma) computes the chains it is timed on: its per-wave
checksum equals a numpy restatement of the same sixteen v_mfma_i32_16x16x64_i8 products per round (lane l
holds row / column l & 15 and bytes 16 (l >> 4) .. + 15 of each 64-byte step; result element r of lane l is
D[4 (l >> 4) + r][l & 15]), so bench.py's achievable-rate line times real work."""
import numpy as np
import pytest
import torch

from fanarvse_paper_amd import _lib

pytestmark = pytest.mark.gpu


def expected_checksum(iters):
    lanes = np.arange(64)

    def rows_of(words):  # words [64 lanes, 4 dwords] -> operand [16 rows, 64 bytes] (int8)
        by = words.astype(np.uint32).view(np.uint8).reshape(64, 16).view(np.int8).astype(np.int64)
        op = np.zeros((16, 64), np.int64)
        for l in range(64):
            op[l & 15, 16 * (l >> 4):16 * (l >> 4) + 16] = by[l]
        return op

    A, Bm = [], []
    for s in range(4):
        a = np.stack([(lanes + s) * 0x01010101, (lanes + 1) * 0x01010101, (lanes + 2) * 0x01010101,
                      (lanes + 3) * 0x01010101], axis=1)
        b = np.stack([0x01020304 ^ (lanes + s), 0x05060708 ^ lanes, np.full(64, 0x090a0b0c), np.full(64, 0x0d0e0f10)],
                     axis=1)
        A.append(rows_of(a))
        Bm.append(rows_of(b))
    acc = 0
    for i in range(iters):
        for j in range(4):
            D = sum(A[s] @ Bm[(s + j) & 3].T for s in range(4))
            D[0::4, :] += i  # the chain's first accumulator: element 0 of every lane is i
            acc ^= int(np.int64(D[j, 0]).astype(np.int32))  # no product sum here leaves the int32 range
    return acc


def test_calibration_checksum():
    blocks, iters = 3, 5
    out = torch.zeros(4 * blocks, dtype=torch.int32, device="cuda")
    _lib.calib_mfma(out, iters)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.all(got == got[0])
    assert int(got[0]) == int(expected_checksum(iters))
