"""The row tier: full-precision vectors on an NVMe drive, read in batches for stage 3.

Same role as the reference's AsyncTier (src/nvme_async.py:13-25) over its Win32 reader
(src/native/nvme_reader.c): a tier file holds one fp16 row per sector-aligned slot, and
read_into(ids, out) fills out[i] with row ids[i], many reads in flight. The reader is libfvs_tier.so
(include/fvs_tier.h): io_uring, or a pread() thread pool where io_uring is unavailable, on a file opened
with O_DIRECT where the file system allows it.

    tier.write_tier(path, X16)                 # rows padded to a multiple of 4096 bytes
    T = tier.RowTier(path, d=X16.shape[1], qd=128)
    T.read_into(ids, out)                      # out: [len(ids), d] fp16, numpy or (pinned) CPU tensor
"""
import ctypes
import errno
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfvs_tier.so")
SECTOR = 4096
URING, THREADS = 1, 2           # backends (FVS_TIER_URING, FVS_TIER_THREADS)
FORCE_THREADS, BUFFERED = 1, 2  # open flags

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run fanarvse_paper_amd/build.py (or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        L.fvs_tier_open.restype = P
        L.fvs_tier_open.argtypes = [ctypes.c_char_p, I32, I32, I32, ctypes.POINTER(I32)]
        L.fvs_tier_backend.restype = I32
        L.fvs_tier_backend.argtypes = [P]
        L.fvs_tier_rows.restype = I64
        L.fvs_tier_rows.argtypes = [P]
        L.fvs_tier_read_rows.restype = I64
        L.fvs_tier_read_rows.argtypes = [P, P, I64, P, I32]
        L.fvs_tier_close.restype = None
        L.fvs_tier_close.argtypes = [P]
        _lib = L
    return _lib


def stride_for(d, itemsize=2):
    """Bytes per row slot: the row rounded up to whole 4096-byte sectors."""
    return -(-d * itemsize // SECTOR) * SECTOR


def write_tier(path, X16, stride=None, chunk=16384):
    """Write the rows of X16 ([N, d] fp16, torch or numpy, any device) as a tier file: row i at byte
    i * stride, zero padded. Returns the stride."""
    N, d = X16.shape
    stride = stride or stride_for(d)
    if stride % SECTOR or stride < 2 * d:
        raise ValueError(f"stride {stride} must be a multiple of {SECTOR} and hold {2 * d} bytes")
    with open(path, "wb") as f:
        for j in range(0, N, chunk):
            x = X16[j:j + chunk]
            x = x.detach().cpu().numpy() if isinstance(x, torch.Tensor) else np.asarray(x)
            buf = np.zeros((len(x), stride), np.uint8)
            buf[:, :2 * d] = np.ascontiguousarray(x, dtype=np.float16).view(np.uint8).reshape(len(x), 2 * d)
            f.write(buf.tobytes())
    return stride


class RowTier:
    """Batched row reads from a tier file (the reference's AsyncTier). backend: None (io_uring when the
    kernel allows it), "threads" (pread() pool); buffered: do not ask for O_DIRECT."""

    def __init__(self, path, d, qd=128, stride=None, backend=None, buffered=False):
        self.path, self.d, self.qd = path, d, qd
        self.stride = stride or stride_for(d)
        self.row_bytes = 2 * d
        flags = (FORCE_THREADS if backend == "threads" else 0) | (BUFFERED if buffered else 0)
        st = ctypes.c_int32(0)
        self.h = lib().fvs_tier_open(path.encode(), self.stride, qd, flags, ctypes.byref(st))
        if not self.h:
            raise OSError(-st.value, f"fvs_tier_open({path}): {os.strerror(-st.value)}")

    @property
    def backend(self):
        return {URING: "io_uring", THREADS: "threads"}[lib().fvs_tier_backend(self.h)]

    @property
    def rows(self):
        return lib().fvs_tier_rows(self.h)

    def read_into(self, ids, out):
        """Fill out[i] ([len(ids), d] fp16: numpy array or contiguous CPU tensor, pinned or not) with row
        ids[i]. Returns out."""
        if self.h is None:
            raise ValueError("RowTier is closed")
        ids = np.ascontiguousarray(ids, dtype=np.int64).reshape(-1)
        if isinstance(out, torch.Tensor):
            if out.is_cuda or not out.is_contiguous() or out.dtype != torch.float16:
                raise ValueError("out must be a contiguous fp16 CPU tensor")
            ptr, shape = out.data_ptr(), tuple(out.shape)
        else:
            if not out.flags["C_CONTIGUOUS"] or out.dtype != np.float16:
                raise ValueError("out must be a C-contiguous fp16 array")
            ptr, shape = out.ctypes.data, out.shape
        if shape != (len(ids), self.d):
            raise ValueError(f"out has shape {shape}, expected {(len(ids), self.d)}")
        r = lib().fvs_tier_read_rows(self.h, ids.ctypes.data, len(ids), ptr, self.row_bytes)
        if r == -errno.ERANGE:
            raise IndexError(f"row id outside the tier file ({self.rows} rows)")
        if r < 0:
            raise OSError(-r, f"fvs_tier_read_rows: {os.strerror(-r)}")
        return out

    def read(self, ids):
        """Rows ids as a new [len(ids), d] fp16 numpy array."""
        out = np.empty((len(ids), self.d), np.float16)
        return self.read_into(ids, out)

    def close(self):
        if self.h is not None:
            lib().fvs_tier_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
