"""The C ABI without a GPU: libfvs.so loads and exports every function include/fvs.h declares, the
argument checks reject out-of-range calls before anything is launched, the Python wrappers refuse CPU
tensors (there is no CPU fallback), and no device code contains packed-fp32 instructions."""
import ctypes
import os
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fvs.h")


@pytest.fixture(scope="module")
def L():
    from fanarvse_paper_amd import _lib, build

    if not os.path.exists(_lib.LIB_PATH):
        build.build()
    return _lib.lib()


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|int64_t|const char \*)\s*\*?\s*(fvs_\w+)\s*\(", text, re.M)))


def test_every_declared_symbol_is_exported(L):
    from fanarvse_paper_amd import _lib

    names = declared()
    assert len(names) >= 13, names
    for n in names:
        assert hasattr(L, n), n
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"
    assert L.fvs_abi_version() == 2
    assert L.fvs_error_string(-1) and L.fvs_error_string(-3) and L.fvs_error_string(0)


def test_argument_checks_need_no_gpu(L):
    """Out-of-range sizes return FVS_E_* codes before any HIP call (null pointers stand in for buffers)."""
    n = None
    E_ARG, E_SHAPE, E_CAP = -1, -2, -3
    assert L.fvs_select(n, n, n, 4, 16, 0, 0, 0.0, n, n, n, n, n) == E_ARG             # K = 0
    assert L.fvs_select(n, n, n, 4, 16, 5000, 0, 0.0, n, n, n, n, n) == E_CAP          # K > 4096
    assert L.fvs_select(n, n, n, 4, 16, 8, 8, 0.0, n, n, n, n, n) == E_ARG             # kd >= K
    assert L.fvs_route_topk(n, 4, 100, 0, n, n) == E_ARG
    assert L.fvs_pack_ids(n, n, 4, 0, n, n) == E_ARG                                  # k = 0
    assert L.fvs_pack_ids(n, n, 0, 10, n, n) == 0                                     # empty batch
    assert L.fvs_dense_small(n, 9, 1536, n, 256, n, n, 4096, n, n, 1536, n, n, n, n) == E_ARG  # B > 8
    assert L.fvs_dense_small(n, 1, 1538, n, 256, n, n, 4096, n, n, 1536, n, n, n, n) == E_ARG  # d % 4
    assert L.fvs_route_topk(n, 4, 100, 101, n, n) == E_ARG                             # nprobe > NC
    assert L.fvs_i8_scan(0, 10, *[n] * 12, 100, 128, *[n] * 6, 1, 1, 1, n) == E_SHAPE  # R != 256
    assert L.fvs_i8_scan(2, 10, *[n] * 12, 100, 256, *[n] * 6, 1, 1, 1, n) == E_ARG    # bad mode
    assert L.fvs_refine(*[n] * 6, 4, 10, 64, 1.0, 10, *[n] * 5) == E_ARG               # K <= k
    assert L.fvs_refine(*[n] * 6, 4, 20, 60, 1.0, 10, *[n] * 5) == E_ARG               # d % 8
    assert L.fvs_threshold(n, n, 4, n, 16, 4, 5, 2, 3, n, n, n) == E_ARG               # n1 > npr
    assert L.fvs_threshold(n, n, 4, n, 0, 4, 2, 2, 3, n, n, n) == E_ARG                # NC = 0
    assert L.fvs_pairs_scratch_bytes(10, 7) > 0
    # zero-sized batches are valid no-ops
    assert L.fvs_select(n, n, n, 0, 16, 8, 0, 0.0, n, n, n, n, n) == 0
    assert L.fvs_i8_scan(1, 0, *[n] * 12, 100, 256, *[n] * 6, 1, 1, 1, n) == 0
    assert L.fvs_i8_scan_civf8(2, 10, *[n] * 17, 1, 1, n) == E_ARG                    # bad mode
    assert L.fvs_i8_scan_civf8(0, 10, *[n] * 17, 1, 1, n) == E_ARG                    # null buffers
    assert L.fvs_i8_scan_civf8(1, 0, *[n] * 17, 1, 1, n) == 0                         # no items
    # routing-free dense scan: (mode, Qt, qs, B, Bpad, Zt, zs, N, Npad, R, t0, cnt, bval, bpos, CAP, out, stream)
    assert L.fvs_dense_scan(2, n, n, 4, 128, n, n, 8, 256, 128, n, n, n, n, 1, n, n) == E_ARG   # bad mode
    assert L.fvs_dense_scan(0, n, n, 4, 128, n, n, 8, 256, 96, n, n, n, n, 1, n, n) == E_SHAPE  # R % 128
    assert L.fvs_dense_scan(0, n, n, 4, 64, n, n, 8, 256, 128, n, n, n, n, 1, n, n) == E_ARG    # Bpad % 128
    assert L.fvs_dense_scan(0, n, n, 4, 128, n, n, 300, 256, 128, n, n, n, n, 1, n, n) == E_ARG  # Npad < N
    assert L.fvs_dense_scan(0, n, n, 4, 128, n, n, 8, 256, 128, n, n, n, n, 1, n, n) == E_ARG   # null buffers
    assert L.fvs_dense_scan(1, n, n, 0, 128, n, n, 8, 256, 128, n, n, n, n, 1, n, n) == 0       # no queries
    assert L.fvs_dense_pack(n, 4, 40, 32, 128, n, n) == E_ARG                                    # R % 16
    assert L.fvs_dense_pack(n, 4, 256, 32, 128, n, n) == E_ARG                                   # Rp < R
    assert L.fvs_dense_pack(n, 40, 64, 32, 128, n, n) == E_ARG                                   # npad < n
    assert L.fvs_dense_threshold(n, 4, 10, 11, n, n, n) == E_ARG                                 # r > n
    assert L.fvs_dense_threshold(n, 4, 10, 0, n, n, n) == E_ARG                                  # r = 0
    assert L.fvs_quantize_i8(n, 4, 0, n, n, n, n) == E_ARG                                       # R = 0
    assert L.fvs_calib_mfma(0, 16, n, n) == E_ARG                                                # no workgroups
    assert L.fvs_calib_mfma(4, 0, n, n) == E_ARG                                                 # no rounds
    assert L.fvs_calib_mfma(4, 16, n, n) == E_ARG                                                # no output


def test_lut_score_layout_checks_need_no_gpu(L):
    """fvs_lut_score refuses a table width that is not whole 512-byte groups, and a record whose per-dword
    schedule (passed as a kernel argument) would exceed 512 dwords, before any launch: host buffers stand
    in for the device pointers, which are never touched."""
    E_ARG, E_CAP = -1, -3
    buf = (ctypes.c_uint8 * 64)()
    p = ctypes.cast(buf, ctypes.c_void_p)

    def call(LW, D, bits, RB):
        tiers = (ctypes.c_int32 * 3)(0, D, bits)
        deltas = (ctypes.c_float * 1)(1.0)
        soff = D * bits // 8
        toff = (ctypes.c_int32 * 1)(0)
        return L.fvs_lut_score(p, p, p, 1, LW, p, p, p, 10, RB, soff, 1, tiers, deltas, toff, 0, None, 1, 10, p, p, None)

    assert call(LW=1552, D=388, bits=4, RB=208) == E_ARG      # LW % 128 (tiers are whole 32-coordinate blocks)
    assert call(LW=16384, D=4096, bits=4, RB=2064) == E_CAP   # 513 dwords of planes and pair: past 512

    # the fused form takes the query width D instead of a table: D % 32, D <= 4096, the last tier ending at D
    def call_zq(D, tier_end, bits, RB):
        tiers = (ctypes.c_int32 * 3)(0, tier_end, bits)
        deltas = (ctypes.c_float * 1)(1.0)
        soff = tier_end * bits // 8
        toff = (ctypes.c_int32 * 1)(0)
        return L.fvs_lut_score_zq(p, p, p, D, 1, p, 10, RB, soff, 1, tiers, deltas, toff, 0, None, 1, 10, p, p, None)

    E_SHAPE = -2
    assert call_zq(D=388, tier_end=388, bits=4, RB=208) == E_ARG     # D % 32
    assert call_zq(D=4128, tier_end=4128, bits=1, RB=528) == E_ARG   # D > 4096
    assert call_zq(D=384, tier_end=352, bits=4, RB=192) == E_SHAPE  # the tiers end before D
    assert call_zq(D=4096, tier_end=4096, bits=4, RB=2064) == E_CAP  # the record's schedule past 512 dwords


def test_wrappers_refuse_cpu_tensors(L):
    from fanarvse_paper_amd import _lib

    QM = torch.zeros((4, 16), dtype=torch.float16)
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        _lib.route_topk(QM, 4)
    with pytest.raises((RuntimeError, ValueError, TypeError)):
        _lib.fill_u32(torch.zeros(8, dtype=torch.int32), 0)


def test_civf8_seam_checks_before_launch(L):
    """fanarvse_paper_amd.civf8.launch keeps the reference's argument list (throughput/civf8.py:89-91) and
    refuses wrong shapes and host tensors before anything is launched."""
    import inspect

    from fanarvse_paper_amd import civf8

    names = list(inspect.signature(civf8.launch).parameters)
    assert names == ["mode", "P", "q8", "qs", "qid", "coff", "ccnt", "pcell", "pblk", "ps", "pe", "Z", "zs", "qcp",
                     "t0", "cnt", "bval", "bpos", "bmc", "CAP", "MB"]
    i32 = lambda n: torch.zeros(n, dtype=torch.int32)
    f32 = lambda *s: torch.zeros(*s)
    B, N, P = 4, 64, 2
    args = dict(mode=0, P=P, q8=torch.zeros((B, 256), dtype=torch.int8), qs=f32(B), qid=i32(8), coff=i32(3),
                ccnt=i32(3), pcell=i32(P), pblk=i32(P), ps=i32(P), pe=i32(P),
                Z=torch.zeros((N, 256), dtype=torch.int8), zs=f32(N), qcp=f32(8), t0=f32(1), cnt=i32(1),
                bval=f32(1), bpos=i32(1), bmc=f32(8, 3), CAP=1, MB=3)
    with pytest.raises(ValueError):  # host tensors: no CPU fallback
        civf8.launch(**args)
    for k, v in (("Z", torch.zeros((N, 128), dtype=torch.int8)), ("bmc", f32(8, 2)), ("mode", 2), ("P", 3),
                 ("zs", f32(N - 1)), ("qcp", f32(7))):
        with pytest.raises(ValueError):
            civf8.launch(**{**args, k: v})
    with pytest.raises(ValueError):  # mode 1: emit buffers of B * CAP
        civf8.launch(**{**args, "mode": 1, "t0": f32(B), "cnt": i32(B), "bval": f32(B, 5), "bpos": i32(B * 5),
                        "CAP": 4})


def test_no_packed_fp32_in_device_code():
    """Every kernel source, compiled with the library's own flags, has no v_pk_{add,mul,fma}_f32."""
    from fanarvse_paper_amd import build

    def asm(src):
        out = f"/tmp/fvs_abi_{os.getpid()}_{os.path.basename(src)}.s"
        cmd = [build.HIPCC, *[f for f in build.FLAGS if f != "-fPIC"], "--cuda-device-only", "-S", src, "-o", out]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr
        text = open(out).read()
        os.remove(out)
        return src, text

    with ThreadPoolExecutor(8) as ex:
        for src, text in ex.map(asm, build.sources()):
            bad = re.findall(r"v_pk_(?:add|mul|fma)_f32", text)
            assert not bad, f"{os.path.basename(src)}: {len(bad)} packed-fp32 instructions"
            assert "v_mfma" in text or "fvs_scan" not in src
