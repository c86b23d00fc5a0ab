"""Drop-in for the reference's `civf8` module (throughput/civf8.py): the int8 stage-1 scan behind the
operator seam that EngineI8.stage1_i8 switches to when its CUDA knob is set (throughput/enginei8.py:49-52,58).

    import civf8                                   # the reference's CuPy/NVRTC twin
    from fanarvse_paper_amd import civf8           # this module: the same call on gfx950

`launch` keeps the reference's 21 arguments, their meaning and its launch on torch's current stream
(throughput/civf8.py:89-91); it runs libfvs's fvs_i8_scan_civf8. The tensors are the ones stage1_i8
already holds: q8 int8 [B, 256], qs f32 [B]; the pair lists of pairs_fast (qid, coff, ccnt int32, qcp f32);
the one-block work list of _static_blocks (pcell, pblk, ps, pe int32); Z int8 [N, 256], zs f32 [N]; and for
mode 1 t0 f32 [B], cnt int32 [B] (zeroed), bval f32 / bpos int32 [B, CAP]; for mode 0 bmc f32 [pairs, MB]
(pre-filled with -1e30). The unused arguments of a mode may be the reference's one-element dummies.
Unlike the reference, the shapes and dtypes are checked before the launch, and a failed launch raises.
"""
import torch

from . import _lib

R = 256


def launch(mode, P, q8, qs, qid, coff, ccnt, pcell, pblk, ps, pe, Z, zs, qcp, t0, cnt, bval, bpos, bmc, CAP, MB):
    if mode not in (0, 1):
        raise ValueError("civf8.launch: mode must be 0 (block maxima) or 1 (threshold emit)")
    P, CAP, MB = int(P), int(CAP), int(MB)
    if P < 0 or P > pcell.numel() or not (pcell.numel() == pblk.numel() == ps.numel() == pe.numel()):
        raise ValueError("civf8.launch: the work list must hold P items")
    if Z.dim() != 2 or Z.shape[1] != R or q8.dim() != 2 or q8.shape[1] != R:
        raise ValueError(f"civf8.launch: codes must be [*, {R}] int8")
    N, B = Z.shape[0], q8.shape[0]
    if zs.numel() != N or qs.numel() != B:
        raise ValueError("civf8.launch: one scale per code row and per query")
    npairs = qid.numel()
    if qcp.numel() != npairs or coff.numel() != ccnt.numel():
        raise ValueError("civf8.launch: pair lists of different lengths")
    f32, i32 = torch.float32, torch.int32
    if mode == 0:
        if MB <= 0 or bmc.numel() < npairs * MB:
            raise ValueError("civf8.launch: bmc must hold pairs * MB values")
    else:
        if CAP <= 0 or t0.numel() != B or cnt.numel() != B or bval.numel() != B * CAP or bpos.numel() != B * CAP:
            raise ValueError("civf8.launch: t0, cnt [B] and bval, bpos [B, CAP] expected")
    d = _lib._dev
    rc = _lib.lib().fvs_i8_scan_civf8(
        mode, P, d(q8, torch.int8, "q8"), d(qs, f32, "qs"), d(qid, i32, "qid"), d(coff, i32, "coff"),
        d(ccnt, i32, "ccnt"), d(pcell, i32, "pcell"), d(pblk, i32, "pblk"), d(ps, i32, "ps"), d(pe, i32, "pe"),
        d(Z, torch.int8, "Z"), d(zs, f32, "zs"), d(qcp, f32, "qcp"), d(t0, f32, "t0"), d(cnt, i32, "cnt"),
        d(bval, f32, "bval"), d(bpos, i32, "bpos"), d(bmc, f32, "bmc"), CAP, MB, _lib._stream())
    _lib._check(rc, "fvs_i8_scan_civf8")
