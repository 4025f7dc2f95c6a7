"""Multiscale residual vector quantization on device tensors.

encode() is the tokenizer forward of the multiscale residual quantizer
(research/reference/vq_forward_semantics.md:59-82): per level, average-pool
the residual by strides[l], take the nearest code (lowest index on ties),
repeat it back and subtract; codes are concatenated level 0 first
(PROJECT.md:279). The reference has no implementation of this path
(ROADMAP.md:257-259); the names follow its conventions (flat buffers,
explicit dimensions, caller-visible outputs).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _check as _ck
from ._lib import NcmError, check, lib
from .context import default_context


def _ctx(t, ctx):
    ctx = ctx or default_context(t.device.index or 0)
    ctx.bind_stream()
    return ctx


def codes_per_batch(t: int, strides) -> int:
    return int(sum(t // int(s) for s in strides))


def prepare(codebooks, ctx=None):
    """Squared norms of every codeword, [levels, v] float32 (fixed fp32 order)."""
    import torch

    W = "rvq_prepare"
    a = _ck.Args(W)
    L, V, D = _ck.dims(codebooks, "codebooks", W, 3)
    pc = a.dev(codebooks, "codebooks", _ck.BF16, (L, V, D))
    csq = torch.empty((L, V), dtype=torch.float32, device=codebooks.device)
    a.done()
    ctx = _ctx(codebooks, ctx)
    check(lib().ncm_rvq_prepare(ctx.handle, pc, L, V, D, C.c_void_p(csq.data_ptr())), W)
    return csq


def encode(x, codebooks, strides, csq=None, want_recon=True, want_gap=True, force_codes=None,
           count_flagged=False, out=None, ctx=None, level_counts=False):
    """x: float32 [b, t, d]; codebooks: bfloat16 [levels, v, d]; csq float32
    [levels, v] (prepare) or None; force_codes int32 [b, sum t/s] or None.
    out: optional dict of preallocated outputs (codes int32 [b, sum t/s],
    recon float32 [b, t, d], gap float32 [b, sum t/s]).
    level_counts: also return, per level, the rows with an incomplete
    candidate chunk ("flagged") and the rows that needed any exact distance
    ("scored"), through ncm_rvq_encode_counts.
    Returns dict(codes, recon, gap, n_flagged[, flagged, scored])."""
    import torch

    W = "rvq_encode"
    a = _ck.Args(W)
    B, T, D = _ck.dims(x, "x", W, 3)
    L, V, D2 = _ck.dims(codebooks, "codebooks", W, 3)
    if D2 != D or len(strides) != L:
        raise NcmError(-2, W, "codebooks / strides do not match x")
    if any(int(s) < 1 or T % int(s) for s in strides):
        raise NcmError(-2, W, "every stride must divide t")
    dv = x.device
    px = a.dev(x, "x", _ck.F32, (B, T, D))
    pcb = a.dev(codebooks, "codebooks", _ck.BF16, (L, V, D))
    if csq is None:
        csq = prepare(codebooks, ctx)
    pcs = a.dev(csq, "csq", _ck.F32, (L, V))
    total = codes_per_batch(T, strides)
    pf = a.dev(force_codes, "force_codes", _ck.I32, (B, total), optional=True)
    out = out or {}
    codes = out.get("codes")
    if codes is None:
        codes = torch.empty((B, total), dtype=torch.int32, device=dv)
    recon = out.get("recon")
    if want_recon and recon is None:
        recon = torch.empty((B, T, D), dtype=torch.float32, device=dv)
    gap = out.get("gap")
    if want_gap and gap is None:
        gap = torch.empty((B, total), dtype=torch.float32, device=dv)
    pco = a.dev(codes, "codes", _ck.I32, (B, total))
    pr = a.dev(recon, "recon", _ck.F32, (B, T, D)) if want_recon else None
    pg = a.dev(gap, "gap", _ck.F32, (B, total)) if want_gap else None
    s = np.ascontiguousarray(strides, dtype=np.int32)
    nf = C.c_int64(-1)
    a.done()
    ctx = _ctx(x, ctx)
    if level_counts:
        fl = np.zeros(L, dtype=np.int64)
        sc = np.zeros(L, dtype=np.int64)
        check(lib().ncm_rvq_encode_counts(ctx.handle, px, B, T, D, L, C.c_void_p(s.ctypes.data),
                                          pcb, pcs, V, pco, pr, pg, pf,
                                          C.c_void_p(fl.ctypes.data), C.c_void_p(sc.ctypes.data)),
              W)
        return {"codes": codes, "recon": recon if want_recon else None,
                "gap": gap if want_gap else None, "n_flagged": int(fl.sum()),
                "flagged": fl.tolist(), "scored": sc.tolist()}
    check(lib().ncm_rvq_encode(ctx.handle, px, B, T, D, L, C.c_void_p(s.ctypes.data), pcb, pcs, V,
                               pco, pr, pg, pf, C.byref(nf) if count_flagged else None), W)
    return {"codes": codes, "recon": recon if want_recon else None,
            "gap": gap if want_gap else None,
            "n_flagged": int(nf.value) if count_flagged else None}


def decode(codes, codebooks, strides, t, ctx=None):
    """recon[b, t, :] = sum over levels of codebooks[l][code_l]; codes int32
    [b, sum t/s], codebooks bfloat16 [levels, v, d]."""
    import torch

    W = "rvq_decode"
    a = _ck.Args(W)
    B, total = _ck.dims(codes, "codes", W, 2)
    L, V, D = _ck.dims(codebooks, "codebooks", W, 3)
    if len(strides) != L or any(int(s) < 1 or t % int(s) for s in strides):
        raise NcmError(-2, W, "strides do not match codebooks / t")
    dv = codes.device
    pco = a.dev(codes, "codes", _ck.I32, (B, codes_per_batch(t, strides)))
    pcb = a.dev(codebooks, "codebooks", _ck.BF16, (L, V, D))
    recon = torch.empty((B, t, D), dtype=torch.float32, device=dv)
    s = np.ascontiguousarray(strides, dtype=np.int32)
    a.done()
    ctx = _ctx(codes, ctx)
    check(lib().ncm_rvq_decode(ctx.handle, pco, B, t, D, L, C.c_void_p(s.ctypes.data), pcb, V,
                               C.c_void_p(recon.data_ptr())), W)
    return recon
