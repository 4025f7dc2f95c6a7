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

from ._lib import check, lib
from .context import default_context


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("expected a contiguous GPU tensor")
    return C.c_void_p(t.data_ptr())


def _ctx(t, ctx):
    ctx = ctx or default_context(t.device.index or 0)
    ctx.bind_stream()
    return ctx


def codes_per_batch(t: int, strides) -> int:
    return int(sum(t // int(s) for s in strides))


def prepare(codebooks, ctx=None):
    """Squared norms of every codeword, [levels, v] float32 (fixed fp32 order)."""
    import torch

    L, V, D = codebooks.shape
    csq = torch.empty((L, V), dtype=torch.float32, device=codebooks.device)
    ctx = _ctx(codebooks, ctx)
    check(lib().ncm_rvq_prepare(ctx.handle, _ptr(codebooks), L, V, D, _ptr(csq)), "rvq_prepare")
    return csq


def encode(x, codebooks, strides, csq=None, want_recon=True, want_gap=True, force_codes=None,
           count_flagged=False, out=None, ctx=None):
    """x: float32 [b, t, d]; codebooks: bfloat16 [levels, v, d].
    Returns dict(codes int32 [b, sum t/s], recon, gap, n_flagged)."""
    import torch

    B, T, D = x.shape
    L, V, D2 = codebooks.shape
    if D2 != D or len(strides) != L:
        raise ValueError("codebooks / strides do not match x")
    if csq is None:
        csq = prepare(codebooks, ctx)
    total = codes_per_batch(T, strides)
    out = out or {}
    codes = out.get("codes")
    if codes is None:
        codes = torch.empty((B, total), dtype=torch.int32, device=x.device)
    recon = out.get("recon")
    if want_recon and recon is None:
        recon = torch.empty((B, T, D), dtype=torch.float32, device=x.device)
    gap = out.get("gap")
    if want_gap and gap is None:
        gap = torch.empty((B, total), dtype=torch.float32, device=x.device)
    s = np.ascontiguousarray(strides, dtype=np.int32)
    nf = C.c_int64(-1)
    ctx = _ctx(x, ctx)
    check(lib().ncm_rvq_encode(ctx.handle, _ptr(x), B, T, D, L,
                               C.c_void_p(s.ctypes.data), _ptr(codebooks), _ptr(csq), V,
                               _ptr(codes), _ptr(recon) if want_recon else None,
                               _ptr(gap) if want_gap else None, _ptr(force_codes),
                               C.byref(nf) if count_flagged else None),
          "rvq_encode")
    return {"codes": codes, "recon": recon if want_recon else None,
            "gap": gap if want_gap else None,
            "n_flagged": int(nf.value) if count_flagged else None}


def decode(codes, codebooks, strides, t, ctx=None):
    """recon[b, t, :] = sum over levels of codebooks[l][code_l]."""
    import torch

    B = codes.shape[0]
    L, V, D = codebooks.shape
    recon = torch.empty((B, t, D), dtype=torch.float32, device=codes.device)
    s = np.ascontiguousarray(strides, dtype=np.int32)
    ctx = _ctx(codes, ctx)
    check(lib().ncm_rvq_decode(ctx.handle, _ptr(codes), B, t, D, L, C.c_void_p(s.ctypes.data),
                               _ptr(codebooks), V, _ptr(recon)), "rvq_decode")
    return recon
