"""Mirror of the reference's Zig `kernels` operator surface for the linear.

Host-slice functions keep the reference signatures and argument meaning
(packages/kernels/root.zig:10-12, :25-65, :96-104): flat float32 buffers, explicit
dimensions, caller-owned output. Where the reference asserts
(root.zig:107-110) these raise NcmError. They run on the GPU through the C
ABI; nothing here computes on the CPU.

`linear_bf16` / `linear_f32` are the device-resident paths: torch tensors
already in HBM, bf16 (or fp32) operands, fp32 (or bf16) output,
stream-ordered on torch's current stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _check as _ck
from ._lib import NCM_OUT_BF16, NCM_OUT_BF16_F32, NCM_OUT_F32, NcmError, check, lib
from .context import default_context

_OUT_MODES = {"f32": NCM_OUT_F32, "bf16_f32": NCM_OUT_BF16_F32, "bf16": NCM_OUT_BF16}


def _host_f32(a, name):
    if not isinstance(a, np.ndarray) or a.dtype != np.float32 or not a.flags.c_contiguous:
        raise TypeError(f"{name} must be a C-contiguous float32 numpy array")
    return a


def _p(a):
    return C.c_void_p(a.ctypes.data) if a is not None and a.size else None


def matmul(input, weights, output, token_count, input_width, output_width):
    """kernels.matmul (root.zig:25-65): fp32 output = input * weightsT on the
    GPU's fp32 MFMA (accumulation order differs from the reference's
    increasing k; both meet |y - y_f64| <= (K + 1) 2^-24 sum|x w|)."""
    for a, n in ((input, "input"), (weights, "weights"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_matmul_f32(_p(input), input.size, _p(weights), weights.size, _p(output),
                               output.size, token_count, input_width, output_width),
          "matmul")


def matmul_bf16(input, weights, output, token_count, input_width, output_width):
    """kernels.matmul_bf16 (root.zig:96-98): output = round_bf16(input * weightsT)
    with bf16 operands and fp32 accumulation, computed on the GPU."""
    for a, n in ((input, "input"), (weights, "weights"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_matmul_bf16(_p(input), input.size, _p(weights), weights.size, _p(output),
                                output.size, token_count, input_width, output_width),
          "matmul_bf16")


def matmul_bf16_bias(input, weights, bias, output, token_count, input_width, output_width):
    """kernels.matmul_bf16_bias (root.zig:102-104): the bf16 bias is added to
    the fp32 sum before the single bf16 output rounding."""
    for a, n in ((input, "input"), (weights, "weights"), (bias, "bias"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_matmul_bf16_bias(_p(input), input.size, _p(weights), weights.size,
                                     C.c_void_p(bias.ctypes.data), bias.size,
                                     _p(output), output.size, token_count, input_width,
                                     output_width),
          "matmul_bf16_bias")


def matmul_bf16_exact(input, weights, output, token_count, input_width, output_width):
    """kernels.matmul_bf16 (root.zig:96-98, :106-142) in the reference's own
    arithmetic bit for bit (pair-order fma chains, 512 / 1024 K blocks,
    operand and partial flush) on the GPU's VALU: for callers that compare
    bf16 outputs with the reference's exactly."""
    for a, n in ((input, "input"), (weights, "weights"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_matmul_bf16_exact(_p(input), input.size, _p(weights), weights.size,
                                      _p(output), output.size, token_count, input_width,
                                      output_width),
          "matmul_bf16_exact")


def matmul_bf16_bias_exact(input, weights, bias, output, token_count, input_width,
                           output_width):
    """kernels.matmul_bf16_bias (root.zig:102-104) bit for bit, as
    matmul_bf16_exact."""
    for a, n in ((input, "input"), (weights, "weights"), (bias, "bias"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_matmul_bf16_bias_exact(_p(input), input.size, _p(weights), weights.size,
                                           C.c_void_p(bias.ctypes.data), bias.size,
                                           _p(output), output.size, token_count, input_width,
                                           output_width),
          "matmul_bf16_bias_exact")


def rms_norm_bf16(input, weight, output, epsilon):
    """kernels.rms_norm_bf16 (root.zig:246-254) of one vector, on the GPU,
    bit-identical to the reference."""
    for a, n in ((input, "input"), (weight, "weight"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_rms_norm_bf16(_p(input), input.size, _p(weight), weight.size, _p(output),
                                  output.size, float(epsilon)), "rms_norm_bf16")


def silu_bf16(input, output):
    """kernels.silu_bf16 (root.zig:265-270) on the GPU."""
    for a, n in ((input, "input"), (output, "output")):
        _host_f32(a, n)
    check(lib().ncm_silu_bf16(_p(input), input.size, _p(output), output.size), "silu_bf16")


def round_bf16(value):
    """kernels.round_bf16 (root.zig:10-12) on a scalar or a float32 array,
    RNE with every NaN -> 0x7FC0, computed on the GPU."""
    scalar = np.isscalar(value) or np.ndim(value) == 0
    a = np.ascontiguousarray(np.atleast_1d(np.asarray(value, dtype=np.float32)))
    out = np.empty_like(a)
    check(lib().ncm_round_bf16(_p(a), _p(out), a.size), "round_bf16")
    return np.float32(out[0]) if scalar else out.reshape(np.shape(value))


# ------------------------------------------------------------ device path
# Every tensor argument, caller-supplied outputs included, is checked for
# dtype, exact shape and device before the call (ncmorph_amd._check): the C
# ABI cannot see allocation sizes.
def _ctx_for(t, ctx):
    ctx = ctx or default_context(t.device.index or 0)
    ctx.bind_stream()
    return ctx


def _out_dtypes(mode):
    return _ck.BF16 if mode == NCM_OUT_BF16 else _ck.F32


def _new_out(torch, mode, shape, device, bf16_dtype=None):
    """A new output: float32, or for the bf16 mode bf16_dtype (default
    torch.bfloat16)."""
    dt = (bf16_dtype or torch.bfloat16) if mode == NCM_OUT_BF16 else torch.float32
    return torch.empty(shape, dtype=dt, device=device)


def _mode(out_mode, where):
    if out_mode not in _OUT_MODES:
        raise NcmError(-7, where, f"out_mode must be one of {sorted(_OUT_MODES)}")
    return _OUT_MODES[out_mode]


def linear_bf16(x, w, bias=None, out=None, out_mode: str = "f32", ctx=None):
    """y = x @ w.T with bf16 operands (torch.bfloat16 tensors [m, k] and
    [n, k]), optional bf16 bias [n], fp32 accumulation, on torch's current
    stream; out [m, n] float32 ("f32", "bf16_f32") or 16-bit bf16 patterns
    ("bf16": int16 when allocated here; a bfloat16 out is accepted too)."""
    import torch

    W = "linear_bf16"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n, _ = _ck.dims(w, "w", W, 2)
    mode = _mode(out_mode, W)
    dv = x.device
    px = a.dev(x, "x", _ck.BF16, (m, k))
    pw = a.dev(w, "w", _ck.BF16, (n, k))
    pb = a.dev(bias, "bias", _ck.BF16, (n,), optional=True)
    if out is None:
        out = _new_out(torch, mode, (m, n), dv, torch.int16)
    po = a.dev(out, "out", _out_dtypes(mode), (m, n))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_bf16(ctx.handle, px, pw, pb, po, m, k, n, mode), W)
    return out


def linear_bf16_exact(x, w, bias=None, out=None, out_mode: str = "bf16_f32", ctx=None):
    """linear_bf16 in the reference's arithmetic bit for bit (the VALU
    pair-order fma chains of matmul_bf16_impl, root.zig:106-142): "bf16_f32"
    gives its output, "f32" its fp32 sum before the output rounding. Any k;
    not the fast path."""
    import torch

    W = "linear_bf16_exact"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n, _ = _ck.dims(w, "w", W, 2)
    mode = _mode(out_mode, W)
    dv = x.device
    px = a.dev(x, "x", _ck.BF16, (m, k))
    pw = a.dev(w, "w", _ck.BF16, (n, k))
    pb = a.dev(bias, "bias", _ck.BF16, (n,), optional=True)
    if out is None:
        out = _new_out(torch, mode, (m, n), dv, torch.int16)
    po = a.dev(out, "out", _out_dtypes(mode), (m, n))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_bf16_exact(ctx.handle, px, pw, pb, po, m, k, n, mode), W)
    return out


def linear_bf16_residual(x, w, residual, bias=None, out=None, out_mode: str = "bf16_f32",
                         ctx=None):
    """y = residual + x @ w.T (+ bias) in one pass: the projection followed by
    the decoder's residual add (src/decoder.zig:279-282). residual: float32
    [m, n]; out may be residual itself for the "f32" and "bf16_f32" modes."""
    import torch

    W = "linear_bf16_residual"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n, _ = _ck.dims(w, "w", W, 2)
    mode = _mode(out_mode, W)
    dv = x.device
    px = a.dev(x, "x", _ck.BF16, (m, k))
    pw = a.dev(w, "w", _ck.BF16, (n, k))
    pr = a.dev(residual, "residual", _ck.F32, (m, n))
    pb = a.dev(bias, "bias", _ck.BF16, (n,), optional=True)
    if out is None:
        out = _new_out(torch, mode, (m, n), dv, torch.int16)
    po = a.dev(out, "out", _out_dtypes(mode), (m, n))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_bf16_residual(ctx.handle, px, pw, pb, pr, po, m, k, n, mode), W)
    return out


def linear_bf16_swiglu(x, w, bias=None, out=None, ctx=None):
    """round(silu_bf16(gate) * up) of the gate/up projection in one pass: w
    torch.bfloat16 [2 I, k] with gate and up rows interleaved in groups of
    32 (see interleave_gate_up), bias bf16 [2 I] or None; returns
    torch.bfloat16 [m, I]."""
    import torch

    W = "linear_bf16_swiglu"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n2, _ = _ck.dims(w, "w", W, 2)
    if n2 % 64:
        raise NcmError(-2, W, "w must have a multiple of 64 rows")
    dv = x.device
    px = a.dev(x, "x", _ck.BF16, (m, k))
    pw = a.dev(w, "w", _ck.BF16, (n2, k))
    pb = a.dev(bias, "bias", _ck.BF16, (n2,), optional=True)
    if out is None:
        out = torch.empty((m, n2 // 2), dtype=torch.bfloat16, device=dv)
    po = a.dev(out, "out", _ck.BF16, (m, n2 // 2))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_bf16_swiglu(ctx.handle, px, pw, pb, po, m, k, n2), W)
    return out


def interleave_gate_up(gate, up):
    """[2 I, ...] rows in the order linear_bf16_swiglu reads: groups of 32
    gate rows followed by the matching 32 up rows (I % 32 == 0)."""
    inter = gate.shape[0]
    if inter % 32 or up.shape[0] != inter:
        raise ValueError("gate and up need the same row count, a multiple of 32")
    rest = tuple(gate.shape[1:])
    g = gate.reshape((inter // 32, 32) + rest)
    u = up.reshape((inter // 32, 32) + rest)
    try:
        import torch

        if isinstance(gate, torch.Tensor):
            return torch.stack([g, u], dim=1).reshape((2 * inter,) + rest).contiguous()
    except ImportError:
        pass
    return np.ascontiguousarray(np.stack([g, u], axis=1).reshape((2 * inter,) + rest))


def linear_bf16_rope64(x, w, rot_cols: int, seq_len: int, cosine, sine, bias=None, out=None,
                       ctx=None):
    """bf16 projection with the RoPE of its 64-wide heads in columns
    [0, rot_cols) fused (table row = row % seq_len; cosine, sine float32
    [seq_len, 64]); torch.bfloat16 out [m, n]."""
    import torch

    W = "linear_bf16_rope64"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n, _ = _ck.dims(w, "w", W, 2)
    dv = x.device
    px = a.dev(x, "x", _ck.BF16, (m, k))
    pw = a.dev(w, "w", _ck.BF16, (n, k))
    pb = a.dev(bias, "bias", _ck.BF16, (n,), optional=True)
    rot = int(rot_cols) > 0
    pc = a.dev(cosine, "cosine", _ck.F32, (seq_len, 64), optional=not rot)
    ps = a.dev(sine, "sine", _ck.F32, (seq_len, 64), optional=not rot)
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=dv)
    po = a.dev(out, "out", _ck.BF16, (m, n))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_bf16_rope64(ctx.handle, px, pw, pb, po, m, k, n, rot_cols, seq_len,
                                       pc, ps), W)
    return out


def linear_f32(x, w, out=None, ctx=None):
    """y = x @ w.T with float32 operands [m, k] and [n, k] (k % 4 == 0) on
    the fp32 MFMA, on torch's current stream."""
    import torch

    W = "linear_f32"
    a = _ck.Args(W)
    m, k = _ck.dims(x, "x", W, 2)
    n, _ = _ck.dims(w, "w", W, 2)
    dv = x.device
    px = a.dev(x, "x", _ck.F32, (m, k))
    pw = a.dev(w, "w", _ck.F32, (n, k))
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=dv)
    po = a.dev(out, "out", _ck.F32, (m, n))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_linear_f32(ctx.handle, px, pw, po, m, k, n), W)
    return out


def bf16_from_f32(src, flush: bool = False, ctx=None):
    """Device f32 -> bf16 (RNE, NaN -> 0x7FC0), returned as torch.bfloat16."""
    import torch

    W = "bf16_from_f32"
    a = _ck.Args(W)
    ps = a.dev(src, "src", _ck.F32)
    out = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
    a.done()
    ctx = _ctx_for(src, ctx)
    check(lib().ncm_bf16_from_f32_dev(ctx.handle, ps, C.c_void_p(out.data_ptr()), src.numel(),
                                      1 if flush else 0), W)
    return out


def bf16_widen(src, ctx=None):
    """Device bf16 -> f32 (exact)."""
    import torch

    W = "bf16_widen"
    a = _ck.Args(W)
    ps = a.dev(src, "src", _ck.BF16)
    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    a.done()
    ctx = _ctx_for(src, ctx)
    check(lib().ncm_bf16_widen_dev(ctx.handle, ps, C.c_void_p(out.data_ptr()), src.numel()), W)
    return out


def rms_norm_rows(x, weight, epsilon: float, out_mode: str = "bf16_f32", out=None, ctx=None):
    """RMSNorm of every row of x (float32 [rows, width]) with weight (float32
    [width]) on torch's current stream: bf16 mode with out_mode "bf16_f32"
    (float32 holding bf16 values) or "bf16" (torch.bfloat16); the f32 mode
    (rms_norm, root.zig:226-239) with out_mode "f32"."""
    import torch

    W = "rms_norm_rows"
    a = _ck.Args(W)
    rows_, width = _ck.dims(x, "x", W, 2)
    mode = _mode(out_mode, W)
    dv = x.device
    px = a.dev(x, "x", _ck.F32, (rows_, width))
    pw = a.dev(weight, "weight", _ck.F32, (width,))
    if out is None:
        out = _new_out(torch, mode, (rows_, width), dv)
    po = a.dev(out, "out", _out_dtypes(mode), (rows_, width))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_rms_norm_rows_dev(ctx.handle, px, pw, po, rows_, width, float(epsilon), mode),
          W)
    return out


def silu_mul(gate, up=None, out_mode: str = "bf16_f32", out=None, ctx=None):
    """round_bf16(silu_bf16(gate) * up) elementwise (up None: silu_bf16) on
    torch's current stream, or with out_mode "f32" the f32 mode silu(gate) *
    up (root.zig:255-261); gate, up float32 of one shape."""
    import torch

    W = "silu_mul"
    a = _ck.Args(W)
    mode = _mode(out_mode, W)
    if gate is None:
        raise NcmError(-1, W, "gate is required")
    dv = gate.device
    shape = tuple(gate.shape)
    pg = a.dev(gate, "gate", _ck.F32, shape)
    pu = a.dev(up, "up", _ck.F32, shape, optional=True)
    if out is None:
        out = _new_out(torch, mode, shape, dv)
    po = a.dev(out, "out", _out_dtypes(mode), shape)
    a.done()
    ctx = _ctx_for(gate, ctx)
    check(lib().ncm_silu_mul_dev(ctx.handle, pg, pu, po, gate.numel(), mode), W)
    return out


def rope_rotate(x, heads: int, head_dim: int, seq_len: int, cosine, sine, ctx=None):
    """In-place bf16 RoPE (rotate_head, root.zig:615-634) of every head of
    every row of x (torch.bfloat16 [rows, >= heads * head_dim], rows may be
    strided); row r uses table row r % seq_len of cosine/sine (float32
    [seq_len, head_dim])."""
    W = "rope_rotate"
    a = _ck.Args(W)
    n_rows, _ = _ck.dims(x, "x", W, 2)
    dv = x.device
    ptr, stride = a.rows(x, "x", _ck.BF16, n_rows, heads * head_dim)
    pc = a.dev(cosine, "cosine", _ck.F32, (seq_len, head_dim))
    ps = a.dev(sine, "sine", _ck.F32, (seq_len, head_dim))
    a.done()
    ctx = _ctx_for(x, ctx)
    check(lib().ncm_rope_rotate_dev(ctx.handle, ptr, n_rows, stride, heads, head_dim, seq_len,
                                    pc, ps), W)
    return x


def _attention_operands(a, q, k, v, out, batch, seq_len, q_heads, kv_heads, head_dim, mode):
    import torch

    W = a.where
    n = batch * seq_len
    dv = q.device if q is not None else None
    qp, qs = a.rows(q, "q", _ck.BF16, n, q_heads * head_dim)
    kp, ks = a.rows(k, "k", _ck.BF16, n, kv_heads * head_dim)
    vp_, vs = a.rows(v, "v", _ck.BF16, n, kv_heads * head_dim)
    if ks != vs:
        raise NcmError(-2, W, "k and v row strides differ")
    if out is None:
        out = _new_out(torch, mode, (n, q_heads * head_dim), dv)
    op, os_ = a.rows(out, "out", _out_dtypes(mode), n, q_heads * head_dim)
    return out, qp, qs, kp, ks, vp_, op, os_


def attention_bf16(q, k, v, batch: int, seq_len: int, q_heads: int, kv_heads: int,
                   head_dim: int, window: int = 0, out_mode: str = "bf16_f32", out=None,
                   ctx=None):
    """Causal bf16 attention (root.zig:536-578) of `batch` sequences: q
    [batch * seq_len, >= q_heads * head_dim], k and v [batch * seq_len,
    >= kv_heads * head_dim], torch.bfloat16 with contiguous rows (column
    slices of one q|k|v buffer are allowed)."""
    W = "attention_bf16"
    a = _ck.Args(W)
    mode = _mode(out_mode, W)
    out, qp, qs, kp, ks, vp_, op, os_ = _attention_operands(
        a, q, k, v, out, batch, seq_len, q_heads, kv_heads, head_dim, mode)
    a.done()
    ctx = _ctx_for(q, ctx)
    check(lib().ncm_attention_bf16_dev(ctx.handle, qp, kp, vp_, op, batch, seq_len, q_heads,
                                       kv_heads, head_dim, qs, ks, os_, window, mode), W)
    return out


def block_diagonal_segments(prefix_len: int, level_lengths, prefix_pad_mask=None):
    """Host: (seg_lo, seg_hi, pad_bits) numpy arrays of NCM's block-diagonal
    mask (src/ncm_mask.zig:10-42) for ncm_attention_bf16_seg_dev."""
    lv = np.ascontiguousarray(level_lengths, dtype=np.int64)
    seq = int(prefix_len + lv.sum())
    lo = np.zeros(seq, np.int32)
    hi = np.zeros(seq, np.int32)
    pad = None if prefix_pad_mask is None else np.ascontiguousarray(prefix_pad_mask, np.uint8)
    bits = np.zeros(max(1, (prefix_len + 63) // 64), np.uint64)
    check(lib().ncm_block_diagonal_segments(
        prefix_len, lv.ctypes.data_as(C.c_void_p), lv.size,
        None if pad is None else pad.ctypes.data_as(C.c_void_p), 0 if pad is None else pad.size,
        seq, lo.ctypes.data_as(C.c_void_p), hi.ctypes.data_as(C.c_void_p),
        bits.ctypes.data_as(C.c_void_p)), "block_diagonal_segments")
    return lo, hi, bits


def attention_bf16_seg(q, k, v, batch: int, seq_len: int, q_heads: int, kv_heads: int,
                       head_dim: int, prefix_len: int, seg_lo, seg_hi, pad_bits=None,
                       out_mode: str = "bf16_f32", out=None, ctx=None):
    """bf16 attention under NCM's block-diagonal level mask; seg_lo / seg_hi
    int32 [seq_len] and pad_bits uint64 [ceil(prefix_len / 64)] device
    tensors (block_diagonal_segments)."""
    W = "attention_bf16_seg"
    a = _ck.Args(W)
    mode = _mode(out_mode, W)
    out, qp, qs, kp, ks, vp_, op, os_ = _attention_operands(
        a, q, k, v, out, batch, seq_len, q_heads, kv_heads, head_dim, mode)
    dv = q.device
    pl = a.dev(seg_lo, "seg_lo", _ck.I32, (seq_len,))
    ph = a.dev(seg_hi, "seg_hi", _ck.I32, (seq_len,))
    pp = a.dev(pad_bits, "pad_bits", _ck.U64, (max(1, (prefix_len + 63) // 64),),
                 optional=True)
    a.done()
    ctx = _ctx_for(q, ctx)
    check(lib().ncm_attention_bf16_seg_dev(ctx.handle, qp, kp, vp_, op, batch, seq_len, q_heads,
                                           kv_heads, head_dim, qs, ks, os_, prefix_len, pl, ph,
                                           pp, mode), W)
    return out


def tied_head_logits(z, codebook, csq, log_inv_t: float = 0.0, bias=None, out=None, ctx=None):
    """Codebook-tied NCM code head (PROJECT.md:222): logits = (2 z E^T - csq)
    * exp(log_inv_t) / mean(csq) (+ bias). z: torch.bfloat16 [rows, d] on the
    GPU, codebook: torch.bfloat16 [v, d], csq: float32 [v] (vq.prepare), bias:
    float32 [v] or None; returns float32 [rows, v]."""
    import torch

    W = "tied_head_logits"
    a = _ck.Args(W)
    rows_, d = _ck.dims(z, "z", W, 2)
    v, _ = _ck.dims(codebook, "codebook", W, 2)
    dv = z.device
    pz = a.dev(z, "z", _ck.BF16, (rows_, d))
    pe = a.dev(codebook, "codebook", _ck.BF16, (v, d))
    pc = a.dev(csq, "csq", _ck.F32, (v,))
    pb = a.dev(bias, "bias", _ck.F32, (v,), optional=True)
    if out is None:
        out = torch.empty((rows_, v), dtype=torch.float32, device=dv)
    po = a.dev(out, "out", _ck.F32, (rows_, v))
    a.done()
    ctx = _ctx_for(z, ctx)
    check(lib().ncm_tied_head_logits(ctx.handle, pz, pe, pc, pb, float(log_inv_t), po, rows_, d,
                                     v), W)
    return out


def tied_head_logits_levels(z, codebooks, csq, level_rows, log_inv_t=None, bias=None, out=None,
                            ctx=None):
    """Every level's tied head in one launch: z torch.bfloat16 [sum rows, d]
    (level blocks in order, level_rows[l] rows each), codebooks bfloat16
    [levels, v, d], csq float32 [levels, v], log_inv_t: one float per level
    (default 0), bias float32 [levels, v] or None; float32 [sum rows, v]."""
    import torch

    W = "tied_head_logits_levels"
    a = _ck.Args(W)
    L, v, d = _ck.dims(codebooks, "codebooks", W, 3)
    rows = np.ascontiguousarray(level_rows, dtype=np.int64)
    lit = np.ascontiguousarray(np.zeros(L) if log_inv_t is None else log_inv_t, dtype=np.float32)
    if rows.size != L or lit.size != L:
        raise NcmError(-2, W, "level_rows and log_inv_t need one entry per level")
    total = int(rows.sum())
    dv = codebooks.device
    pz = a.dev(z, "z", _ck.BF16, (total, d))
    pe = a.dev(codebooks, "codebooks", _ck.BF16, (L, v, d))
    pc = a.dev(csq, "csq", _ck.F32, (L, v))
    pb = a.dev(bias, "bias", _ck.F32, (L, v), optional=True)
    if out is None:
        out = torch.empty((total, v), dtype=torch.float32, device=dv)
    po = a.dev(out, "out", _ck.F32, (total, v))
    a.done()
    ctx = _ctx_for(codebooks, ctx)
    check(lib().ncm_tied_head_logits_levels(
        ctx.handle, pz, pe, pc, pb, lit.ctypes.data_as(C.c_void_p),
        rows.ctypes.data_as(C.c_void_p), L, d, v, po), W)
    return out
