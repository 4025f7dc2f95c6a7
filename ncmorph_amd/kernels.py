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
def _dev_ptr(t, name):
    if t is None:
        return None
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous GPU tensor")
    return C.c_void_p(t.data_ptr())


def linear_bf16(x, w, bias=None, out=None, out_mode: str = "f32", ctx=None):
    """y = x @ w.T with bf16 operands (torch.bfloat16 tensors [m, k] and
    [n, k]), fp32 accumulation, on torch's current stream."""
    import torch

    m, k = x.shape
    n, k2 = w.shape
    if k != k2:
        raise NcmError(-2, "linear_bf16")
    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.int16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty((m, n), dtype=dt, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_linear_bf16(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(w, "w"),
                                _dev_ptr(bias, "bias"), _dev_ptr(out, "out"), m, k, n, mode),
          "linear_bf16")
    return out


def linear_bf16_residual(x, w, residual, bias=None, out=None, out_mode: str = "bf16_f32",
                         ctx=None):
    """y = residual + x @ w.T (+ bias) in one pass: the projection followed by
    the decoder's residual add (src/decoder.zig:279-282). residual: float32
    [m, n]; out may be residual itself for the "f32" and "bf16_f32" modes."""
    import torch

    m, k = x.shape
    n, k2 = w.shape
    if k != k2 or tuple(residual.shape) != (m, n) or residual.dtype != torch.float32:
        raise NcmError(-2, "linear_bf16_residual")
    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.int16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty((m, n), dtype=dt, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_linear_bf16_residual(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(w, "w"),
                                         _dev_ptr(bias, "bias"), _dev_ptr(residual, "residual"),
                                         _dev_ptr(out, "out"), m, k, n, mode),
          "linear_bf16_residual")
    return out


def linear_bf16_swiglu(x, w, bias=None, out=None, ctx=None):
    """round(silu_bf16(gate) * up) of the gate/up projection in one pass: w
    torch.bfloat16 [2 I, k] with gate and up rows interleaved in groups of
    32 (see interleave_gate_up); returns torch.bfloat16 [m, I]."""
    import torch

    m, k = x.shape
    n2, k2 = w.shape
    if k != k2:
        raise NcmError(-2, "linear_bf16_swiglu")
    if out is None:
        out = torch.empty((m, n2 // 2), dtype=torch.bfloat16, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_linear_bf16_swiglu(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(w, "w"),
                                       _dev_ptr(bias, "bias"), _dev_ptr(out, "out"), m, k, n2),
          "linear_bf16_swiglu")
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
    [0, rot_cols) fused (table row = row % seq_len); torch.bfloat16 out."""
    import torch

    m, k = x.shape
    n, k2 = w.shape
    if k != k2:
        raise NcmError(-2, "linear_bf16_rope64")
    if out is None:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_linear_bf16_rope64(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(w, "w"),
                                       _dev_ptr(bias, "bias"), _dev_ptr(out, "out"), m, k, n,
                                       rot_cols, seq_len, _dev_ptr(cosine, "cosine"),
                                       _dev_ptr(sine, "sine")),
          "linear_bf16_rope64")
    return out


def linear_f32(x, w, out=None, ctx=None):
    """y = x @ w.T with float32 operands [m, k] and [n, k] (k % 4 == 0) on
    the fp32 MFMA, on torch's current stream."""
    import torch

    m, k = x.shape
    n, k2 = w.shape
    if k != k2:
        raise NcmError(-2, "linear_f32")
    if out is None:
        out = torch.empty((m, n), dtype=torch.float32, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_linear_f32(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(w, "w"), _dev_ptr(out, "out"),
                               m, k, n), "linear_f32")
    return out


def bf16_from_f32(src, flush: bool = False, ctx=None):
    """Device f32 -> bf16 (RNE, NaN -> 0x7FC0), returned as torch.bfloat16."""
    import torch

    out = torch.empty(src.shape, dtype=torch.bfloat16, device=src.device)
    ctx = ctx or default_context(src.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_bf16_from_f32_dev(ctx.handle, _dev_ptr(src, "src"), _dev_ptr(out, "out"),
                                      src.numel(), 1 if flush else 0), "bf16_from_f32")
    return out


def bf16_widen(src, ctx=None):
    """Device bf16 -> f32 (exact)."""
    import torch

    out = torch.empty(src.shape, dtype=torch.float32, device=src.device)
    ctx = ctx or default_context(src.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_bf16_widen_dev(ctx.handle, _dev_ptr(src, "src"), _dev_ptr(out, "out"),
                                   src.numel()), "bf16_widen")
    return out


def rms_norm_rows(x, weight, epsilon: float, out_mode: str = "bf16_f32", out=None, ctx=None):
    """RMSNorm (bf16 mode) of every row of x (float32 [rows, width]) with
    weight (float32 [width]) on torch's current stream; out_mode "bf16_f32"
    (float32 holding bf16 values) or "bf16" (torch.bfloat16)."""
    import torch

    rows, width = x.shape
    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.bfloat16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty((rows, width), dtype=dt, device=x.device)
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_rms_norm_rows_dev(ctx.handle, _dev_ptr(x, "x"), _dev_ptr(weight, "weight"),
                                      _dev_ptr(out, "out"), rows, width, float(epsilon), mode),
          "rms_norm_rows")
    return out


def silu_mul(gate, up=None, out_mode: str = "bf16_f32", out=None, ctx=None):
    """round_bf16(silu_bf16(gate) * up) elementwise (up None: silu_bf16) on
    torch's current stream."""
    import torch

    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.bfloat16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty(gate.shape, dtype=dt, device=gate.device)
    ctx = ctx or default_context(gate.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_silu_mul_dev(ctx.handle, _dev_ptr(gate, "gate"), _dev_ptr(up, "up"),
                                 _dev_ptr(out, "out"), gate.numel(), mode), "silu_mul")
    return out


def _rows_ptr(t, name):
    """Pointer and row stride of a 2-D GPU tensor whose rows are contiguous
    (a column slice of a wider buffer is allowed)."""
    if not t.is_cuda or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D GPU tensor with contiguous rows")
    return C.c_void_p(t.data_ptr()), t.stride(0)


def rope_rotate(x, heads: int, head_dim: int, seq_len: int, cosine, sine, ctx=None):
    """In-place bf16 RoPE (rotate_head, root.zig:615-634) of every head of
    every row of x (torch.bfloat16 [rows, >= heads * head_dim], rows may be
    strided); row r uses table row r % seq_len of cosine/sine (float32
    [seq_len, head_dim])."""
    ptr, stride = _rows_ptr(x, "x")
    ctx = ctx or default_context(x.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_rope_rotate_dev(ctx.handle, ptr, x.shape[0], stride, heads, head_dim, seq_len,
                                    _dev_ptr(cosine, "cosine"), _dev_ptr(sine, "sine")),
          "rope_rotate")
    return x


def attention_bf16(q, k, v, batch: int, seq_len: int, q_heads: int, kv_heads: int,
                   head_dim: int, window: int = 0, out_mode: str = "bf16_f32", out=None,
                   ctx=None):
    """Causal bf16 attention (root.zig:536-578) of `batch` sequences: q
    [batch * seq_len, >= q_heads * head_dim], k and v [batch * seq_len,
    >= kv_heads * head_dim], torch.bfloat16 with contiguous rows (column
    slices of one q|k|v buffer are allowed)."""
    import torch

    qp, qs = _rows_ptr(q, "q")
    kp, ks = _rows_ptr(k, "k")
    vp_, vs = _rows_ptr(v, "v")
    if ks != vs:
        raise NcmError(-2, "attention_bf16: k and v row strides differ")
    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.bfloat16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty((batch * seq_len, q_heads * head_dim), dtype=dt, device=q.device)
    op, os_ = _rows_ptr(out, "out")
    ctx = ctx or default_context(q.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_attention_bf16_dev(ctx.handle, qp, kp, vp_, op, batch, seq_len, q_heads,
                                       kv_heads, head_dim, qs, ks, os_, window, mode),
          "attention_bf16")
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
    int32 and pad_bits uint64 device tensors (block_diagonal_segments)."""
    import torch

    qp, qs = _rows_ptr(q, "q")
    kp, ks = _rows_ptr(k, "k")
    vp_, vs = _rows_ptr(v, "v")
    if ks != vs:
        raise NcmError(-2, "attention_bf16_seg: k and v row strides differ")
    mode = _OUT_MODES[out_mode]
    if out is None:
        dt = torch.bfloat16 if mode == NCM_OUT_BF16 else torch.float32
        out = torch.empty((batch * seq_len, q_heads * head_dim), dtype=dt, device=q.device)
    op, os_ = _rows_ptr(out, "out")
    ctx = ctx or default_context(q.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_attention_bf16_seg_dev(ctx.handle, qp, kp, vp_, op, batch, seq_len, q_heads,
                                           kv_heads, head_dim, qs, ks, os_, prefix_len,
                                           _dev_ptr(seg_lo, "seg_lo"), _dev_ptr(seg_hi, "seg_hi"),
                                           _dev_ptr(pad_bits, "pad_bits"), mode),
          "attention_bf16_seg")
    return out


def tied_head_logits(z, codebook, csq, log_inv_t: float = 0.0, bias=None, out=None, ctx=None):
    """Codebook-tied NCM code head (PROJECT.md:222): logits = (2 z E^T - csq)
    * exp(log_inv_t) / mean(csq) (+ bias). z: torch.bfloat16 [rows, d] on the
    GPU, codebook: torch.bfloat16 [v, d], csq: float32 [v] (vq.prepare), bias:
    float32 [v] or None; returns float32 [rows, v]."""
    import torch

    rows, d = z.shape
    v, d2 = codebook.shape
    if d != d2 or tuple(csq.shape) != (v,):
        raise NcmError(-2, "tied_head_logits")
    if out is None:
        out = torch.empty((rows, v), dtype=torch.float32, device=z.device)
    ctx = ctx or default_context(z.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_tied_head_logits(ctx.handle, _dev_ptr(z, "z"), _dev_ptr(codebook, "codebook"),
                                     _dev_ptr(csq, "csq"), _dev_ptr(bias, "bias"),
                                     float(log_inv_t), _dev_ptr(out, "out"), rows, d, v),
          "tied_head_logits")
    return out


def tied_head_logits_levels(z, codebooks, csq, level_rows, log_inv_t=None, bias=None, out=None,
                            ctx=None):
    """Every level's tied head in one launch: z torch.bfloat16 [sum rows, d]
    (level blocks in order, level_rows[l] rows each), codebooks bfloat16
    [levels, v, d], csq float32 [levels, v], log_inv_t: one float per level
    (default 0), bias float32 [levels, v] or None; float32 [sum rows, v]."""
    import torch

    L, v, d = codebooks.shape
    rows = np.ascontiguousarray(level_rows, dtype=np.int64)
    lit = np.ascontiguousarray(np.zeros(L) if log_inv_t is None else log_inv_t, dtype=np.float32)
    if (rows.size != L or lit.size != L or tuple(z.shape) != (int(rows.sum()), d)
            or tuple(csq.shape) != (L, v)):
        raise NcmError(-2, "tied_head_logits_levels")
    if out is None:
        out = torch.empty((int(rows.sum()), v), dtype=torch.float32, device=z.device)
    ctx = ctx or default_context(z.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_tied_head_logits_levels(
        ctx.handle, _dev_ptr(z, "z"), _dev_ptr(codebooks, "codebooks"), _dev_ptr(csq, "csq"),
        _dev_ptr(bias, "bias"), lit.ctypes.data_as(C.c_void_p), rows.ctypes.data_as(C.c_void_p),
        L, d, v, _dev_ptr(out, "out")), "tied_head_logits_levels")
    return out
