"""ctypes wrapper of the C oracle (libncm_oracle.so). TEST INFRASTRUCTURE ONLY.

Imported by the test suite, the smoke check and the benchmark's CPU-baseline
leg. The product path never imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libncm_oracle.so")
_lib = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
vp = C.c_void_p
sz = C.c_size_t
i64 = C.c_int64


def build() -> str:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = C.CDLL(_LIB_PATH)
        L.ncmo_bf16_from_f32.argtypes = [C.c_float]
        L.ncmo_bf16_from_f32.restype = C.c_uint16
        L.ncmo_bf16_to_f32.argtypes = [C.c_uint16]
        L.ncmo_bf16_to_f32.restype = C.c_float
        L.ncmo_round_bf16.argtypes = [C.c_float]
        L.ncmo_round_bf16.restype = C.c_float
        L.ncmo_flush_f32_subnormal.argtypes = [C.c_float]
        L.ncmo_flush_f32_subnormal.restype = C.c_float
        L.ncmo_bf16_from_f32_array.argtypes = [f32p, u16p, sz]
        L.ncmo_widen_little_endian.argtypes = [f32p, u8p, sz]
        L.ncmo_matmul_bf16.argtypes = [f32p, f32p, vp, f32p, vp, sz, sz, sz]
        L.ncmo_matmul_bf16_mt.argtypes = [f32p, f32p, vp, f32p, vp, sz, sz, sz, C.c_int]
        L.ncmo_matmul_bf16_rows.argtypes = [f32p, f32p, vp, f32p, vp, sz, sz, sz, sz, sz]
        L.ncmo_matmul_bf16_u16_rows.argtypes = [u16p, u16p, vp, f32p, vp, sz, sz, sz, sz, sz]
        L.ncmo_matmul_reference.argtypes = [f32p, f32p, f32p, sz, sz, sz]
        L.ncmo_matmul_f64.argtypes = [f32p, f32p, f64p, vp, sz, sz, sz]
        L.ncmo_fnv1a_bf16_digest.argtypes = [f32p, sz]
        L.ncmo_fnv1a_bf16_digest.restype = C.c_uint64
        L.ncmo_dot_fixed.argtypes = [f32p, u16p, i64]
        L.ncmo_dot_fixed.restype = C.c_float
        L.ncmo_sumsq_bf16_fixed.argtypes = [u16p, i64]
        L.ncmo_sumsq_bf16_fixed.restype = C.c_float
        L.ncmo_rvq_csq.argtypes = [u16p, i64, i64, i64, f32p]
        L.ncmo_rvq_check_strides.argtypes = [i64, i64, i32p]
        L.ncmo_rvq_codes_per_batch.argtypes = [i64, i64, i32p]
        L.ncmo_rvq_codes_per_batch.restype = i64
        L.ncmo_rvq_encode.argtypes = [f32p, i64, i64, i64, i64, i32p, u16p, f32p, i64, i32p,
                                      vp, vp, vp, C.c_int]
        L.ncmo_rvq_level_rows.argtypes = [f32p, i64, i64, i64, i64, i32p, u16p, f32p, i64,
                                          i32p, i64, i64p, i64, i32p, vp, vp]
        L.ncmo_rvq_decode.argtypes = [i32p, i64, i64, i64, i64, i32p, u16p, i64, f32p]
        L.ncmo_rvq_encode_f64.argtypes = [f32p, i64, i64, i64, i64, i32p, u16p, i64, i32p,
                                          vp, vp]
        L.ncmo_sum_squares_pinned.argtypes = [f32p, sz]
        L.ncmo_sum_squares_pinned.restype = C.c_float
        L.ncmo_rms_norm.argtypes = [f32p, f32p, f32p, sz, C.c_float, C.c_int]
        L.ncmo_silu_bf16.argtypes = [f32p, f32p, sz]
        L.ncmo_silu_mul_bf16.argtypes = [f32p, f32p, f32p, sz]
        L.ncmo_rotate_head.argtypes = [f32p, f32p, f32p, sz, C.c_int]
        L.ncmo_causal_mask.argtypes = [sz, sz, sz, u8p]
        L.ncmo_block_diagonal_mask.argtypes = [sz, vp, sz, vp, sz, u8p, sz]
        L.ncmo_rope_default_frequencies.argtypes = [sz, C.c_float, f32p]
        L.ncmo_rope_llama3.argtypes = [sz, C.c_float, C.c_float, C.c_float, C.c_float, sz, f32p]
        L.ncmo_rope_tables.argtypes = [f32p, sz, sz, f32p, f32p]
        L.ncmo_attention_core.argtypes = [f32p, f32p, f32p, u8p, f32p, sz, sz, sz, sz, C.c_int]
        L.ncmo_silu.argtypes = [f32p, f32p, sz]
        L.ncmo_fill_level_positions.argtypes = [sz, vp, sz, i64p, sz]
        L.ncmo_post_upsample_conv.argtypes = [f32p, f32p, f32p, sz, sz]
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- bf16
def bf16_from_f32(values) -> np.ndarray:
    a = np.ascontiguousarray(values, dtype=np.float32).ravel()
    out = np.empty(a.shape, np.uint16)
    lib().ncmo_bf16_from_f32_array(a, out, a.size)
    return out.reshape(np.shape(values))


def bf16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(values) -> np.ndarray:
    return bf16_to_f32(bf16_from_f32(values))


# ---------------------------------------------------------------- linear
def matmul_bf16(x, w, bias=None, token_count=None, input_width=None, output_width=None,
                want_sum=False):
    """Reference matmul_bf16 / matmul_bf16_bias (root.zig:96-142).
    x: f32 [T, in]; w: f32 [out, in]; bias: f32 [out] or None."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    T = x.shape[0] if token_count is None else token_count
    K = x.shape[-1] if input_width is None else input_width
    N = w.shape[0] if output_width is None else output_width
    out = np.empty((T, N), np.float32)
    s = np.empty((T, N), np.float32) if want_sum else None
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    if _THREADS > 1:
        lib().ncmo_matmul_bf16_mt(x.ravel(), w.ravel(), _ptr(b), out, _ptr(s), T, K, N,
                                  _THREADS)
    else:
        lib().ncmo_matmul_bf16(x.ravel(), w.ravel(), _ptr(b), out, _ptr(s), T, K, N)
    return (out, s) if want_sum else out


_THREADS = 1


def set_threads(n: int) -> int:
    """Threads for matmul_bf16 (and so decoder_forward): output columns split
    over POSIX threads, bit-identical results. Returns the previous value."""
    global _THREADS
    prev, _THREADS = _THREADS, max(1, int(n))
    return prev


def matmul_bf16_u16_rows(x_bits, w_bits, row_begin, row_end, bias_bits=None):
    """Same arithmetic on bf16 bit patterns; rows [row_begin, row_end) only.
    Returns (bf16-rounded output rows, fp32 pre-rounding sums)."""
    x_bits = np.ascontiguousarray(x_bits, np.uint16)
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    T, K = x_bits.shape
    N = w_bits.shape[0]
    out = np.zeros((T, N), np.float32)
    s = np.zeros((T, N), np.float32)
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)
    lib().ncmo_matmul_bf16_u16_rows(x_bits, w_bits, _ptr(b), out, _ptr(s), T, K, N,
                                    row_begin, row_end)
    return out[row_begin:row_end], s[row_begin:row_end]


def matmul_reference(x, w):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().ncmo_matmul_reference(x, w, out, x.shape[0], x.shape[1], w.shape[0])
    return out


def matmul_f64(x, w):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty((x.shape[0], w.shape[0]), np.float64)
    a = np.empty_like(out)
    lib().ncmo_matmul_f64(x, w, out, _ptr(a), x.shape[0], x.shape[1], w.shape[0])
    return out, a


def digest(values) -> int:
    v = np.ascontiguousarray(values, np.float32).ravel()
    return int(lib().ncmo_fnv1a_bf16_digest(v, v.size))


# ---------------------------------------------------------------- RVQ
def rvq_csq(codebooks_bits):
    cb = np.ascontiguousarray(codebooks_bits, np.uint16)
    L, V, D = cb.shape
    csq = np.empty((L, V), np.float32)
    lib().ncmo_rvq_csq(cb, L, V, D, csq)
    return csq


def codes_per_batch(t, strides):
    s = np.ascontiguousarray(strides, np.int32)
    return int(lib().ncmo_rvq_codes_per_batch(t, len(s), s))


def rvq_encode(x, codebooks_bits, strides, csq=None, forced=None, want_recon=True,
               want_gap=True, threads=1):
    """x: f32 [B, T, d]; codebooks: bf16 bits [L, V, d]. Returns dict."""
    x = np.ascontiguousarray(x, np.float32)
    cb = np.ascontiguousarray(codebooks_bits, np.uint16)
    B, T, D = x.shape
    L, V, _ = cb.shape
    s = np.ascontiguousarray(strides, np.int32)
    rc = lib().ncmo_rvq_check_strides(T, len(s), s)
    if rc != 0:
        raise ValueError(f"invalid strides {tuple(strides)} for t={T}: {rc}")
    if csq is None:
        csq = rvq_csq(cb)
    csq = np.ascontiguousarray(csq, np.float32)
    total = codes_per_batch(T, s)
    codes = np.zeros((B, total), np.int32)
    recon = np.empty((B, T, D), np.float32) if want_recon else None
    gap = np.empty((B, total), np.float32) if want_gap else None
    fr = None if forced is None else np.ascontiguousarray(forced, np.int32)
    rc = lib().ncmo_rvq_encode(x, B, T, D, L, s, cb, csq, V, codes, _ptr(recon), _ptr(gap),
                               _ptr(fr), threads)
    if rc != 0:
        raise ValueError(f"ncmo_rvq_encode failed: {rc}")
    return {"codes": codes, "recon": recon, "gap": gap, "csq": csq}


def rvq_level_rows(x, codebooks_bits, strides, csq, codes, level, rows, want_u=False):
    x = np.ascontiguousarray(x, np.float32)
    cb = np.ascontiguousarray(codebooks_bits, np.uint16)
    B, T, D = x.shape
    L, V, _ = cb.shape
    s = np.ascontiguousarray(strides, np.int32)
    rows = np.ascontiguousarray(rows, np.int64)
    out = np.empty(rows.shape[0], np.int32)
    gap = np.empty(rows.shape[0], np.float32)
    u = np.empty((rows.shape[0], D), np.float32) if want_u else None
    rc = lib().ncmo_rvq_level_rows(x, B, T, D, L, s, cb, np.ascontiguousarray(csq, np.float32),
                                   V, np.ascontiguousarray(codes, np.int32), level, rows,
                                   rows.shape[0], out, _ptr(gap), _ptr(u))
    if rc != 0:
        raise ValueError(f"ncmo_rvq_level_rows failed: {rc}")
    return (out, gap, u) if want_u else (out, gap)


def rvq_decode(codes, codebooks_bits, strides, t):
    cb = np.ascontiguousarray(codebooks_bits, np.uint16)
    L, V, D = cb.shape
    codes = np.ascontiguousarray(codes, np.int32)
    B = codes.shape[0]
    s = np.ascontiguousarray(strides, np.int32)
    recon = np.empty((B, t, D), np.float32)
    rc = lib().ncmo_rvq_decode(codes, B, t, D, L, s, cb, V, recon)
    if rc != 0:
        raise ValueError(f"ncmo_rvq_decode failed: {rc}")
    return recon


def rvq_encode_f64(x, codebooks_bits, strides, forced=None):
    x = np.ascontiguousarray(x, np.float32)
    cb = np.ascontiguousarray(codebooks_bits, np.uint16)
    B, T, D = x.shape
    L, V, _ = cb.shape
    s = np.ascontiguousarray(strides, np.int32)
    total = int(sum(T // int(v) for v in s))
    codes = np.zeros((B, total), np.int32)
    gap = np.empty((B, total), np.float64)
    fr = None if forced is None else np.ascontiguousarray(forced, np.int32)
    rc = lib().ncmo_rvq_encode_f64(x, B, T, D, L, s, cb, V, codes, _ptr(gap), _ptr(fr))
    if rc != 0:
        raise ValueError(f"ncmo_rvq_encode_f64 failed: {rc}")
    return codes, gap


# ------------------------------------------------------------ decoder ops
def sum_squares_pinned(x) -> np.float32:
    """pinned_torch_sum_squares_f32 (packages/kernels/root.zig:152-227)."""
    a = np.ascontiguousarray(x, np.float32).ravel()
    return np.float32(lib().ncmo_sum_squares_pinned(a, a.size))


def rms_norm(x, weight, epsilon: float, bf16: bool = True) -> np.ndarray:
    """rms_norm / rms_norm_bf16 (root.zig:229-254) of every row of x [.., n]."""
    a = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(weight, np.float32).ravel()
    n = a.shape[-1]
    rows = a.reshape(-1, n)
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        lib().ncmo_rms_norm(np.ascontiguousarray(rows[r]), w, out[r], n, epsilon, 1 if bf16 else 0)
    return out.reshape(a.shape)


def silu_bf16(x) -> np.ndarray:
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    lib().ncmo_silu_bf16(a.ravel(), out.ravel(), a.size)
    return out


def silu_mul_bf16(gate, up) -> np.ndarray:
    g = np.ascontiguousarray(gate, np.float32)
    u = np.ascontiguousarray(up, np.float32)
    out = np.empty_like(g)
    lib().ncmo_silu_mul_bf16(g.ravel(), u.ravel(), out.ravel(), g.size)
    return out


def rotate_heads(x, cosine, sine, heads: int, head_dim: int, bf16: bool = True) -> np.ndarray:
    """rotate_head (root.zig:615-634) applied to every head of every row of
    x [rows, heads * head_dim]; row r uses table row r of cosine/sine
    [rows, head_dim]. Returns a new array."""
    out = np.array(x, np.float32, copy=True).reshape(-1, heads * head_dim)
    cos = np.ascontiguousarray(cosine, np.float32).reshape(-1, head_dim)
    sin = np.ascontiguousarray(sine, np.float32).reshape(-1, head_dim)
    for r in range(out.shape[0]):
        for h in range(heads):
            seg = np.ascontiguousarray(out[r, h * head_dim:(h + 1) * head_dim])
            lib().ncmo_rotate_head(seg, np.ascontiguousarray(cos[r]), np.ascontiguousarray(sin[r]),
                                   head_dim, 1 if bf16 else 0)
            out[r, h * head_dim:(h + 1) * head_dim] = seg
    return out


def causal_mask(count: int, window: int = 0) -> np.ndarray:
    """causal_mask (root.zig:380-399) for positions 0..count-1, uint8 [count, count]."""
    out = np.empty((count, count), np.uint8)
    lib().ncmo_causal_mask(count, count, window, out)
    return out


def attention_core(q, k, v, mask, q_heads: int, kv_heads: int, head_dim: int,
                   bf16: bool = True) -> np.ndarray:
    """Scores, softmax and context of attention_impl (root.zig:536-578) for
    one sequence: q [T, q_heads * head_dim], k/v [T, kv_heads * head_dim]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    t = q.shape[0]
    m = np.ascontiguousarray(mask, np.uint8)
    out = np.empty((t, q_heads * head_dim), np.float32)
    lib().ncmo_attention_core(q, k, v, m, out, t, q_heads, kv_heads, head_dim, 1 if bf16 else 0)
    return out


def rope_default_frequencies(head_dim: int, theta: float) -> np.ndarray:
    """Inverse frequencies of rope_default (root.zig:305-326, 676-682)."""
    out = np.empty(head_dim // 2, np.float32)
    lib().ncmo_rope_default_frequencies(head_dim, theta, out)
    return out


def rope_llama3(head_dim: int, theta: float, factor: float, low_freq_factor: float,
                high_freq_factor: float, original_max_positions: int) -> np.ndarray:
    """Llama 3 adjusted inverse frequencies (root.zig:636-674)."""
    out = np.empty(head_dim // 2, np.float32)
    lib().ncmo_rope_llama3(head_dim, theta, factor, low_freq_factor, high_freq_factor,
                           original_max_positions, out)
    return out


def rope_tables(inv, positions: int):
    """Duplicated rotate-half cosine and sine tables (root.zig:328-348),
    each [positions, 2 * len(inv)]."""
    inv = np.ascontiguousarray(inv, np.float32)
    half = inv.size
    cos = np.empty((positions, 2 * half), np.float32)
    sin = np.empty((positions, 2 * half), np.float32)
    lib().ncmo_rope_tables(inv, half, positions, cos, sin)
    return cos, sin


def decoder_forward(ids, embed, layers, final_norm, lm_head, cos, sin, q_heads, kv_heads,
                    head_dim, eps, window=0, bf16=True, trace=None):
    """forward_with_trace (src/decoder.zig:62-228) for one sequence, composed
    of the restatements above: bf16_compute (bf16=True) or the f32 mode.
    Weights are float32 (bf16 values in bf16 mode); each layer is a dict with
    input_norm, qkv_weight [(q_heads + 2 kv_heads) head_dim, hidden] (the q,
    k and v projections' rows in that order), qkv_bias, o_weight, o_bias,
    post_attention_norm, gate_up_weight [2 intermediate, hidden] (gate rows
    then up rows), gate_up_bias, down_weight, down_bias (biases may be None),
    and optionally q_norm and k_norm [head_dim]: RMSNorm scales applied to
    every query and key head before the rotation (attention_impl's QK-norm,
    root.zig:501-530). lm_head None: tied to embed. cos, sin: [len(ids),
    head_dim]. trace: a dict that receives the stages of decoder_trace_t
    (decoder.zig:30-47), each [layers, tokens, width] (block_input [tokens,
    hidden])."""
    t = len(ids)
    rb = round_bf16 if bf16 else (lambda a: np.asarray(a, np.float32))
    hidden = rb(np.asarray(embed, np.float32)[np.asarray(ids)])
    qw, kvw = q_heads * head_dim, kv_heads * head_dim
    mask = causal_mask(t, window)
    stages = {k: [] for k in ("input_norm", "attention_context", "attention_output",
                              "attention_residual", "post_attention_norm", "gate_projection",
                              "up_projection", "gate_up_product", "mlp_output",
                              "block_output")}
    if trace is not None:
        trace["block_input"] = hidden.copy()

    def proj(x, w, b, lo=None, hi=None):
        w = np.asarray(w, np.float32)
        if lo is not None:
            w = w[lo:hi]
            b = None if b is None else np.asarray(b, np.float32)[lo:hi]
        if bf16:
            return matmul_bf16(x, w, b)
        y = matmul_reference(x, w)   # kernels.matmul, then the bias (root.zig:583-609)
        return y if b is None else (y + np.asarray(b, np.float32)[None, :]).astype(np.float32)

    for layer in layers:
        n = rms_norm(hidden, layer["input_norm"], eps, bf16=bf16)
        stages["input_norm"].append(n)
        wq, bq = layer["qkv_weight"], layer.get("qkv_bias")
        q = proj(n, wq, bq, 0, qw)
        k = proj(n, wq, bq, qw, qw + kvw)
        v = proj(n, wq, bq, qw + kvw, qw + 2 * kvw)
        if layer.get("q_norm") is not None:
            q = rms_norm(q.reshape(t * q_heads, head_dim), layer["q_norm"], eps,
                         bf16=bf16).reshape(t, qw)
            k = rms_norm(k.reshape(t * kv_heads, head_dim), layer["k_norm"], eps,
                         bf16=bf16).reshape(t, kvw)
        q = rotate_heads(q, cos, sin, q_heads, head_dim, bf16=bf16)
        k = rotate_heads(k, cos, sin, kv_heads, head_dim, bf16=bf16)
        ctx = attention_core(q, k, v, mask, q_heads, kv_heads, head_dim, bf16=bf16)
        stages["attention_context"].append(ctx)
        attn = proj(ctx, layer["o_weight"], layer.get("o_bias"))
        stages["attention_output"].append(attn)
        hidden = rb(hidden + attn)
        stages["attention_residual"].append(hidden)
        n = rms_norm(hidden, layer["post_attention_norm"], eps, bf16=bf16)
        stages["post_attention_norm"].append(n)
        inter = layer["gate_up_weight"].shape[0] // 2
        wg, bg = layer["gate_up_weight"], layer.get("gate_up_bias")
        gate = proj(n, wg, bg, 0, inter)
        up = proj(n, wg, bg, inter, 2 * inter)
        stages["gate_projection"].append(gate)
        stages["up_projection"].append(up)
        act = silu_mul_bf16(gate, up) if bf16 else (silu(gate) * up).astype(np.float32)
        stages["gate_up_product"].append(act)
        mlp = proj(act, layer["down_weight"], layer.get("down_bias"))
        stages["mlp_output"].append(mlp)
        hidden = rb(hidden + mlp)
        stages["block_output"].append(hidden)
    n = rms_norm(hidden, final_norm, eps, bf16=bf16)
    if trace is not None:
        for key, vals in stages.items():
            trace[key] = np.stack(vals) if vals else np.zeros((0, t, 0), np.float32)
    head = embed if lm_head is None else lm_head
    return matmul_bf16(n, head) if bf16 else matmul_reference(n, head)


# ------------------------------------------------------------ NCM body
def silu(x) -> np.ndarray:
    """kernels.silu, f32 mode (root.zig:255-261)."""
    a = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(a)
    lib().ncmo_silu(a.ravel(), out.ravel(), a.size)
    return out


def fill_level_positions(prefix_length: int, level_lengths) -> np.ndarray:
    """src/ncm_position.zig:11-22: prefix 0 .. P-1, each level from 0."""
    lv = np.ascontiguousarray(level_lengths, dtype=np.uintp)
    out = np.empty(prefix_length + int(lv.sum()), np.int64)
    rc = lib().ncmo_fill_level_positions(prefix_length, lv.ctypes.data_as(C.c_void_p), lv.size,
                                         out, out.size)
    if rc:
        raise ValueError("InvalidPositionBuffer")
    return out


def tables_at_positions(inv, positions):
    """src/ncm_position.zig:73-118: rope_tables over 0 .. max(positions), then
    the rows at `positions`."""
    pos = np.asarray(positions, np.int64)
    cos, sin = rope_tables(inv, int(pos.max()) + 1 if pos.size else 0)
    return np.ascontiguousarray(cos[pos]), np.ascontiguousarray(sin[pos])


def post_upsample_conv(x, weight, bias) -> np.ndarray:
    """apply_post_upsample_conv (src/ncm_model.zig:296-326) of one level chunk
    x [rows, width] with weight [width, width, 3] and bias [width]."""
    a = np.array(x, np.float32, copy=True, order="C")
    w = np.ascontiguousarray(weight, np.float32)
    b = np.ascontiguousarray(bias, np.float32)
    rows, width = a.shape
    if w.size != width * width * 3 or b.size != width:
        raise ValueError("InvalidNcmTensorSize")
    rc = lib().ncmo_post_upsample_conv(a.ravel(), w.ravel(), b.ravel(), rows, width)
    if rc:
        raise ValueError("InvalidNcmTensorSize")
    return a


def block_causal_mask(prefix_length: int, level_lengths, prefix_pad_mask=None):
    """Block-causal level mask (no reference code: the reference builds only
    block_diagonal_mask, decision D8): prefix queries see the unpadded prefix
    keys, and a level-l query sees the unpadded prefix keys and every key of
    levels 0 .. l. uint8 [S, S]."""
    lv = [int(n) for n in level_lengths]
    seq = prefix_length + sum(lv)
    pad = np.zeros(prefix_length, bool) if prefix_pad_mask is None else \
        np.asarray(prefix_pad_mask, bool)
    if pad.size != prefix_length:
        raise ValueError("InvalidPrefixMask")
    out = np.zeros((seq, seq), np.uint8)
    out[:, :prefix_length] = ~pad[None, :]
    off = prefix_length
    for n in lv:
        out[off:off + n, prefix_length:off + n] = 1
        off += n
    return out


def rms_norm_rows_with_bias(x, weight, bias, epsilon: float, bf16: bool) -> np.ndarray:
    """src/ncm_norm.zig:22-49: rms_norm of every row, then + bias. bf16 mode:
    rms_norm_bf16, and the bias add rounded to bf16 as every other tensor op
    of the bf16 forward (src/decoder.zig:279-282)."""
    y = rms_norm(x, weight, epsilon, bf16=bf16)
    if bias is not None:
        y = y + np.asarray(bias, np.float32)[None, :]
        if bf16:
            y = round_bf16(y)
    return y


def _ncm_dims(cfg):
    return (cfg["hidden_size"], cfg["vq_width"], cfg["num_attention_heads"],
            cfg["num_key_value_heads"], cfg["head_dim"], cfg["intermediate_size"],
            cfg["rms_norm_epsilon"], [int(n) for n in cfg["level_lengths"]],
            cfg["prefix_length"])


def _ncm_project(bf16):
    def project(x, w, b):
        if bf16:
            return matmul_bf16(x, w, b)
        y = matmul_reference(x, w)
        return y if b is None else (y + np.asarray(b, np.float32)[None, :]).astype(np.float32)
    return project


def ncm_input_stage(cfg, weights, prefix_ids, target_inputs, bf16: bool = False):
    """The NCM body's input stage (src/ncm_model.zig:99-168): prefix table
    rows, the target inputs (level 0 replaced by l0_queries when
    query_level0), each level's post-upsample conv, the input projection
    (+ bias) and the level embeddings. Returns hidden [S, hidden]."""
    H, vq, hq, hkv, hd, inter, eps, levels, P = _ncm_dims(cfg)
    ids = [int(i) for i in prefix_ids]
    T = sum(levels)
    S = P + T
    tgt = np.asarray(target_inputs, np.float32).reshape(-1)
    if tgt.size != T * vq:
        raise ValueError("InvalidNcmTensorSize")
    table = np.asarray(weights["prefix_token_embedding"], np.float32).reshape(-1, vq)
    l0q = weights.get("l0_queries")
    if cfg.get("query_level0", False):
        if l0q is None or np.asarray(l0q).size != levels[0] * vq:
            raise ValueError("InvalidNcmTensorSize")
    convs = weights.get("post_upsample_convs") or []
    if convs and len(convs) != len(levels):
        raise ValueError("InvalidNcmTensorSize")
    rb = round_bf16 if bf16 else (lambda a: np.asarray(a, np.float32))
    project = _ncm_project(bf16)
    projected = np.empty((S, vq), np.float32)
    for i, t in enumerate(ids):
        if t >= table.shape[0] or t < 0:
            raise ValueError("PrefixTokenOutOfRange")
        projected[i] = table[t]
    projected[P:] = tgt.reshape(T, vq)
    if cfg.get("query_level0", False):
        projected[P:P + levels[0]] = np.asarray(l0q, np.float32).reshape(levels[0], vq)
    off = P
    for n, conv in zip(levels, convs):
        projected[off:off + n] = post_upsample_conv(projected[off:off + n], conv["weight"],
                                                    conv["bias"])
        off += n
    hidden = project(projected, weights["input_projection"], weights["input_projection_bias"])
    if cfg.get("use_level_encoding", True):
        emb = np.asarray(weights["level_embedding"], np.float32).reshape(len(levels), H)
        off = P
        for l, n in enumerate(levels):
            hidden[off:off + n] = rb(hidden[off:off + n] + emb[l][None, :])
            off += n
    return hidden


def ncm_tables_and_mask(cfg, prefix_pad_mask=None, mask: str = "block_diagonal"):
    """The RoPE tables at the restarting level positions
    (src/ncm_position.zig:11-118) and the attention mask of the NCM body:
    (cos, sin, mask [S, S] bool)."""
    H, vq, hq, hkv, hd, inter, eps, levels, P = _ncm_dims(cfg)
    pad = [] if prefix_pad_mask is None else list(prefix_pad_mask)
    S = P + sum(levels)
    positions = fill_level_positions(P, levels)
    if cfg.get("rope", "default") == "llama3":
        inv = rope_llama3(hd, cfg["rope_theta"], cfg.get("rope_factor", 1.0),
                          cfg.get("rope_low_freq_factor", 1.0),
                          cfg.get("rope_high_freq_factor", 4.0),
                          cfg.get("rope_original_max_position_embeddings", 8192))
    else:
        inv = rope_default_frequencies(hd, cfg["rope_theta"])
    cos, sin = tables_at_positions(inv, positions)
    if cfg.get("source_causal", False):
        m = causal_mask(S, cfg.get("sliding_window") or 0)
    elif mask == "block_causal":
        m = block_causal_mask(P, levels, pad if pad else None)
    else:
        m = block_diagonal_mask(P, levels, pad if pad else None)
    return cos, sin, m


def ncm_layer(cfg, layer, hidden, cos, sin, mask, bf16: bool = False):
    """One layer of the NCM body (src/ncm_model.zig:172-242): normalized
    input (+ norm bias), fused q|k|v projection, optional QK-norm, rotation
    at the level positions, masked attention, output projection and
    residual, post-attention norm, SiLU MLP and residual."""
    H, vq, hq, hkv, hd, inter, eps, levels, P = _ncm_dims(cfg)
    S = hidden.shape[0]
    rb = round_bf16 if bf16 else (lambda a: np.asarray(a, np.float32))
    project = _ncm_project(bf16)
    qw, kvw = hq * hd, hkv * hd
    n = rms_norm_rows_with_bias(hidden, layer["ln_1_weight"], layer.get("ln_1_bias"), eps, bf16)
    wq, bq = np.asarray(layer["fused_qkv_weight"], np.float32), layer.get("fused_qkv_bias")
    sl = lambda lo, hi: (wq[lo:hi], None if bq is None else np.asarray(bq)[lo:hi])
    q = project(n, *sl(0, qw))
    k = project(n, *sl(qw, qw + kvw))
    v = project(n, *sl(qw + kvw, qw + 2 * kvw))
    if layer.get("query_norm_weight") is not None:
        q = rms_norm(q.reshape(S * hq, hd), layer["query_norm_weight"], eps,
                     bf16=bf16).reshape(S, qw)
        k = rms_norm(k.reshape(S * hkv, hd), layer["key_norm_weight"], eps,
                     bf16=bf16).reshape(S, kvw)
    q = rotate_heads(q, cos, sin, hq, hd, bf16=bf16)
    k = rotate_heads(k, cos, sin, hkv, hd, bf16=bf16)
    ctx = attention_core(q, k, v, mask, hq, hkv, hd, bf16=bf16)
    attn = project(ctx, layer["output_weight"], layer.get("output_bias"))
    hidden = rb(hidden + attn)
    n = rms_norm_rows_with_bias(hidden, layer["ln_2_weight"], layer.get("ln_2_bias"), eps, bf16)
    gate = project(n, layer["gate_weight"], layer.get("gate_bias"))
    up = project(n, layer["up_weight"], layer.get("up_bias"))
    act = silu_mul_bf16(gate, up) if bf16 else (silu(gate) * up).astype(np.float32)
    mlp = project(act, layer["down_weight"], layer.get("down_bias"))
    return rb(hidden + mlp)


def ncm_final_norm(cfg, weights, hidden, bf16: bool = False):
    """The body's final norm (+ bias)."""
    return rms_norm_rows_with_bias(hidden, weights["final_norm_weight"],
                                   weights.get("final_norm_bias"), cfg["rms_norm_epsilon"], bf16)


def ncm_forward(cfg, weights, prefix_ids, prefix_pad_mask, target_inputs, bf16: bool = False,
                mask: str = "block_diagonal", trace: bool = False):
    """forward_with_trace of the NCM level-parallel body (src/ncm_model.zig:
    89-250). bf16=False restates the reference exactly (f32 matmul,
    attention, RMSNorm and SiLU); bf16=True is the same body in the bf16
    mode of the source decoder (src/decoder.zig:62-228 with bf16_compute):
    every projection is matmul_bf16(_bias), norms are rms_norm_bf16, SiLU is
    silu_bf16 with a rounded product, attention is attention_bf16, and every
    add (level embedding, norm bias, residual) is rounded to bf16.
    mask: "block_diagonal" (the reference, src/ncm_mask.zig:10-42) or
    "block_causal". Returns the final-normalized hidden states [S, hidden]
    (and the states after the input stage and each layer when trace)."""
    H, vq, hq, hkv, hd, inter, eps, levels, P = _ncm_dims(cfg)
    ids = [int(i) for i in prefix_ids]
    pad = [] if prefix_pad_mask is None else list(prefix_pad_mask)
    if len(ids) != P:
        raise ValueError("InvalidPrefixLength")
    if len(pad) not in (0, P):
        raise ValueError("InvalidPrefixMask")
    if not levels:
        raise ValueError("InvalidNcmMode")
    if min(H, vq, hd, inter) == 0 or hd % 2 or hq == 0 or hkv == 0 or hq % hkv:
        raise ValueError("InvalidNcmDimensions")
    layers = weights["layers"]
    if not layers:
        raise ValueError("InvalidNcmTensorSize")
    hidden = ncm_input_stage(cfg, weights, ids, target_inputs, bf16)
    states = [hidden.copy()] if trace else None
    cos, sin, m = ncm_tables_and_mask(cfg, pad if pad else None, mask)
    for layer in layers:
        hidden = ncm_layer(cfg, layer, hidden, cos, sin, m, bf16)
        if trace:
            states.append(hidden.copy())
    out = ncm_final_norm(cfg, weights, hidden, bf16)
    if trace:
        states[-1] = out
        return out, states
    return out


# ------------------------------------------------------------ safetensors
# Restatement of packages/safetensors/root.zig:136-193 (header) and 197-228
# (index) with Python's json module. Errors are returned as the reference's
# error names.
ST_DTYPES = [("BOOL", 8), ("U8", 8), ("I8", 8), ("U16", 16), ("I16", 16), ("U32", 32),
             ("I32", 32), ("U64", 64), ("I64", 64), ("F4", 4), ("F6_E2M3", 6), ("F6_E3M2", 6),
             ("F8_E5M2", 8), ("F8_E4M3", 8), ("F8_E8M0", 8), ("F8_E4M3FNUZ", 8),
             ("F8_E5M2FNUZ", 8), ("F16", 16), ("BF16", 16), ("F32", 32), ("F64", 64),
             ("C64", 64)]
ST_MAX_HEADER = 100_000_000


class StError(Exception):
    pass


def _st_json(text):
    import json

    def pairs(kv):
        out = {}
        for k, v in kv:
            out[k] = v  # a repeated key keeps its first position, last value
        return out

    def bad_constant(_):
        raise StError("SyntaxError")

    try:
        root = json.loads(text, object_pairs_hook=pairs, parse_constant=bad_constant)
    except ValueError:
        raise StError("SyntaxError")

    def check(v):  # a lone surrogate escape is not a valid JSON string
        for x in (list(v.keys()) + list(v.values()) if isinstance(v, dict) else
                  v if isinstance(v, list) else [v]):
            if isinstance(x, str):
                try:
                    x.encode("utf-8")
                except UnicodeEncodeError:
                    raise StError("SyntaxError")
            elif isinstance(x, (dict, list)):
                check(x)

    check(root)
    return root


def _st_uint(v):
    # std.json integers are i64; anything else (floats, bools, larger
    # integers, negatives) is not a non-negative integer.
    if isinstance(v, bool) or not isinstance(v, int) or v < 0 or v > 2**63 - 1:
        raise StError("InvalidHeader")
    return v


def st_parse_header(data: bytes, file_size: int):
    """Returns (header_len, data_len, [(name, dtype_index, shape, begin, end)])
    in data-offset order, or raises StError(name)."""
    if len(data) < 8:
        raise StError("HeaderTooSmall")
    hl = int.from_bytes(data[:8], "little")
    if hl > ST_MAX_HEADER:
        raise StError("HeaderTooLarge")
    if len(data) < 8 + hl:
        raise StError("InvalidHeaderLength")
    try:
        text = data[8:8 + hl].decode("utf-8")
    except UnicodeDecodeError:
        raise StError("InvalidUtf8")
    root = _st_json(text)
    if not isinstance(root, dict):
        raise StError("InvalidHeader")
    names = [n for n, _ in ST_DTYPES]
    tensors = []
    for name, value in root.items():
        if name == "__metadata__":
            if not isinstance(value, dict) or not all(isinstance(x, str) for x in value.values()):
                raise StError("InvalidHeader")
            continue
        if not isinstance(value, dict):
            raise StError("InvalidHeader")
        dt = value.get("dtype")
        if not isinstance(dt, str):
            raise StError("InvalidHeader")
        if dt not in names:
            raise StError("UnknownDtype")
        shape = value.get("shape")
        if not isinstance(shape, list):
            raise StError("InvalidHeader")
        shape = [_st_uint(d) for d in shape]
        offs = value.get("data_offsets")
        if not isinstance(offs, list) or len(offs) != 2:
            raise StError("InvalidHeader")
        begin, end = _st_uint(offs[0]), _st_uint(offs[1])
        tensors.append((name, names.index(dt), shape, begin, end))
    tensors.sort(key=lambda t: (t[3], t[4]))
    expected = 0
    for name, dt, shape, begin, end in tensors:
        if begin != expected or end < begin:
            raise StError("InvalidOffsets")
        expected = end
        count = 1
        for d in shape:
            count *= d
            if count >= 2**64:
                raise StError("ShapeOverflow")
        bits = count * ST_DTYPES[dt][1]
        if bits >= 2**64:
            raise StError("ShapeOverflow")
        if bits % 8:
            raise StError("MisalignedBits")
        if end - begin != bits // 8:
            raise StError("SizeMismatch")
    if 8 + hl + expected != file_size:
        raise StError("FileSizeMismatch")
    return hl, expected, tensors


def st_parse_index(text: str):
    """Returns ([(tensor, shard)], total_size or None), or raises StError."""
    root = _st_json(text)
    if not isinstance(root, dict):
        raise StError("InvalidIndex")
    wm = root.get("weight_map")
    if not isinstance(wm, dict):
        raise StError("InvalidIndex")
    entries = []
    for tensor, shard in wm.items():
        if not isinstance(shard, str):
            raise StError("InvalidIndex")
        if shard in ("", ".", "..") or any(c in shard for c in "/\\\0"):
            raise StError("UnsafeShardName")
        entries.append((tensor, shard))
    total = None
    if "metadata" in root:
        md = root["metadata"]
        if not isinstance(md, dict):
            raise StError("InvalidIndex")
        if "total_size" in md:
            total = _st_uint(md["total_size"])
    return entries, total



def block_diagonal_mask(prefix_length: int, level_lengths, prefix_pad_mask=None):
    """NCM's block-diagonal allow mask (src/ncm_mask.zig:10-42), uint8 [S, S];
    raises ValueError("InvalidPrefixMask") for a pad mask of the wrong length."""
    lv = np.ascontiguousarray(level_lengths, dtype=np.uintp)
    pad = None if prefix_pad_mask is None else np.ascontiguousarray(prefix_pad_mask, np.uint8)
    seq = prefix_length + int(lv.sum())
    out = np.empty((seq, seq), np.uint8)
    rc = lib().ncmo_block_diagonal_mask(prefix_length, lv.ctypes.data_as(C.c_void_p), lv.size,
                                        None if pad is None else pad.ctypes.data_as(C.c_void_p),
                                        0 if pad is None else pad.size, out, out.size)
    if rc == -1:
        raise ValueError("InvalidPrefixMask")
    return out


def tied_head_logits_f64(z, codebook, log_inv_t=0.0, bias=None):
    """The NCM codebook-tied code head as the reference describes it
    (PROJECT.md:222, upstream _TiedCodebookHead; no reference code exists):
    E_sq = sum E^2 per code, d_scale = mean(E_sq), logits = (2 z E^T - E_sq)
    / d_scale * exp(log_inv_T) (+ bias), evaluated in f64 on the values given
    (bf16 operands widened to float). Returns (logits, sum of |2 z_i E_ki|
    per entry) for error bounds."""
    z64 = np.asarray(z, np.float64)
    e64 = np.asarray(codebook, np.float64)
    esq = np.sum(e64 * e64, axis=1)
    scale = np.exp(np.float64(log_inv_t)) / esq.mean()
    s = z64 @ e64.T
    logits = (2.0 * s - esq[None, :]) * scale
    if bias is not None:
        logits = logits + np.asarray(bias, np.float64)[None, :]
    mag = 2.0 * (np.abs(z64) @ np.abs(e64).T)
    return logits, mag
