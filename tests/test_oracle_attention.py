"""Pins of the oracle's RoPE and attention restatements (packages/kernels/
root.zig:272-284, 305-348, 380-399, 536-578, 615-682) against what the
mathematics and the published formulas fix: the rotate-half form of RoPE,
Meta's Llama 3 frequency scaling, f64 attention, closed forms of the
softmax, and the reference's own masked-query check."""
import math

import numpy as np
import pytest


def _rotate_half_f32(x, cos, sin, heads, hd):
    """q * cos + rotate_half(q) * sin, float32, product then sum per element."""
    out = np.empty_like(x)
    half = hd // 2
    for h in range(heads):
        s = x[:, h * hd:(h + 1) * hd]
        rot = np.concatenate([-s[:, half:], s[:, :half]], axis=1)
        out[:, h * hd:(h + 1) * hd] = (s * cos) + (rot * sin)
    return out


def _tables(oracle, positions, hd=64, theta=500000.0):
    inv = oracle.rope_llama3(hd, theta, 32.0, 1.0, 4.0, 8192)
    return oracle.rope_tables(inv, positions)


def test_rotate_f32_is_rotate_half(oracle):
    rng = np.random.default_rng(11)
    cos, sin = _tables(oracle, 96)
    x = rng.standard_normal((96, 2 * 64)).astype(np.float32)
    got = oracle.rotate_heads(x, cos, sin, 2, 64, bf16=False)
    assert np.array_equal(got.view(np.uint32), _rotate_half_f32(x, cos, sin, 2, 64).view(np.uint32))


def test_rotate_bf16_rounds_at_each_tensor_op(oracle):
    # The bf16 tensors of the rotate-half form: q*cos, rotate_half(q)*sin and
    # their sum each rounded to bf16, with bf16 tables.
    rng = np.random.default_rng(12)
    cos, sin = _tables(oracle, 50)
    x = oracle.round_bf16(rng.standard_normal((50, 3 * 64)).astype(np.float32) * 3)
    rb = oracle.round_bf16
    cb, sb = rb(cos), rb(sin)
    want = np.empty_like(x)
    for h in range(3):
        s = x[:, h * 64:(h + 1) * 64]
        rot = np.concatenate([-s[:, 32:], s[:, :32]], axis=1)
        want[:, h * 64:(h + 1) * 64] = rb(rb(s * cb) + rb(rot * sb))
    got = oracle.rotate_heads(x, cos, sin, 3, 64, bf16=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_rotate_identity_and_quarter_turn(oracle):
    x = oracle.round_bf16(np.random.default_rng(13).standard_normal((4, 8)).astype(np.float32))
    one, zero = np.ones((4, 8), np.float32), np.zeros((4, 8), np.float32)
    for bf in (False, True):
        assert np.array_equal(oracle.rotate_heads(x, one, zero, 1, 8, bf16=bf), x)
        # cos 0, sin 1: (a, b) -> (-b, a)
        got = oracle.rotate_heads(x, zero, one, 1, 8, bf16=bf)
        assert np.array_equal(got, np.concatenate([-x[:, 4:], x[:, :4]], axis=1))


def test_rope_default_frequencies_f64(oracle):
    for hd, theta in ((64, 500000.0), (128, 10000.0), (2, 10000.0)):
        got = oracle.rope_default_frequencies(hd, theta).astype(np.float64)
        want = theta ** (-(2.0 * np.arange(hd // 2)) / hd)
        assert np.all(np.abs(got - want) <= 4 * 2.0**-24 * want)


def _llama3_f64(hd, theta, factor, low, high, orig):
    """Meta's published Llama 3 frequency scaling, in f64."""
    out = []
    low_wl, high_wl = orig / low, orig / high
    for i in range(hd // 2):
        f = theta ** (-(2.0 * i) / hd)
        wl = 2 * math.pi / f
        if wl < high_wl:
            out.append(f)
        elif wl > low_wl:
            out.append(f / factor)
        else:
            s = (orig / wl - low) / (high - low)
            out.append((1 - s) * f / factor + s * f)
    return np.array(out)


def test_rope_llama3_matches_published_scaling(oracle):
    # The Llama-3.2-1B parameters (the reference's B4 check, root.zig:960-984,
    # holds 1e-6 relative against Transformers' table).
    got = oracle.rope_llama3(64, 500000.0, 32.0, 1.0, 4.0, 8192).astype(np.float64)
    want = _llama3_f64(64, 500000.0, 32.0, 1.0, 4.0, 8192)
    assert np.all(np.abs(got - want) <= 1e-6 * want)
    # All three regimes occur at these parameters.
    wl = 2 * math.pi / want
    assert (wl < 8192 / 4).any() and (wl > 8192).any() and ((wl >= 2048) & (wl <= 8192)).any()


def test_rope_tables_layout_and_values(oracle):
    inv = oracle.rope_default_frequencies(16, 10000.0)
    cos, sin = oracle.rope_tables(inv, 300)
    assert np.array_equal(cos[:, :8], cos[:, 8:]) and np.array_equal(sin[:, :8], sin[:, 8:])
    ang = (np.arange(300, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    assert np.all(np.abs(cos[:, :8] - np.cos(ang)) <= 2.0**-23)
    assert np.all(np.abs(sin[:, :8] - np.sin(ang)) <= 2.0**-23)
    assert np.all(cos[0] == 1) and np.all(sin[0] == 0)


@pytest.mark.parametrize("window", [0, 1, 3, 50])
def test_causal_mask(oracle, window):
    n = 20
    q, k = np.meshgrid(np.arange(n), np.arange(n), indexing="ij")
    want = (k <= q) & ((window == 0) | (q - window < k))
    assert np.array_equal(oracle.causal_mask(n, window).astype(bool), want)


def _attention_f64(q, k, v, mask, hq, hkv, hd):
    t = q.shape[0]
    out = np.zeros((t, hq * hd))
    g = hq // hkv
    for h in range(hq):
        kv = h // g
        qs = q[:, h * hd:(h + 1) * hd].astype(np.float64)
        ks = k[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        vs = v[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        s = qs @ ks.T / math.sqrt(hd)
        s = np.where(mask.astype(bool), s, -np.inf)
        e = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (e / e.sum(axis=1, keepdims=True)) @ vs
    return out


@pytest.mark.parametrize("window", [0, 5])
def test_attention_f32_mode_against_f64(oracle, window):
    rng = np.random.default_rng(20 + window)
    t, hq, hkv, hd = 40, 4, 2, 16
    q = rng.standard_normal((t, hq * hd)).astype(np.float32)
    k = rng.standard_normal((t, hkv * hd)).astype(np.float32)
    # Distinct value heads, so a wrong query-to-kv head map fails.
    v = (rng.standard_normal((t, hkv * hd)) + np.repeat(np.arange(hkv) * 10.0, hd)).astype(np.float32)
    mask = oracle.causal_mask(t, window)
    got = oracle.attention_core(q, k, v, mask, hq, hkv, hd, bf16=False)
    want = _attention_f64(q, k, v, mask, hq, hkv, hd)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(v))


def test_attention_bf16_uniform_scores_closed_form(oracle):
    # q = 0: every allowed score is 0, p = round_bf16(1 / allowed count), and
    # the context is the bf16 rounding of the key-order fp32 sum of p v.
    rng = np.random.default_rng(21)
    t, hd = 30, 8
    q = np.zeros((t, hd), np.float32)
    k = oracle.round_bf16(rng.standard_normal((t, hd)).astype(np.float32))
    v = oracle.round_bf16(rng.standard_normal((t, hd)).astype(np.float32))
    got = oracle.attention_core(q, k, v, oracle.causal_mask(t), 1, 1, hd, bf16=True)
    for i in range(t):
        p = oracle.round_bf16(np.float32(1.0) / np.float32(i + 1))
        acc = np.cumsum((p * v[: i + 1]).astype(np.float32), axis=0, dtype=np.float32)[-1]
        assert np.array_equal(got[i], oracle.round_bf16(acc)), i
    # Query 0 sees only key 0: its context is v[0] exactly.
    assert np.array_equal(got[0], v[0])


def test_attention_fully_masked_query_is_zero(oracle):
    # root.zig:1068-1101: a query with no allowed key has zero context.
    rng = np.random.default_rng(22)
    q, k, v = (rng.standard_normal((3, 4)).astype(np.float32) for _ in range(3))
    mask = np.array([[0, 0, 0], [1, 1, 0], [1, 1, 1]], np.uint8)
    for bf in (False, True):
        got = oracle.attention_core(q, k, v, mask, 1, 1, 4, bf16=bf)
        assert np.all(got[0] == 0)
        assert np.all(np.isfinite(got))


def test_attention_bf16_against_f64(oracle):
    rng = np.random.default_rng(23)
    t, hq, hkv, hd = 64, 2, 1, 64
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((t, hq * hd)).astype(np.float32))
    k = rb(rng.standard_normal((t, hkv * hd)).astype(np.float32))
    v = rb(rng.standard_normal((t, hkv * hd)).astype(np.float32))
    mask = oracle.causal_mask(t)
    got = oracle.attention_core(q, k, v, mask, hq, hkv, hd, bf16=True)
    want = _attention_f64(q, k, v, mask, hq, hkv, hd)
    # bf16 scores (|s| <~ 4: a step is <= 2^-6 absolute), bf16 probabilities
    # and a bf16 context: a few percent of max |v| at most.
    assert np.max(np.abs(got - want)) <= 0.05 * np.max(np.abs(v))


def test_block_diagonal_mask_reference_case(oracle):
    # src/ncm_mask.zig:46-64
    m = oracle.block_diagonal_mask(2, [1, 2], [0, 1]).astype(bool)
    assert m[0, 0] and not m[0, 1] and not m[0, 2]
    assert m[2, 0] and not m[2, 1] and m[2, 2] and not m[2, 3]
    assert m[3, 3] and m[3, 4] and m[4, 3]
    with pytest.raises(ValueError):
        oracle.block_diagonal_mask(2, [1], [0])


@pytest.mark.parametrize("prefix,levels,pad", [(0, [5], None), (3, [1, 2], [0, 1, 0]),
                                               (70, [64, 1, 100], "rand"), (5, [], None),
                                               (130, [8, 8, 8, 8, 8, 8, 8, 8], "rand")])
def test_block_diagonal_segments_expand_to_the_mask(ncm, oracle, prefix, levels, pad):
    from ncmorph_amd import kernels

    if pad == "rand":
        pad = (np.random.default_rng(prefix).random(prefix) < 0.3).astype(np.uint8)
    lo, hi, bits = kernels.block_diagonal_segments(prefix, levels, pad)
    seq = lo.size
    q, k = np.meshgrid(np.arange(seq), np.arange(seq), indexing="ij")
    padded = np.array([(int(bits[i // 64]) >> (i % 64)) & 1 for i in range(prefix)], bool)
    prefix_ok = (k < prefix) & ~padded[np.minimum(k, max(prefix - 1, 0))] if prefix else k < 0
    mine = prefix_ok | ((k >= lo[q]) & (k < hi[q]))
    want = oracle.block_diagonal_mask(prefix, levels, pad).astype(bool)
    assert np.array_equal(mine, want)


def test_block_diagonal_segments_errors(ncm):
    import ctypes as C

    L = ncm.lib()
    lv = np.array([2, 3], np.int64)
    lo = np.zeros(8, np.int32)
    hi = np.zeros(8, np.int32)
    pad = np.zeros(2, np.uint8)
    p = lambda a: C.c_void_p(a.ctypes.data)
    # pad mask of the wrong length (InvalidPrefixMask), wrong total (InvalidMaskSize)
    assert L.ncm_block_diagonal_segments(3, p(lv), 2, p(pad), 2, 8, p(lo), p(hi), None) == -3
    assert L.ncm_block_diagonal_segments(3, p(lv), 2, None, 0, 7, p(lo), p(hi), None) == -3
    assert L.ncm_block_diagonal_segments(3, p(lv), 2, None, 0, 8, p(lo), p(hi), None) == 0
