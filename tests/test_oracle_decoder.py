"""Pins of the oracle's bf16 decoder composition (src/decoder.zig:62-228)
against an independent f64 forward of the published architecture, and of
the host-built RoPE tables against the oracle's."""
import ctypes as C

import numpy as np
import pytest

from .decoder_f64 import forward_f64, random_model


@pytest.mark.parametrize("biases,window,qk_norm", [(False, 0, False), (True, 0, False),
                                                   (False, 9, False), (False, 0, True)])
def test_oracle_decoder_against_f64(oracle, biases, window, qk_norm):
    rng = np.random.default_rng(5 + window + biases)
    hidden, inter, vocab, hq, hkv, hd, nl, t = 256, 512, 300, 4, 2, 64, 2, 48
    embed, layers, fnorm = random_model(rng, oracle.round_bf16, hidden, inter, vocab, hq, hkv,
                                        hd, nl, biases=biases, qk_norm=qk_norm)
    cos, sin = oracle.rope_tables(oracle.rope_llama3(hd, 500000.0, 32.0, 1.0, 4.0, 8192), t)
    ids = rng.integers(0, vocab, t)
    got = oracle.decoder_forward(ids, embed, layers, fnorm, None, cos, sin, hq, hkv, hd, 1e-5,
                                 window=window)
    args = (ids, embed, layers, fnorm, None, cos, sin, hq, hkv, hd, 1e-5, window)
    ref = forward_f64(*args)
    scale = np.max(np.abs(ref))
    # bf16 roundings throughout two layers: a few parts in a thousand.
    assert np.max(np.abs(got - ref)) <= 0.02 * scale
    # The bound separates the right composition from plausible wrong ones.
    for mistake in ("rope", "residual") + (("qk_norm",) if qk_norm else ()):
        assert np.max(np.abs(forward_f64(*args, skip=mistake) - ref)) > 0.05 * scale


def test_oracle_decoder_untied_head_and_zero_layers(oracle):
    rng = np.random.default_rng(8)
    hidden, vocab, t = 128, 50, 10
    embed = oracle.round_bf16(rng.standard_normal((vocab, hidden)).astype(np.float32) * 0.2)
    head = oracle.round_bf16(rng.standard_normal((vocab, hidden)).astype(np.float32) * 0.2)
    fnorm = np.ones(hidden, np.float32)
    ids = rng.integers(0, vocab, t)
    cos, sin = np.ones((t, 64), np.float32), np.zeros((t, 64), np.float32)
    got = oracle.decoder_forward(ids, embed, [], fnorm, head, cos, sin, 1, 1, 64, 1e-5)
    # No layers: logits = round(rms_norm_bf16(embedding rows) . head), exactly.
    want = oracle.matmul_bf16(oracle.rms_norm(embed[ids], fnorm, 1e-5, bf16=True), head)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("theta,llama3,hd", [(500000.0, (32.0, 1.0, 4.0, 8192), 64),
                                             (10000.0, None, 128)])
def test_host_rope_tables_match_oracle(oracle, theta, llama3, hd):
    from ncmorph_amd import decoder

    spec = decoder.DecoderSpec(hidden=256, intermediate=512, vocab=10, q_heads=2, kv_heads=1,
                               head_dim=hd, layers=1, rope_theta=theta, rope_llama3=llama3)
    cos, sin = decoder.rope_tables(spec, 300)
    inv = (oracle.rope_llama3(hd, theta, *llama3) if llama3
           else oracle.rope_default_frequencies(hd, theta))
    c2, s2 = oracle.rope_tables(inv, 300)
    assert np.array_equal(cos.view(np.uint32), c2.view(np.uint32))
    assert np.array_equal(sin.view(np.uint32), s2.view(np.uint32))


def test_decoder_struct_layout(ncm):
    from ncmorph_amd import decoder

    # int64 x 3, int32 x 4, int64, float (+4 padding); ten pointers.
    assert C.sizeof(decoder._Shape) == 56
    assert decoder._Shape.window.offset == 40 and decoder._Shape.rms_eps.offset == 48
    # ten weight pointers, then q_norm, k_norm and the two norm biases
    assert C.sizeof(decoder._Layer) == 112


def test_decoder_entry_rejects_before_device_use(ncm):
    L = ncm.lib()
    assert L.ncm_decoder_forward_dev(None, None, None, None, None, None, None, None, None, 1, 1,
                                     None, None) == -1


def test_tiny_decoder_kat(oracle):
    """src/decoder.zig:292-364, f32 mode: vocab 4, hidden 2, intermediate 3,
    one layer with one head of width 2, zero q / k / MLP weights, identity v
    and o, tied embeddings [0.1 .. 0.8], tokens [1, 3]. With zero scores the
    first token attends to itself and the second averages both, so the
    context equals the normalized inputs (token 0) and their mean (token 1);
    every logit is finite."""
    embed = np.array([0.1, 0.2, 0.3, 0.4, 0.5, 0.6, 0.7, 0.8], np.float32).reshape(4, 2)
    layer = dict(input_norm=np.ones(2, np.float32),
                 qkv_weight=np.array([0, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 1],
                                     np.float32).reshape(6, 2),
                 qkv_bias=None, o_weight=np.eye(2, dtype=np.float32), o_bias=None,
                 post_attention_norm=np.ones(2, np.float32),
                 gate_up_weight=np.zeros((6, 2), np.float32), gate_up_bias=None,
                 down_weight=np.zeros((2, 3), np.float32), down_bias=None)
    inv = oracle.rope_default_frequencies(2, 10000.0)
    cos, sin = oracle.rope_tables(inv, 2)
    trace = {}
    logits = oracle.decoder_forward([1, 3], embed, [layer], np.ones(2, np.float32), None, cos,
                                    sin, 1, 1, 2, 1e-5, bf16=False, trace=trace)
    assert logits.shape == (2, 4) and np.all(np.isfinite(logits))
    n, ctx = trace["input_norm"][0], trace["attention_context"][0]
    assert abs(n[0, 0] - ctx[0, 0]) <= 1e-6 and abs(n[0, 1] - ctx[0, 1]) <= 1e-6
    assert abs((n[0, 0] + n[1, 0]) * 0.5 - ctx[1, 0]) <= 1e-6
    assert abs((n[0, 1] + n[1, 1]) * 0.5 - ctx[1, 1]) <= 1e-6
    # The trace's own identities: block input = embedding rows, residuals.
    assert np.array_equal(trace["block_input"], embed[[1, 3]])
    assert np.array_equal(trace["attention_residual"][0],
                          trace["block_input"] + trace["attention_output"][0])
    assert np.array_equal(trace["block_output"][0], trace["attention_residual"][0])


@pytest.mark.parametrize("biases,qk_norm", [(False, False), (True, True)])
def test_oracle_decoder_f32_mode_against_f64(oracle, biases, qk_norm):
    """The f32 mode (no bf16 roundings, kernels.matmul, f32 attention and
    SiLU) within 1e-4 of max|logit| of the f64 forward on f32 weights; the
    bound separates a missing rotation, residual or QK-norm."""
    rng = np.random.default_rng(21 + biases)
    hidden, inter, vocab, hq, hkv, hd, nl, t = 128, 256, 200, 4, 2, 32, 2, 40
    embed, layers, fnorm = random_model(rng, lambda a: np.asarray(a, np.float32), hidden, inter,
                                        vocab, hq, hkv, hd, nl, biases=biases, qk_norm=qk_norm)
    cos, sin = oracle.rope_tables(oracle.rope_default_frequencies(hd, 10000.0), t)
    ids = rng.integers(0, vocab, t)
    got = oracle.decoder_forward(ids, embed, layers, fnorm, None, cos, sin, hq, hkv, hd, 1e-5,
                                 bf16=False)
    args = (ids, embed, layers, fnorm, None, cos, sin, hq, hkv, hd, 1e-5, 0)
    ref = forward_f64(*args)
    scale = np.max(np.abs(ref))
    assert np.max(np.abs(got - ref)) <= 1e-4 * scale
    for mistake in ("rope", "residual") + (("qk_norm",) if qk_norm else ()):
        assert np.max(np.abs(forward_f64(*args, skip=mistake) - ref)) > 1e-2 * scale
