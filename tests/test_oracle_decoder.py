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
                                     None) == -1
