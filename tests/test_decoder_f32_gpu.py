"""The decoder prefill forward in the reference's f32 mode on the GPU
(ncm_decoder_forward_f32_dev) against the oracle's f32-mode composition
(pinned by the reference's tiny-decoder KAT, src/decoder.zig:292-364, and an
f64 forward), its per-stage trace, and the f32 modes of the row ops.

Bars: RMSNorm f32 mode bit-identical to the oracle; SiLU·up f32 mode within
two fp32 ulps (device expf against libm). The forward: the projections sum
on the fp32 MFMA in its own order (the reference in increasing k), so every
logit and traced stage agrees with the oracle within 1e-4 of the stage's
largest magnitude after two layers; the attention context of the KAT's
shape (zero scores) equals the reference's averages within 1e-6."""
import numpy as np
import pytest

from .decoder_f64 import random_model

pytestmark = pytest.mark.gpu


def _dev(a, cuda):
    import torch

    return None if a is None else torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(cuda)


def _f32_weights(decoder, cuda, embed, layers, fnorm, lm_head=None):
    dl = []
    for L in layers:
        inter = L["gate_up_weight"].shape[0] // 2
        gb = L.get("gate_up_bias")
        dl.append({"input_norm": _dev(L["input_norm"], cuda),
                   "qkv_weight": _dev(L["qkv_weight"], cuda),
                   "qkv_bias": _dev(L.get("qkv_bias"), cuda),
                   "o_weight": _dev(L["o_weight"], cuda), "o_bias": _dev(L.get("o_bias"), cuda),
                   "post_attention_norm": _dev(L["post_attention_norm"], cuda),
                   "gate_weight": _dev(L["gate_up_weight"][:inter], cuda),
                   "gate_bias": None if gb is None else _dev(gb[:inter], cuda),
                   "up_weight": _dev(L["gate_up_weight"][inter:], cuda),
                   "up_bias": None if gb is None else _dev(gb[inter:], cuda),
                   "down_weight": _dev(L["down_weight"], cuda),
                   "down_bias": _dev(L.get("down_bias"), cuda),
                   "q_norm": _dev(L.get("q_norm"), cuda), "k_norm": _dev(L.get("k_norm"), cuda)})
    return decoder.DecoderWeights(embed=_dev(embed, cuda), final_norm=_dev(fnorm, cuda),
                                  layers=dl, lm_head=_dev(lm_head, cuda))


def test_row_ops_f32_mode(ncm, oracle, cuda):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(31)
    for rows, width in ((5, 11), (3, 2048), (2, 16384)):
        x = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
        w = (rng.standard_normal(width) * 0.1 + 1).astype(np.float32)
        y = kernels.rms_norm_rows(_dev(x, cuda), _dev(w, cuda), 1e-5, out_mode="f32").cpu()
        ref = oracle.rms_norm(x, w, 1e-5, bf16=False)
        assert np.array_equal(y.numpy().view(np.uint32), ref.view(np.uint32)), width
    g = (rng.standard_normal(4099) * 4).astype(np.float32)
    u = rng.standard_normal(4099).astype(np.float32)
    y = kernels.silu_mul(_dev(g, cuda), _dev(u, cuda), out_mode="f32").cpu().numpy()
    ref = (oracle.silu(g) * u).astype(np.float32)
    ulp = np.abs(y.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2


@pytest.mark.parametrize("hd,window,biases,qk_norm,batch", [(32, 0, False, False, 2),
                                                           (64, 0, True, True, 1),
                                                           (128, 9, False, False, 2)])
def test_decoder_f32_matches_oracle(ncm, oracle, cuda, hd, window, biases, qk_norm, batch):
    import torch
    from ncmorph_amd import decoder

    print(f"f32 decoder case hd={hd} window={window} biases={biases} qk_norm={qk_norm}",
          flush=True)
    rng = np.random.default_rng(hd + window)
    hidden, inter, vocab, hq, hkv, nl, t = 128, 256, 200, 4, 2, 2, 37
    embed, layers, fnorm = random_model(rng, lambda a: np.asarray(a, np.float32), hidden, inter,
                                        vocab, hq, hkv, hd, nl, biases=biases, qk_norm=qk_norm)
    spec = decoder.DecoderSpec(hidden=hidden, intermediate=inter, vocab=vocab, q_heads=hq,
                               kv_heads=hkv, head_dim=hd, layers=nl, window=window,
                               rope_theta=10000.0)
    cos, sin = oracle.rope_tables(oracle.rope_default_frequencies(hd, 10000.0), t)
    w = _f32_weights(decoder, cuda, embed, layers, fnorm)
    ids = rng.integers(0, vocab, (batch, t))
    logits, tr = decoder.forward_f32(spec, w, ids, _dev(cos, cuda), _dev(sin, cuda), trace=True)
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(batch, t, vocab)
    for b in range(batch):
        trace = {}
        ref = oracle.decoder_forward(ids[b], embed, layers, fnorm, None, cos, sin, hq, hkv, hd,
                                     1e-5, window=window, bf16=False, trace=trace)
        scale = np.max(np.abs(ref))
        assert np.max(np.abs(got[b] - ref)) <= 1e-4 * scale, b
        rows = slice(b * t, (b + 1) * t)
        assert np.max(np.abs(tr["block_input"][rows].cpu().numpy() - trace["block_input"])) == 0
        for key in decoder.TRACE_FIELDS[1:]:
            g = tr[key][:, rows].cpu().numpy()
            r = trace[key]
            assert g.shape == r.shape, key
            assert np.max(np.abs(g - r)) <= 1e-4 * max(np.max(np.abs(r)), 1e-30), key


def test_decoder_f32_tiny_kat_shape(ncm, oracle, cuda):
    """The reference's tiny-decoder KAT (src/decoder.zig:292-364) at the
    device's smallest widths (hidden 4, one head of 4, intermediate 4,
    vocab 4): zero q / k weights make every score 0, so token 0's context is
    its normalized input and token 1's the mean of both; identity v and o,
    zero MLP, tied embeddings."""
    import torch
    from ncmorph_amd import decoder

    embed = np.arange(1, 17, dtype=np.float32).reshape(4, 4) * np.float32(0.1)
    layer = dict(input_norm=np.ones(4, np.float32),
                 qkv_weight=np.concatenate([np.zeros((8, 4), np.float32),
                                            np.eye(4, dtype=np.float32)]),
                 qkv_bias=None, o_weight=np.eye(4, dtype=np.float32), o_bias=None,
                 post_attention_norm=np.ones(4, np.float32),
                 gate_up_weight=np.zeros((8, 4), np.float32), gate_up_bias=None,
                 down_weight=np.zeros((4, 4), np.float32), down_bias=None)
    spec = decoder.DecoderSpec(hidden=4, intermediate=4, vocab=4, q_heads=1, kv_heads=1,
                               head_dim=4, layers=1, rope_theta=10000.0,
                               tie_word_embeddings=True)
    cos, sin = oracle.rope_tables(oracle.rope_default_frequencies(4, 10000.0), 2)
    w = _f32_weights(decoder, cuda, embed, [layer], np.ones(4, np.float32))
    logits, tr = decoder.forward_f32(spec, w, np.array([[1, 3]]), _dev(cos, cuda),
                                     _dev(sin, cuda), trace=True)
    torch.cuda.synchronize()
    n = tr["input_norm"][0].cpu().numpy()
    ctx = tr["attention_context"][0].cpu().numpy()
    assert np.all(np.isfinite(logits.cpu().numpy()))
    assert np.max(np.abs(ctx[0] - n[0])) <= 1e-6
    assert np.max(np.abs(ctx[1] - (n[0] + n[1]) * 0.5)) <= 1e-6
    ref = oracle.decoder_forward([1, 3], embed, [layer], np.ones(4, np.float32), None, cos, sin,
                                 1, 1, 4, 1e-5, bf16=False)
    assert np.max(np.abs(logits.cpu().numpy() - ref)) <= 1e-6 * np.max(np.abs(ref))
