"""Pins of the VQ-VAE tokenizer oracle (oracle/vq_tokenizer.py).

Each primitive is checked against the PyTorch routine the upstream model
calls (research/reference/vq_forward_semantics.md:80-82, :46, :121; the
decoder at :84-94), run on the CPU in float64; the quantizer loop against
brute force, its telescoping identity and the closed form of the cascade's
identity initialisation (vq_forward_semantics.md:132-135); the WMT14 key
table against the counts of research/converter/wmt14_tokenizer_keys.md
section 6.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import vq_tokenizer as vt

RNG = np.random.default_rng(7)


def _t(x):
    """[B, L, C] numpy -> [B, C, L] float64 torch (the PyTorch modules' layout)."""
    return torch.from_numpy(np.ascontiguousarray(np.asarray(x, np.float64))).transpose(1, 2)


def _n(t):
    return t.transpose(1, 2).numpy()


@pytest.mark.parametrize("length,groups", [(64, 8), (16, 8), (1, 8), (4, 2)])
def test_group_norm_matches_torch(length, groups):
    x = RNG.standard_normal((3, length, 48)) * 3 + 1
    got = vt.group_norm(x, groups, 1e-5)
    want = _n(F.group_norm(_t(x), groups, eps=1e-5))
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n", [1, 4, 8, 14, 20, 26, 32, 40, 48, 56, 64, 3, 7, 25])
def test_area_pool_matches_torch(n):
    x = RNG.standard_normal((2, 64, 8))
    got = vt.area_pool(x, n)
    want = _n(F.interpolate(_t(x), size=n, mode="area"))
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_area_pool_uneven_owt_lengths():
    # (k+1)^2 levels of a 1024-position sequence: windows overlap when the
    # level does not divide 1024.
    x = RNG.standard_normal((1, 1024, 4))
    for n in (9, 25, 49, 100, 961):
        np.testing.assert_allclose(vt.area_pool(x, n),
                                   _n(F.interpolate(_t(x), size=n, mode="area")),
                                   rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("n", [1, 4, 8, 14, 20, 26, 32, 40, 48, 56, 64, 3, 9])
def test_linear_up_matches_torch(n):
    x = RNG.standard_normal((2, n, 8))
    got = vt.linear_up(x, 64)
    want = _n(F.interpolate(_t(x), size=64, mode="linear"))
    np.testing.assert_allclose(got, want, rtol=1e-13, atol=1e-13)


def test_linear_up_endpoints_and_constant():
    # Constant input stays constant; the first and last outputs clamp to the
    # first and last inputs (align_corners=False).
    x = np.ones((1, 14, 3)) * 2.5
    np.testing.assert_array_equal(vt.linear_up(x, 64), np.full((1, 64, 3), 2.5))
    y = RNG.standard_normal((1, 14, 3))
    up = vt.linear_up(y, 64)
    np.testing.assert_allclose(up[:, 0], y[:, 0])
    np.testing.assert_allclose(up[:, -1], y[:, -1])


@pytest.mark.parametrize("s", [4, 2])
def test_stages_match_torch_convs(s):
    c = 12
    x = RNG.standard_normal((2, 16, c))
    w = RNG.standard_normal((c, c, s))
    b = RNG.standard_normal(c)
    want = _n(F.conv1d(_t(x), torch.from_numpy(w), torch.from_numpy(b), stride=s))
    np.testing.assert_allclose(vt.down_stage(x, w, b, s), want, rtol=1e-12, atol=1e-12)
    want = _n(F.conv_transpose1d(_t(x), torch.from_numpy(w), torch.from_numpy(b), stride=s))
    np.testing.assert_allclose(vt.up_stage(x, w, b, s), want, rtol=1e-12, atol=1e-12)


def test_phi_matches_torch_conv():
    c = 16
    h = RNG.standard_normal((2, 20, c))
    w = RNG.standard_normal((c, c, 3))
    b = RNG.standard_normal(c)
    conv = _n(F.conv1d(_t(h), torch.from_numpy(w), torch.from_numpy(b), padding=1))
    np.testing.assert_allclose(vt.phi(h, w, b, 0.5), 0.5 * h + 0.5 * conv, rtol=1e-12, atol=1e-12)
    # ratio 0 is the identity, ratio 1 the bare conv
    np.testing.assert_allclose(vt.phi(h, w, b, 0.0), h)
    np.testing.assert_allclose(vt.phi(h, w, b, 1.0), conv, rtol=1e-12, atol=1e-12)


def test_cascade_strides():
    assert vt.cascade_strides(64, 4) == [4, 4, 4]
    assert vt.cascade_strides(1024, 4) == [4] * 5
    assert vt.cascade_strides(1, 4) == []
    assert vt.WMT14.cascade_strides() == [4, 4, 4]
    with pytest.raises(ValueError):
        vt.cascade_strides(48, 4)


def _identity_cascade(cfg, d):
    strides = cfg.cascade_strides()
    eye = np.eye(d)
    return vt.QuantizerWeights(
        codebooks=[],
        down_weight=[np.repeat(eye[:, :, None], s, axis=2) / s for s in strides],
        down_bias=[np.zeros(d) for _ in strides],
        up_weight=[np.repeat(eye[:, :, None], s, axis=2) for s in strides],
        up_bias=[np.zeros(d) for _ in strides])


def test_cascade_identity_init_is_mean_and_repeat():
    # vq_forward_semantics.md:132-135: with identity/s weights, zero biases and
    # no norms the down cascade is the mean over all positions and the up
    # cascade repeats its input (nearest neighbour).
    cfg = vt.TokenizerConfig(embed_dim=8, levels=(1, 64), vocab_sizes=(4, 4),
                             cascade_norm=False, cascade_norm_final=False)
    w = _identity_cascade(cfg, 8)
    r = RNG.standard_normal((3, 64, 8))
    np.testing.assert_allclose(vt.cascade_down(cfg, w, r), r.mean(axis=1, keepdims=True),
                               rtol=1e-12, atol=1e-12)
    q = RNG.standard_normal((3, 1, 8))
    np.testing.assert_allclose(vt.cascade_up(cfg, w, q), np.repeat(q, 64, axis=1))


def test_cascade_norms_match_torch_modules():
    # The WMT14 arrangement (keys doc section 4): down = conv, GN, conv, GN,
    # conv, GN; up = convT, GN, convT, GN, convT; GroupNorm(8, D, affine=False).
    d = 16
    cfg = vt.TokenizerConfig(embed_dim=d, levels=(1, 64), vocab_sizes=(4, 4))
    enc, qw, _ = vt.random_weights(cfg, seed=3, vocab_cap=8)
    r = RNG.standard_normal((2, 64, d))
    x = _t(r)
    for i, s in enumerate(cfg.cascade_strides()):
        x = F.conv1d(x, torch.from_numpy(qw.down_weight[i].astype(np.float64)),
                     torch.from_numpy(qw.down_bias[i].astype(np.float64)), stride=s)
        x = F.group_norm(x, 8, eps=1e-5)
    np.testing.assert_allclose(vt.cascade_down(cfg, qw, r), _n(x), rtol=1e-10, atol=1e-10)
    q = RNG.standard_normal((2, 1, d))
    x = _t(q)
    for i, s in enumerate(cfg.cascade_strides()):
        x = F.conv_transpose1d(x, torch.from_numpy(qw.up_weight[i].astype(np.float64)),
                               torch.from_numpy(qw.up_bias[i].astype(np.float64)), stride=s)
        if i < 2:
            x = F.group_norm(x, 8, eps=1e-5)
    np.testing.assert_allclose(vt.cascade_up(cfg, qw, q), _n(x), rtol=1e-10, atol=1e-10)


def _small_cfg(**kw):
    base = dict(embed_dim=32, in_vocab=50, context_length=16, levels=(1, 2, 5, 8, 16),
                vocab_sizes=(16, 32, 24, 16, 40), groups=4, cascade_base=4)
    base.update(kw)
    return vt.TokenizerConfig(**base)


def test_quantize_codes_are_brute_force_argmins_and_telescope():
    cfg = _small_cfg()
    enc, qw, _ = vt.random_weights(cfg, seed=11)
    ids = RNG.integers(0, cfg.in_vocab, size=(3, cfg.seq_len))
    z = vt.encode_front(cfg, ids, enc["wte"], enc["wpe"])
    out = vt.quantize(cfg, qw, z)
    # zhat + r telescopes back to z
    np.testing.assert_allclose(out["zhat"] + out["r"], z, rtol=1e-12, atol=1e-12)
    # each level's code is the nearest by brute force over the residual
    # entering it, recomputed here from the previous levels' codes
    r = z.copy()
    off = 0
    for level, n in enumerate(cfg.levels):
        u = vt._down(cfg, qw, level, r)
        e = qw.codebooks[level].astype(np.float64)
        for bi in range(3):
            for j in range(n):
                dd = [np.sum((u[bi, j] - e[k]) ** 2) for k in range(e.shape[0])]
                assert out["codes"][bi, off + j] == int(np.argmin(dd))
        idx = out["codes"][:, off:off + n]
        r = r - vt._resi(cfg, qw, level, vt._up(cfg, qw, level, e[idx]))
        off += n
    np.testing.assert_allclose(r, out["r"], rtol=1e-12, atol=1e-12)
    # reconstruct from the codes gives the same zhat
    np.testing.assert_allclose(vt.reconstruct(cfg, qw, out["codes"]), out["zhat"],
                               rtol=1e-12, atol=1e-12)
    assert all((du == db).all() for du, db in zip(out["d_used"], out["d_best"]))


def test_quantize_planted_single_level_code():
    # One level of full length, no Phi: z equal to a codebook row per position
    # quantizes to exactly that row with a zero residual.
    cfg = _small_cfg(levels=(16,), vocab_sizes=(40,), learned_level0=False, quant_resi=False)
    _, qw, _ = vt.random_weights(cfg, seed=2)
    want = RNG.integers(0, 40, size=(2, 16))
    z = qw.codebooks[0].astype(np.float64)[want]
    out = vt.quantize(cfg, qw, z)
    np.testing.assert_array_equal(out["codes"], want)
    np.testing.assert_array_equal(out["r"], np.zeros_like(z))


def test_quantize_forced_codes_report_distance_gaps():
    cfg = _small_cfg()
    enc, qw, _ = vt.random_weights(cfg, seed=5)
    z = vt.encode_front(cfg, RNG.integers(0, 50, size=(2, 16)), enc["wte"], enc["wpe"])
    best = vt.quantize(cfg, qw, z)
    forced = best["codes"].copy()
    forced[:, 3] = (forced[:, 3] + 1) % cfg.vocab_sizes[2]     # a wrong level-2 code
    out = vt.quantize(cfg, qw, z, forced=forced)
    np.testing.assert_array_equal(out["codes"], forced)
    assert (out["d_used"][2][:, 0] > out["d_best"][2][:, 0]).all()
    np.testing.assert_array_equal(out["d_used"][1], out["d_best"][1])


def test_encode_front_matches_torch():
    cfg = _small_cfg()
    enc, _, _ = vt.random_weights(cfg, seed=9)
    ids = RNG.integers(0, cfg.in_vocab, size=(2, 16))
    x = F.embedding(torch.from_numpy(ids), torch.from_numpy(enc["wte"].astype(np.float64)))
    x = x + torch.from_numpy(enc["wpe"].astype(np.float64))[:16]
    want = F.group_norm(x.transpose(1, 2), cfg.groups, eps=1e-5).transpose(1, 2).numpy()
    np.testing.assert_allclose(vt.encode_front(cfg, ids, enc["wte"], enc["wpe"]), want,
                               rtol=1e-12, atol=1e-12)


def test_decoder_forward_matches_torch_functional():
    cfg = _small_cfg(embed_dim=48, n_head=3)
    _, _, dw = vt.random_weights(cfg, seed=4)
    dw = {k: torch.from_numpy(v.astype(np.float64)) for k, v in dw.items()}
    x = torch.from_numpy(RNG.standard_normal((2, 16, 48)))
    p = "middle_block."
    h = F.layer_norm(x, (48,), dw[p + "ln_1.weight"], dw[p + "ln_1.bias"], 1e-6)
    qkv = F.linear(h, dw[p + "attn.c_attn.weight"], dw[p + "attn.c_attn.bias"])
    q, k, v = qkv.split(48, dim=-1)
    q, k, v = (t.view(2, 16, 3, 16).transpose(1, 2) for t in (q, k, v))
    q = F.rms_norm(q, (16,), dw[p + "attn.q_norm.weight"], 1e-6)
    k = F.rms_norm(k, (16,), dw[p + "attn.k_norm.weight"], 1e-6)
    a = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(2, 16, 48)
    x1 = x + F.linear(a, dw[p + "attn.c_proj.weight"], dw[p + "attn.c_proj.bias"])
    h = F.layer_norm(x1, (48,), dw[p + "ln_2.weight"], dw[p + "ln_2.bias"], 1e-6)
    h = F.gelu(F.linear(h, dw[p + "mlp.c_fc.weight"], dw[p + "mlp.c_fc.bias"]))
    x2 = x1 + F.linear(h, dw[p + "mlp.c_proj.weight"], dw[p + "mlp.c_proj.bias"])
    want = F.linear(F.layer_norm(x2, (48,), dw["ln_f.weight"], None, 1e-6),
                    dw["output_layer.weight"]).numpy()
    got = vt.decoder_forward(cfg, {k: v.numpy() for k, v in dw.items()}, x.numpy())
    np.testing.assert_allclose(got, want, rtol=1e-10, atol=1e-10)


def test_gelu_is_exact_erf_form():
    x = np.linspace(-6, 6, 97)
    want = F.gelu(torch.from_numpy(x)).numpy()
    np.testing.assert_allclose(vt.gelu(x), want, rtol=1e-14, atol=1e-15)
    assert vt.gelu(np.array([0.0]))[0] == 0.0
    assert math.isclose(vt.gelu(np.array([1.0]))[0], 0.8413447460685429, rel_tol=1e-14)
