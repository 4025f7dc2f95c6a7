"""GPU parity of the decoder's RoPE rotation and causal bf16 attention
against the oracle (restatement of packages/kernels/root.zig:536-578,
615-634).

RoPE: bit-identical (every operand and result is a bf16 rounding of one fp32
operation, done in the reference's order).

Attention: q . k and P V are sums of exact fp32 products that the MFMA adds
in its own order (the reference adds in key order), and the softmax sum is
accumulated online. A score that sits at a bf16 rounding boundary can then
round one step the other way, which moves its probability by up to
|s| 2^-8 relative. The test holds the device context to
|dev - ref| <= 2^-7 |ref| + 2^-7 max|v| elementwise, asks >= 99% of the
elements bit-identical to the oracle, and holds both to the same f64 bound.
"""
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bf16_dev(a, cuda):
    import torch

    from ncmorph_amd import synth

    bits = synth.bf16_bits(np.ascontiguousarray(a, np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).to(cuda).view(torch.bfloat16)


def _f32_of(t):
    import torch

    return (t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16).astype(np.uint32)
            << 16).view(np.float32)


def _tables(oracle, positions, hd):
    inv = oracle.rope_llama3(hd, 500000.0, 32.0, 1.0, 4.0, 8192)
    return oracle.rope_tables(inv, positions)


@pytest.mark.parametrize("batch,seq,hq,hkv,hd", [(2, 1024, 32, 8, 64), (1, 37, 2, 1, 128),
                                                 (1, 19, 3, 1, 12)])
def test_rope_rotate_bit_identical(ncm, oracle, cuda, batch, seq, hq, hkv, hd):
    """Four pairs per thread when hd % 8 == 0 (64, 128), one otherwise (12)."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(seq + hd)
    cos, sin = _tables(oracle, seq, hd)
    width = (hq + 2 * hkv) * hd  # one q|k|v row, as the fused projection writes it
    qkv = oracle.round_bf16(rng.standard_normal((batch * seq, width)).astype(np.float32) * 2)
    dev = _bf16_dev(qkv, cuda)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    kernels.rope_rotate(dev[:, :hq * hd], hq, hd, seq, cd, sd)
    kernels.rope_rotate(dev[:, hq * hd:(hq + hkv) * hd], hkv, hd, seq, cd, sd)
    torch.cuda.synchronize()
    got = _f32_of(dev)
    pos = np.arange(batch * seq) % seq
    want = qkv.copy()
    want[:, :hq * hd] = oracle.rotate_heads(qkv[:, :hq * hd], cos[pos], sin[pos], hq, hd)
    want[:, hq * hd:(hq + hkv) * hd] = oracle.rotate_heads(
        qkv[:, hq * hd:(hq + hkv) * hd], cos[pos], sin[pos], hkv, hd)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _attention_f64(q, k, v, mask, hq, hkv, hd):
    t = q.shape[0]
    out = np.zeros((t, hq * hd))
    g = hq // hkv
    for h in range(hq):
        kv = h // g
        s = (q[:, h * hd:(h + 1) * hd].astype(np.float64)
             @ k[:, kv * hd:(kv + 1) * hd].astype(np.float64).T) / math.sqrt(hd)
        s = np.where(mask.astype(bool), s, -np.inf)
        e = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h * hd:(h + 1) * hd] = (e / e.sum(axis=1, keepdims=True)) @ v[:, kv * hd:(kv + 1) * hd]
    return out


def _check(got, ref, v, f64=None):
    vmax = float(np.max(np.abs(v)))
    bound = 2.0**-7 * np.abs(ref) + 2.0**-7 * vmax
    assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref)))
    same = np.mean(got.view(np.uint32) == ref.view(np.uint32))
    assert same >= 0.99, same
    if f64 is not None:
        assert np.max(np.abs(got - f64)) <= 0.05 * vmax
        assert np.max(np.abs(ref - f64)) <= 0.05 * vmax


@pytest.mark.parametrize("batch,seq,hq,hkv,hd,window", [
    (2, 200, 4, 2, 64, 0),     # ragged query and key blocks, GQA
    (1, 300, 2, 2, 128, 0),    # head_dim 128
    (2, 257, 4, 1, 64, 37),    # sliding window inside a key block
    (1, 130, 2, 1, 64, 64),    # window equal to the key block
    (1, 1, 1, 1, 64, 0),       # one token: context = v
])
def test_attention_against_oracle(ncm, oracle, cuda, batch, seq, hq, hkv, hd, window):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(seq * 3 + hd + window)
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((batch * seq, hq * hd)).astype(np.float32) * 1.5)
    k = rb(rng.standard_normal((batch * seq, hkv * hd)).astype(np.float32) * 1.5)
    v = rb((rng.standard_normal((batch * seq, hkv * hd))
            + np.repeat(np.arange(hkv), hd)).astype(np.float32))
    out = kernels.attention_bf16(_bf16_dev(q, cuda), _bf16_dev(k, cuda), _bf16_dev(v, cuda),
                                 batch, seq, hq, hkv, hd, window=window)
    out16 = kernels.attention_bf16(_bf16_dev(q, cuda), _bf16_dev(k, cuda), _bf16_dev(v, cuda),
                                   batch, seq, hq, hkv, hd, window=window, out_mode="bf16")
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(_f32_of(out16).view(np.uint32), got.view(np.uint32))
    mask = oracle.causal_mask(seq, window)
    for b in range(batch):
        rows = slice(b * seq, (b + 1) * seq)
        ref = oracle.attention_core(q[rows], k[rows], v[rows], mask, hq, hkv, hd)
        f64 = _attention_f64(q[rows], k[rows], v[rows], mask, hq, hkv, hd)
        _check(got[rows], ref, v[rows], f64)
    if seq == 1:
        assert np.array_equal(got, np.repeat(v, hq // hkv, axis=1))


@pytest.mark.parametrize("seq,hq,hkv,hd", [(64, 4, 2, 64), (128, 4, 1, 128), (100, 2, 2, 128)])
def test_attention_probabilities_bits(ncm, oracle, cuda, seq, hq, hkv, hd):
    """The probabilities themselves against the reference's rounding path,
    p = round_bf16(exp(s - m) / l) (packages/kernels/root.zig:272-284,
    :563-567): with one-hot value rows (v[k] = e_k, seq <= head_dim) every
    context element is one probability times 1 added to zeros, so the
    context holds the p matrix exactly, on the device and in the oracle.
    Bar: at least 99.95% of the allowed (causal) entries bit-identical
    (measured: 99.99-100%; a score whose fp32 sum, in MFMA order, lies next
    to a bf16 boundary rounds the other way, and exp is the device's), the
    masked ones exactly 0, and every entry within 2^-7 |p| + 2^-16."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(seq + hd)
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((seq, hq * hd)).astype(np.float32) * 1.2)
    k = rb(rng.standard_normal((seq, hkv * hd)).astype(np.float32) * 1.2)
    v = np.zeros((seq, hkv * hd), np.float32)
    for h in range(hkv):
        v[np.arange(seq), h * hd + np.arange(seq)] = 1.0
    out = kernels.attention_bf16(_bf16_dev(q, cuda), _bf16_dev(k, cuda), _bf16_dev(v, cuda),
                                 1, seq, hq, hkv, hd)
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(seq, hq, hd)[:, :, :seq]
    ref = oracle.attention_core(q, k, v, oracle.causal_mask(seq, 0), hq, hkv,
                                hd).reshape(seq, hq, hd)[:, :, :seq]
    allowed = np.broadcast_to(oracle.causal_mask(seq, 0).astype(bool)[:, None, :], got.shape)
    assert np.all(got[~allowed] == 0)
    same = float(np.mean(got[allowed].view(np.uint32) == ref[allowed].view(np.uint32)))
    print(f"p bit-identical: {same:.6f} of {int(allowed.sum())}", flush=True)
    assert np.all(np.abs(got - ref) <= 2.0**-7 * np.abs(ref) + 2.0**-16)
    assert same >= 0.9995, same
    # Each query's probabilities sum to 1 within the bf16 roundings.
    assert np.all(np.abs(got.sum(axis=2) - 1.0) <= 2.0**-7 * (1 + np.arange(seq))[:, None])


def test_attention_decoder_shape_fused_qkv(ncm, oracle, cuda):
    """The Llama-3.2-1B prefill shape (4 sequences x 1024 tokens, 32 query /
    8 key-value heads of 64) read from one q|k|v buffer, after the device
    RoPE; heads of the first and last kv group of two sequences checked."""
    import torch
    from ncmorph_amd import kernels

    batch, seq, hq, hkv, hd = 4, 1024, 32, 8, 64
    rng = np.random.default_rng(99)
    width = (hq + 2 * hkv) * hd
    qkv = oracle.round_bf16(rng.standard_normal((batch * seq, width)).astype(np.float32))
    cos, sin = _tables(oracle, seq, hd)
    dev = _bf16_dev(qkv, cuda)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    qd, kd, vd = dev[:, :hq * hd], dev[:, hq * hd:(hq + hkv) * hd], dev[:, (hq + hkv) * hd:]
    kernels.rope_rotate(qd, hq, hd, seq, cd, sd)
    kernels.rope_rotate(kd, hkv, hd, seq, cd, sd)
    out = kernels.attention_bf16(qd, kd, vd, batch, seq, hq, hkv, hd)
    torch.cuda.synchronize()
    rot = _f32_of(dev)
    got = out.cpu().numpy()
    mask = oracle.causal_mask(seq)
    for b in (0, 3):
        rows = slice(b * seq, (b + 1) * seq)
        for kv in (0, hkv - 1):
            qh = slice(kv * 4 * hd, (kv + 1) * 4 * hd)
            q = rot[rows, qh]
            k = rot[rows, hq * hd + kv * hd:hq * hd + (kv + 1) * hd]
            v = rot[rows, (hq + hkv) * hd + kv * hd:(hq + hkv) * hd + (kv + 1) * hd]
            ref = oracle.attention_core(q, k, v, mask, 4, 1, hd)
            _check(got[rows, qh], ref, v)


def test_attention_rejects_bad_shapes(ncm, cuda):
    import torch
    from ncmorph_amd import kernels
    from ncmorph_amd._lib import NcmError

    x = torch.zeros((8, 96), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(NcmError):  # head_dim 96 is not served
        kernels.attention_bf16(x, x, x, 1, 8, 1, 1, 96)
    y = torch.zeros((8, 192), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(NcmError):  # 3 query heads over 2 kv heads
        kernels.attention_bf16(y[:, :192], y[:, :128], y[:, :128], 1, 8, 3, 2, 64)


@pytest.mark.parametrize("batch,prefix,levels,pad,hq,hkv,hd", [
    (1, 2, [1, 2], [0, 1], 1, 1, 64),              # the reference's mask case
    (2, 70, [64, 1, 100], "rand", 4, 2, 64),       # ragged blocks, padded prefix
    (1, 0, [128, 128, 128], None, 2, 1, 128),      # no prefix, aligned levels
    (1, 64, [8] * 8, "all", 2, 2, 64),             # all-padded prefix: zero contexts
    (2, 130, [256, 33], None, 4, 1, 64),
])
def test_attention_level_mask_against_oracle(ncm, oracle, cuda, batch, prefix, levels, pad, hq,
                                             hkv, hd):
    import torch
    from ncmorph_amd import kernels

    if pad == "rand":
        pad = (np.random.default_rng(prefix).random(prefix) < 0.3).astype(np.uint8)
    elif pad == "all":
        pad = np.ones(prefix, np.uint8)
    seq = prefix + sum(levels)
    rng = np.random.default_rng(seq + hd)
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((batch * seq, hq * hd)).astype(np.float32) * 1.5)
    k = rb(rng.standard_normal((batch * seq, hkv * hd)).astype(np.float32) * 1.5)
    v = rb((rng.standard_normal((batch * seq, hkv * hd))
            + np.repeat(np.arange(hkv), hd)).astype(np.float32))
    lo, hi, bits = kernels.block_diagonal_segments(prefix, levels, pad)
    dl, dh = torch.from_numpy(lo).to(cuda), torch.from_numpy(hi).to(cuda)
    db = torch.from_numpy(bits.view(np.int64)).to(cuda) if pad is not None else None
    out = kernels.attention_bf16_seg(_bf16_dev(q, cuda), _bf16_dev(k, cuda), _bf16_dev(v, cuda),
                                     batch, seq, hq, hkv, hd, prefix, dl, dh, db)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    mask = oracle.block_diagonal_mask(prefix, levels, pad)
    for b in range(batch):
        rows = slice(b * seq, (b + 1) * seq)
        ref = oracle.attention_core(q[rows], k[rows], v[rows], mask, hq, hkv, hd)
        _check(got[rows], ref, v[rows])
    if pad is not None and np.all(pad):
        assert np.all(got.reshape(batch, seq, -1)[:, :prefix] == 0)


@pytest.mark.parametrize("prefix,levels,pad", [(16, [8, 16, 32, 48], "rand"),
                                               (4, [4, 8, 16, 32, 64], None)])
def test_attention_level_mask_probabilities_bits(ncm, oracle, cuda, prefix, levels, pad):
    """The NCM level mask (block-diagonal: prefix keys without their pad bit,
    then the query's own level), head_dim 128: with one-hot value rows the
    context is the p matrix; at least 99.95% of the allowed entries
    bit-identical to the oracle's round_bf16(exp(s - m) / l), the others
    within 2^-7 |p| + 2^-16, masked entries exactly 0."""
    import torch
    from ncmorph_amd import kernels

    if pad == "rand":
        pad = (np.random.default_rng(prefix).random(prefix) < 0.3).astype(np.uint8)
    hq, hkv, hd = 4, 1, 128
    seq = prefix + sum(levels)
    assert seq <= hd
    rng = np.random.default_rng(seq)
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((seq, hq * hd)).astype(np.float32) * 1.2)
    k = rb(rng.standard_normal((seq, hkv * hd)).astype(np.float32) * 1.2)
    v = np.zeros((seq, hkv * hd), np.float32)
    v[np.arange(seq), np.arange(seq)] = 1.0
    lo, hi, bits = kernels.block_diagonal_segments(prefix, levels, pad)
    dl, dh = torch.from_numpy(lo).to(cuda), torch.from_numpy(hi).to(cuda)
    db = torch.from_numpy(bits.view(np.int64)).to(cuda) if pad is not None else None
    out = kernels.attention_bf16_seg(_bf16_dev(q, cuda), _bf16_dev(k, cuda), _bf16_dev(v, cuda),
                                     1, seq, hq, hkv, hd, prefix, dl, dh, db)
    torch.cuda.synchronize()
    mask = oracle.block_diagonal_mask(prefix, levels, pad)
    got = out.cpu().numpy().reshape(seq, hq, hd)[:, :, :seq]
    ref = oracle.attention_core(q, k, v, mask, hq, hkv, hd).reshape(seq, hq, hd)[:, :, :seq]
    allowed = np.broadcast_to(mask.astype(bool)[:, None, :], got.shape)
    assert np.all(got[~allowed] == 0)
    same = float(np.mean(got[allowed].view(np.uint32) == ref[allowed].view(np.uint32)))
    print(f"p bit-identical: {same:.6f} of {int(allowed.sum())}", flush=True)
    assert np.all(np.abs(got - ref) <= 2.0**-7 * np.abs(ref) + 2.0**-16)
    assert same >= 0.9995, same
