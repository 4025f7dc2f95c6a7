"""GPU parity of the linear with fused SwiGLU and RoPE epilogues: the same
bits as the unfused device composition (the bf16 linear, then the SiLU x up
kernel or the RoPE rotation), which the other tests pin against the oracle.
Shapes reach the three automatic tile configurations, partial row tiles and
bias; the RoPE case covers the q|k|v layout with unrotated v columns."""
import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu


def _bf16(rng, shape, std, cuda):
    import torch

    bits = synth.bf16_bits((rng.standard_normal(shape) * std).astype(np.float32))
    return torch.from_numpy(bits.view(np.int16).copy()).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("m,inter,k,bias", [(4096, 8192, 256, False), (200, 256, 1096, True),
                                            (2048, 2048, 512, True), (33, 64, 64, False)])
def test_swiglu_epilogue_matches_unfused(ncm, cuda, m, inter, k, bias):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m + inter + k)
    x = _bf16(rng, (m, k), 1.0, cuda)
    gate = _bf16(rng, (inter, k), 0.05, cuda)
    up = _bf16(rng, (inter, k), 0.05, cuda)
    bg = _bf16(rng, (inter,), 0.5, cuda) if bias else None
    bu = _bf16(rng, (inter,), 0.5, cuda) if bias else None
    w = kernels.interleave_gate_up(gate, up)
    b = kernels.interleave_gate_up(bg, bu) if bias else None
    fused = kernels.linear_bf16_swiglu(x, w, bias=b)
    g = kernels.linear_bf16(x, gate, bias=bg, out_mode="bf16_f32")
    u = kernels.linear_bf16(x, up, bias=bu, out_mode="bf16_f32")
    ref = kernels.silu_mul(g, u, out_mode="bf16")
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize("m,hq,hkv,seq,bias", [(4096, 32, 8, 1024, False), (300, 4, 2, 150, True),
                                               (64, 2, 1, 64, False)])
def test_rope_epilogue_matches_unfused(ncm, oracle, cuda, m, hq, hkv, seq, bias):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m + hq + seq)
    k = 512
    n = (hq + 2 * hkv) * 64
    x = _bf16(rng, (m, k), 1.0, cuda)
    w = _bf16(rng, (n, k), 0.05, cuda)
    b = _bf16(rng, (n,), 0.5, cuda) if bias else None
    inv = oracle.rope_llama3(64, 500000.0, 32.0, 1.0, 4.0, 8192)
    cos, sin = oracle.rope_tables(inv, seq)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    rot = (hq + hkv) * 64
    fused = kernels.linear_bf16_rope64(x, w, rot, seq, cd, sd, bias=b)
    ref = kernels.linear_bf16(x, w, bias=b, out_mode="bf16").view(torch.bfloat16)
    kernels.rope_rotate(ref[:, :hq * 64], hq, 64, seq, cd, sd)
    kernels.rope_rotate(ref[:, hq * 64:rot], hkv, 64, seq, cd, sd)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))


def _special_x(rng, m, k, cuda):
    """bf16 activations with NaN, +-inf and huge entries in a few rows, so that
    projections come out NaN, infinite or overflowing."""
    import torch

    x = rng.standard_normal((m, k)).astype(np.float32)
    x[1, 3] = np.nan
    x[2, 5] = np.inf
    x[3, 0] = -np.inf
    x[4, :] = np.float32(3e38)
    bits = synth.bf16_bits(x)
    return torch.from_numpy(bits.view(np.int16).copy()).to(cuda).view(torch.bfloat16)


def test_fused_epilogues_special_values(ncm, oracle, cuda):
    """NaN and infinite projections through the fused SwiGLU and RoPE
    epilogues: the same bits as the unfused kernels (every NaN -> 0x7FC0)."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(91)
    m, inter, k = 512, 512, 128
    x = _special_x(rng, m, k, cuda)
    gate = _bf16(rng, (inter, k), 0.05, cuda)
    up = _bf16(rng, (inter, k), 0.05, cuda)
    fused = kernels.linear_bf16_swiglu(x, kernels.interleave_gate_up(gate, up))
    g = kernels.linear_bf16(x, gate, out_mode="bf16_f32")
    u = kernels.linear_bf16(x, up, out_mode="bf16_f32")
    ref = kernels.silu_mul(g, u, out_mode="bf16")
    torch.cuda.synchronize()
    assert torch.isnan(fused[1].float()).any()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))

    hq, hkv, seq = 4, 2, 128
    n = (hq + 2 * hkv) * 64
    w = _bf16(rng, (n, k), 0.05, cuda)
    inv = oracle.rope_llama3(64, 500000.0, 32.0, 1.0, 4.0, 8192)
    cos, sin = oracle.rope_tables(inv, seq)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    rot = (hq + hkv) * 64
    fused = kernels.linear_bf16_rope64(x, w, rot, seq, cd, sd)
    ref = kernels.linear_bf16(x, w, out_mode="bf16").view(torch.bfloat16)
    kernels.rope_rotate(ref[:, :hq * 64], hq, 64, seq, cd, sd)
    kernels.rope_rotate(ref[:, hq * 64:rot], hkv, 64, seq, cd, sd)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
