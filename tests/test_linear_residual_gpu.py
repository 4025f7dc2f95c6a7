"""GPU parity of the linear with the residual add fused into its epilogue:
y = residual + x w^T (+ bias), the projection followed by the decoder's
add_rows (src/decoder.zig:279-282).

The projection's own sum is checked by the linear tests; here the fused
result must equal, bit for bit, the unfused composition of the same device
linear and the reference's add: f32 mode residual + v, bf16 modes
round_bf16(residual + round_bf16(v)), computed on the host from the plain
linear's output. Shapes reach the three automatic tile configurations, the
vector and per-element epilogues (ragged M and N), bias, and in-place use.
"""
import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu


def _to_dev(bits, cuda):
    import torch

    return torch.from_numpy(bits.view(np.int16).copy()).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("m,n,k,bias", [(4096, 4096, 256, False), (2048, 4096, 512, True),
                                        (96, 2048, 2048, False), (200, 300, 1096, True),
                                        (5, 7, 8, False)])
def test_linear_residual_matches_unfused(ncm, oracle, cuda, m, n, k, bias):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m * 7 + n + k)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32)) if bias else None
    # Hidden states are bf16-valued in the bf16 mode; include exact cancellations.
    res = oracle.round_bf16(rng.standard_normal((m, n)).astype(np.float32) * 4)
    x, w = _to_dev(xb, cuda), _to_dev(wb, cuda)
    b = None if bb is None else _to_dev(bb, cuda)
    rd = torch.from_numpy(res).to(cuda)

    plain = kernels.linear_bf16(x, w, bias=b, out_mode="f32")
    y32 = kernels.linear_bf16_residual(x, w, rd, bias=b, out_mode="f32")
    ybf = kernels.linear_bf16_residual(x, w, rd, bias=b, out_mode="bf16_f32")
    y16 = kernels.linear_bf16_residual(x, w, rd, bias=b, out_mode="bf16")
    torch.cuda.synchronize()
    v = plain.cpu().numpy()
    assert np.array_equal(y32.cpu().numpy().view(np.uint32), (res + v).view(np.uint32))
    want = oracle.round_bf16(res + synth.bf16_to_f32(synth.bf16_bits(v)))
    assert np.array_equal(ybf.cpu().numpy().view(np.uint32), want.view(np.uint32))
    bits16 = y16.cpu().numpy().view(np.uint16)
    assert np.array_equal(bits16, synth.bf16_bits(want))

    # In place on the hidden state (f32 and bf16_f32 modes).
    for mode, ref in (("f32", res + v), ("bf16_f32", want)):
        h = torch.from_numpy(res).to(cuda)
        out = kernels.linear_bf16_residual(x, w, h, bias=b, out=h, out_mode=mode)
        torch.cuda.synchronize()
        assert out.data_ptr() == h.data_ptr()
        assert np.array_equal(h.cpu().numpy().view(np.uint32), ref.view(np.uint32)), mode


def test_linear_residual_rejects_bf16_in_place(ncm, cuda):
    import torch
    from ncmorph_amd import kernels
    from ncmorph_amd._lib import NcmError

    x = torch.zeros((8, 8), dtype=torch.bfloat16, device=cuda)
    w = torch.zeros((8, 8), dtype=torch.bfloat16, device=cuda)
    h = torch.zeros((8, 8), dtype=torch.float32, device=cuda)
    with pytest.raises(NcmError):
        kernels.linear_bf16_residual(x, w, h, out=h, out_mode="bf16")
