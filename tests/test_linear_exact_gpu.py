"""GPU parity of the exact bf16 linear (ncm_matmul_bf16_exact,
ncm_matmul_bf16_bias_exact, ncm_linear_bf16_exact) against the reference's
matmul_bf16_impl (packages/kernels/root.zig:106-142).

Bar: bit-identical. The reference's own known-answer tests (root.zig:707-770)
through the host drop-ins, then the oracle's restatement (itself pinned by
those KATs) on shapes that cross every rule: K below, at and between the
512 / 1024 block sizes, odd K (the lone last element), K = 1, bias, NaN and
infinity, bf16 subnormal operands, products and partials that underflow, and
several 64 x 64 output tiles with ragged edges.
"""
import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu


def _dev(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).to(cuda).view(
        torch.bfloat16)


def test_reference_kats_bit_exact(ncm, oracle, cuda):
    """root.zig:707-744 (digest and three values), :746-755 (a subnormal
    product flushes to 0), :757-770 (512-wide K blocks give 1.0078125)."""
    from ncmorph_amd import kernels

    from .test_oracle_linear import kat_inputs

    x, w = kat_inputs()
    out = np.zeros((4, 576), np.float32)
    kernels.matmul_bf16_exact(x.ravel(), w.ravel(), out.ravel(), 4, 1536, 576)
    assert oracle.digest(out) == 0x547F69F667C8103F
    assert out.ravel()[0] == np.float32(-0.466796875)
    assert out.ravel()[1] == np.float32(1.109375)
    assert out.ravel()[1793] == np.float32(-0.796875)
    v = np.float32(5.421010862427522e-20)
    o1 = np.full(1, 7.0, np.float32)
    kernels.matmul_bf16_exact(np.array([v, v], np.float32), np.array([v, v], np.float32), o1,
                              1, 2, 1)
    assert o1[0] == 0.0
    xi = np.full(576, 5.960464477539063e-8, np.float32)
    xi[0] = 1.0
    xi[-1] = 0.00390625
    o2 = np.zeros(1, np.float32)
    kernels.matmul_bf16_exact(xi, np.ones(576, np.float32), o2, 1, 576, 1)
    assert o2[0] == np.float32(1.0078125)


@pytest.mark.parametrize("T,K,N", [(1, 1, 1), (3, 7, 5), (17, 130, 33), (65, 512, 70),
                                   (9, 513, 64), (70, 1023, 65), (5, 1024, 129),
                                   (4, 1025, 3), (66, 2048, 130), (2, 3001, 7)])
def test_dropins_match_oracle_bits(ncm, oracle, cuda, T, K, N):
    from ncmorph_amd import kernels

    rng = np.random.default_rng(T * 7919 + K * 31 + N)
    x = rng.standard_normal((T, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    out = np.zeros((T, N), np.float32)
    kernels.matmul_bf16_exact(x.ravel(), w.ravel(), out.ravel(), T, K, N)
    assert np.array_equal(out.view(np.uint32), oracle.matmul_bf16(x, w).view(np.uint32))
    outb = np.zeros((T, N), np.float32)
    kernels.matmul_bf16_bias_exact(x.ravel(), w.ravel(), b, outb.ravel(), T, K, N)
    assert np.array_equal(outb.view(np.uint32),
                          oracle.matmul_bf16(x, w, bias=b).view(np.uint32))


def test_underflow_specials_and_subnormal_operands(ncm, oracle, cuda):
    """Operands straddling the f32 subnormal range (some products and partial
    sums underflow and flush, with their signs), bf16 subnormal operands,
    infinities and a NaN, bit for bit through the drop-in."""
    from ncmorph_amd import kernels

    rng = np.random.default_rng(5)
    T, K, N = 8, 600, 12
    scale = np.float32(2.0) ** rng.integers(-75, -55, size=(T, K)).astype(np.float32)
    x = (rng.standard_normal((T, K)).astype(np.float32) * scale).astype(np.float32)
    w = (rng.standard_normal((N, K)).astype(np.float32) *
         np.float32(2.0) ** rng.integers(-75, -55, size=(N, K)).astype(np.float32))
    x[0, :5] = np.float32(1e-39)  # bf16 subnormal operands: flushed
    x[1, 3] = np.inf
    w[2, 4] = -np.inf
    x[3, 7] = np.nan
    out = np.zeros((T, N), np.float32)
    kernels.matmul_bf16_exact(x.ravel(), w.astype(np.float32).ravel(), out.ravel(), T, K, N)
    ref = oracle.matmul_bf16(x, w.astype(np.float32))
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_device_entry_sum_and_modes(ncm, oracle, cuda):
    """ncm_linear_bf16_exact on device bf16 tensors: "f32" gives the oracle's
    fp32 sum before the output rounding (bias included), "bf16_f32" its
    output and "bf16" its bits; bf16 subnormal operands are flushed in the
    kernel."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(9)
    T, K, N = 130, 1100, 67
    xb = synth.bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((N, K)) * 0.03).astype(np.float32))
    xb[0, :3] = 0x0001  # bf16 subnormal
    wb[1, 5] = 0x8003
    bb = synth.bf16_bits(rng.standard_normal(N).astype(np.float32))
    xd, wd, bd = _dev(xb, cuda), _dev(wb, cuda), _dev(bb, cuda)
    s = kernels.linear_bf16_exact(xd, wd, bias=bd, out_mode="f32")
    y = kernels.linear_bf16_exact(xd, wd, bias=bd, out_mode="bf16_f32")
    yb = kernels.linear_bf16_exact(xd, wd, bias=bd, out_mode="bf16")
    torch.cuda.synchronize()
    xf = oracle.bf16_to_f32(xb)
    wf = oracle.bf16_to_f32(wb)
    bf = oracle.bf16_to_f32(bb)
    ref, ref_sum = oracle.matmul_bf16(xf, wf, bias=bf, want_sum=True)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), ref_sum.view(np.uint32))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(yb.cpu().numpy().view(np.uint16), oracle.bf16_from_f32(ref))
