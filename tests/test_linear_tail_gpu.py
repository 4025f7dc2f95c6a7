"""Rows past the last full 256-row tile of the bf16 linear
(csrc/linear_tail.hip): when M % 256 is at most 64, K % 2048 == 0 and the
partial row tile would cost the chip an extra round, those rows run on the
skinny tail kernel (fp32 sums in another order than the tile kernel's).

Bars (the linear's own, packages/kernels/root.zig:96-142): every tail output
within the D53 bound |y - y_f64| <= (K + 1) 2^-24 sum|x w| (+ |bias|), sampled
tail rows within rel 1e-2 / abs 1e-3 of the oracle's reference arithmetic and
>= 99% equal after bf16 rounding. Bit for bit: a row's outputs are the same
whatever M it is the tail of; the bf16 output modes, the residual epilogue and
the fused SwiGLU are the tail's fp32 result rounded / added / combined exactly
as the tile kernels do it."""
import numpy as np
import pytest

from ncmorph_amd import synth

RTOL, ATOL = 1e-2, 1e-3
pytestmark = pytest.mark.gpu


def _dev(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).to(cuda).view(
        torch.bfloat16)


def _d53(y, xb, wb, bb=None, rows=None):
    x64 = synth.bf16_to_f32(xb if rows is None else xb[rows]).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    ref = x64 @ w64.T
    asum = np.abs(x64) @ np.abs(w64).T
    if bb is not None:
        b64 = synth.bf16_to_f32(bb).astype(np.float64)
        ref, asum = ref + b64, asum + np.abs(b64)
    k = xb.shape[1]
    return np.all(np.abs(y - ref) <= (k + 2) * 2.0**-24 * asum)


@pytest.mark.parametrize("tail", [1, 16, 32, 33, 64])
def test_tail_rows_against_bound_oracle_and_other_batches(ncm, oracle, cuda, tail):
    import torch
    from ncmorph_amd import kernels

    n, k = 8192, 2048
    print(f"linear tail rows={tail} n={n} k={k}", flush=True)
    rng = np.random.default_rng(900 + tail)
    xb = synth.bf16_bits(rng.standard_normal((2048 + tail, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x, w = _dev(xb, cuda), _dev(wb, cuda)
    y = kernels.linear_bf16(x, w)
    # The same tail rows after 4096 other rows (a 17th row tile: 544 tiles),
    # and inside full row tiles (M = 2304: the tile kernel).
    xb2 = np.concatenate([synth.bf16_bits(rng.standard_normal((4096, k)).astype(np.float32)),
                          xb[2048:]])
    y2 = kernels.linear_bf16(_dev(xb2, cuda), w)
    xb3 = np.concatenate([xb, np.zeros((256 - tail, k), np.uint16)])
    y3 = kernels.linear_bf16(_dev(xb3, cuda), w)
    torch.cuda.synchronize()
    y, y2, y3 = y.cpu().numpy(), y2.cpu().numpy(), y3.cpu().numpy()
    t = slice(2048, 2048 + tail)
    assert _d53(y[t], xb, wb, rows=t)
    assert _d53(y[::97], xb, wb, rows=slice(None, None, 97))
    assert np.array_equal(y[t], y2[4096:])
    assert np.array_equal(y[:2048], y3[:2048])
    # Both within the bound, but not the same sums: the tail kernel ran.
    assert _d53(y3[t], xb, wb, rows=t)
    assert not np.array_equal(y[t], y3[t])
    for r in (2048, 2048 + tail - 1):
        yb, s = oracle.matmul_bf16_u16_rows(xb[r:r + 1], wb, 0, 1)
        assert np.all(np.abs(y[r] - s[0]) <= ATOL + RTOL * np.abs(s[0]))
        agree = np.mean(synth.bf16_to_f32(synth.bf16_bits(y[r:r + 1])) == yb)
        assert agree > 0.99, agree


def test_tail_epilogues_bit_for_bit(ncm, cuda):
    """Bias, the bf16 modes and the residual epilogue of the tail against its
    own fp32 output, and the fused SwiGLU tail against the plain tail of the
    interleaved weight followed by the SiLU x up kernel; repeat launches give
    the same bits."""
    import torch
    from ncmorph_amd import kernels

    m, n, k = 2048 + 32, 8192, 4096
    rng = np.random.default_rng(31)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32))
    x, w, b = _dev(xb, cuda), _dev(wb, cuda), _dev(bb, cuda)
    y32 = kernels.linear_bf16(x, w, bias=b)
    ybf = kernels.linear_bf16(x, w, bias=b, out_mode="bf16_f32")
    y16 = kernels.linear_bf16(x, w, bias=b, out_mode="bf16")
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(cuda)
    yres = kernels.linear_bf16_residual(x, w, res, bias=b, out_mode="f32")
    yresb = kernels.linear_bf16_residual(x, w, res, bias=b, out_mode="bf16_f32")
    again = [kernels.linear_bf16(x, w, bias=b) for _ in range(3)]
    torch.cuda.synchronize()
    y32n = y32.cpu().numpy()
    assert _d53(y32n[2048:], xb, wb, bb, rows=slice(2048, None))
    assert np.array_equal(ybf.cpu().numpy(), synth.bf16_to_f32(synth.bf16_bits(y32n)))
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), synth.bf16_bits(y32n))
    r = res.cpu().numpy()
    assert np.array_equal(yres.cpu().numpy(), r + y32n)
    want = synth.bf16_to_f32(synth.bf16_bits(r + synth.bf16_to_f32(synth.bf16_bits(y32n))))
    assert np.array_equal(yresb.cpu().numpy(), want)
    for a in again:
        assert torch.equal(a, y32)

    # SwiGLU: 4096 features, weight rows interleaved in groups of 32.
    fused = kernels.linear_bf16_swiglu(x, w, bias=b)
    proj = kernels.linear_bf16(x, w, bias=b, out_mode="bf16_f32")
    torch.cuda.synchronize()
    cols = np.arange(n).reshape(-1, 64)
    gate = proj[:, torch.from_numpy(cols[:, :32].ravel()).to(cuda)].contiguous()
    up = proj[:, torch.from_numpy(cols[:, 32:].ravel()).to(cuda)].contiguous()
    ref = kernels.silu_mul(gate, up, out_mode="bf16")
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))


def test_tail_special_values(ncm, cuda):
    """NaN, +-inf and overflowing projections in the tail rows: the bf16 and
    residual epilogues against the tail's own fp32 output, and the fused
    SwiGLU tail against the plain tail + SiLU x up (every NaN -> 0x7FC0)."""
    import torch
    from ncmorph_amd import kernels

    m, n, k = 2048 + 16, 8192, 2048
    rng = np.random.default_rng(57)
    xf = rng.standard_normal((m, k)).astype(np.float32)
    xf[2049, 3] = np.nan
    xf[2050, 5] = np.inf
    xf[2051, 0] = -np.inf
    xf[2052, :] = np.float32(3e38)
    xb = synth.bf16_bits(xf)
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x, w = _dev(xb, cuda), _dev(wb, cuda)
    y32 = kernels.linear_bf16(x, w)
    y16 = kernels.linear_bf16(x, w, out_mode="bf16")
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(cuda)
    yresb = kernels.linear_bf16_residual(x, w, res, out_mode="bf16_f32")
    fused = kernels.linear_bf16_swiglu(x, w)
    proj = kernels.linear_bf16(x, w, out_mode="bf16_f32")
    torch.cuda.synchronize()
    y32n = y32.cpu().numpy()
    tail = y32n[2048:]
    assert np.isnan(tail[1]).all() and np.isinf(tail[2]).any() and np.isinf(tail[3]).any()
    assert np.array_equal(y16.cpu().numpy().view(np.uint16), synth.bf16_bits(y32n))
    r = res.cpu().numpy()
    want = synth.bf16_to_f32(synth.bf16_bits(r + synth.bf16_to_f32(synth.bf16_bits(y32n))))
    got = yresb.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    cols = np.arange(n).reshape(-1, 64)
    gate = proj[:, torch.from_numpy(cols[:, :32].ravel()).to(cuda)].contiguous()
    up = proj[:, torch.from_numpy(cols[:, 32:].ravel()).to(cuda)].contiguous()
    ref = kernels.silu_mul(gate, up, out_mode="bf16")
    torch.cuda.synchronize()
    assert torch.isnan(fused[2049].float()).any()
    assert torch.equal(fused.view(torch.int16), ref.view(torch.int16))
