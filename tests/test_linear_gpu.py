"""GPU parity of the bf16 linear against the oracle (restatement of
packages/kernels/root.zig:96-148).

Tolerance (fp32 output vs the oracle's pre-rounding fp32 sum):
|y - ref| <= 1e-3 + 1e-2 |ref|. Every output is additionally held to the
D53 form |y - y_f64| <= (K + 1) 2^-24 sum|x w| (PROJECT.md:506), which any
RNE fp32 summation order of exact bf16 products satisfies.
"""
import numpy as np
import pytest

from ncmorph_amd import synth

RTOL, ATOL = 1e-2, 1e-3
pytestmark = pytest.mark.gpu


def _to_dev(bits, cuda):
    import torch

    return torch.from_numpy(bits.view(np.int16).copy()).to(cuda).view(torch.bfloat16)


def _run(x_bits, w_bits, cuda, bias_bits=None, out_mode="f32"):
    import torch
    from ncmorph_amd import kernels

    x = _to_dev(x_bits, cuda)
    w = _to_dev(w_bits, cuda)
    b = None if bias_bits is None else _to_dev(bias_bits, cuda)
    y = kernels.linear_bf16(x, w, bias=b, out_mode=out_mode)
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    return out.view(np.uint16) if out_mode == "bf16" else out


def test_dropin_kats(ncm, oracle, cuda):
    """The reference KAT inputs through the host drop-in (root.zig:707-770)."""
    from ncmorph_amd import kernels

    from .test_oracle_linear import kat_inputs

    x, w = kat_inputs()
    out = np.zeros((4, 576), np.float32)
    kernels.matmul_bf16(x.ravel(), w.ravel(), out.ravel(), 4, 1536, 576)
    ref, s = oracle.matmul_bf16(x, w, want_sum=True)
    assert np.all(np.abs(out - s) <= ATOL + RTOL * np.abs(s))
    # Output is bf16-valued.
    assert np.array_equal(out, oracle.round_bf16(out))
    agree = np.mean(out == ref)
    assert agree > 0.97, agree
    # Flush KAT (root.zig:746-755): exactly zero.
    v = np.float32(5.421010862427522e-20)
    o1 = np.zeros(1, np.float32)
    kernels.matmul_bf16(np.array([v, v], np.float32), np.array([v, v], np.float32), o1, 1, 2, 1)
    assert o1[0] == 0.0
    # K-block KAT (root.zig:757-770): within tolerance of 1.0078125.
    xi = np.full(576, 5.960464477539063e-8, np.float32)
    xi[0] = 1.0
    xi[-1] = 0.00390625
    o2 = np.zeros(1, np.float32)
    kernels.matmul_bf16(xi, np.ones(576, np.float32), o2, 1, 576, 1)
    assert abs(o2[0] - 1.0078125) <= ATOL + RTOL * 1.0078125


def test_dropin_bias_and_ragged(ncm, oracle, cuda):
    from ncmorph_amd import kernels

    rng = np.random.default_rng(11)
    for T, K, N in [(1, 1, 1), (3, 7, 5), (17, 130, 33), (65, 1030, 257), (300, 64, 129)]:
        x = rng.standard_normal((T, K)).astype(np.float32)
        w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
        b = rng.standard_normal(N).astype(np.float32)
        out = np.zeros((T, N), np.float32)
        kernels.matmul_bf16_bias(x.ravel(), w.ravel(), b, out.ravel(), T, K, N)
        ref, s = oracle.matmul_bf16(x, w, bias=b, want_sum=True)
        assert np.all(np.abs(out - s) <= ATOL + RTOL * np.abs(s)), (T, K, N)
        out2 = np.zeros((T, N), np.float32)
        kernels.matmul_bf16(x.ravel(), w.ravel(), out2.ravel(), T, K, N)
        ref2, s2 = oracle.matmul_bf16(x, w, want_sum=True)
        assert np.all(np.abs(out2 - s2) <= ATOL + RTOL * np.abs(s2)), (T, K, N)


def test_round_bf16_device_matches_reference_vectors(ncm, cuda):
    import os

    from ncmorph_amd import kernels

    pairs = np.load(os.path.join(os.path.dirname(__file__), "golden", "bf16_pairs.npy"))
    f = pairs[:, 0].astype(np.uint32).view(np.float32)
    got = kernels.round_bf16(f).view(np.uint32) >> 16
    assert np.array_equal(got.astype(np.uint16), pairs[:, 1].astype(np.uint16))


def test_device_conversions_against_oracle(ncm, oracle, cuda):
    """Device bf16 conversions: every bf16 pattern widens exactly and
    rounds back to itself (bf16/root.zig:50-59; NaN payloads -> 0x7FC0);
    f32 -> bf16 agrees with the oracle's RNE on rounding-critical patterns,
    with and without the operand flush (kernels/root.zig:144-148)."""
    import torch
    from ncmorph_amd import kernels

    bits = np.arange(65536, dtype=np.uint16)
    wide = kernels.bf16_widen(torch.from_numpy(bits.view(np.int16)).to(cuda).view(torch.bfloat16))
    w = wide.cpu().numpy()
    assert np.array_equal(w.view(np.uint32), bits.astype(np.uint32) << 16)
    back = kernels.bf16_from_f32(wide).cpu().view(torch.int16).numpy().view(np.uint16)
    nan = (bits & 0x7F80) == 0x7F80
    nan &= (bits & 0x007F) != 0
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.all(back[nan] == 0x7FC0)
    rng = np.random.default_rng(11)
    hi = rng.integers(0, 1 << 16, 1 << 18, dtype=np.uint32) << 16
    lo = np.array([0x0000, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    f32 = (hi[:, None] | lo[None, :]).ravel().view(np.float32)
    fd = torch.from_numpy(f32).to(cuda)
    for flush in (False, True):
        got = kernels.bf16_from_f32(fd, flush=flush).cpu().view(torch.int16).numpy().view(np.uint16)
        ref = oracle.bf16_from_f32(f32)
        if flush:
            ref = np.where((ref & 0x7F80) == 0, ref & 0x8000, ref).astype(np.uint16)
        assert np.array_equal(got, ref), flush


@pytest.mark.parametrize("n,k", [(2048, 2048), (8192, 2048), (2048, 8192)])
def test_linear_1b_shapes(ncm, oracle, cuda, n, k):
    """Config shapes: x [2048, k] ~N(0,1), W [n, k] ~N(0, 0.02^2), bf16."""
    m = 2048
    xb = synth.normal_bf16(synth.LINEAR_SEED_X + k, (m, k))
    wb = synth.normal_bf16(synth.LINEAR_SEED_W + n * 7 + k, (n, k), std=0.02)
    y = _run(xb, wb, cuda)
    x64 = synth.bf16_to_f32(xb).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    ref = x64 @ w64.T
    asum = np.abs(x64) @ np.abs(w64).T
    err = np.abs(y - ref)
    assert np.all(err <= (k + 1) * 2.0**-24 * asum), float(np.max(err / asum))
    # Oracle rows (exact reference arithmetic) on a sample of rows.
    rows = [0, 1, 777, m - 1]
    for r in rows:
        yb, s = oracle.matmul_bf16_u16_rows(xb[r:r + 1], wb, 0, 1)
        assert np.all(np.abs(y[r] - s[0]) <= ATOL + RTOL * np.abs(s[0]))
        yb16 = synth.bf16_bits(y[r:r + 1])
        agree = np.mean(synth.bf16_to_f32(yb16) == yb)
        assert agree > 0.99, agree


def test_linear_out_modes_and_bias(ncm, cuda):
    rng = np.random.default_rng(5)
    m, k, n = 300, 520, 260
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32))
    y32 = _run(xb, wb, cuda, bias_bits=bb)
    ybf = _run(xb, wb, cuda, bias_bits=bb, out_mode="bf16_f32")
    y16 = _run(xb, wb, cuda, bias_bits=bb, out_mode="bf16")
    assert np.array_equal(ybf, synth.bf16_to_f32(synth.bf16_bits(y32)))
    assert np.array_equal(y16, synth.bf16_bits(y32))
    ref = (synth.bf16_to_f32(xb).astype(np.float64) @ synth.bf16_to_f32(wb).astype(np.float64).T
           + synth.bf16_to_f32(bb).astype(np.float64))
    assert np.all(np.abs(y32 - ref) <= ATOL + RTOL * np.abs(ref))


def test_linear_zero_k_and_empty(ncm, cuda):
    import torch
    from ncmorph_amd import kernels

    x = torch.zeros((4, 0), dtype=torch.bfloat16, device=cuda)
    w = torch.zeros((3, 0), dtype=torch.bfloat16, device=cuda)
    y = kernels.linear_bf16(x, w)
    torch.cuda.synchronize()
    assert torch.all(y == 0)
    x = torch.zeros((0, 8), dtype=torch.bfloat16, device=cuda)
    w = torch.zeros((3, 8), dtype=torch.bfloat16, device=cuda)
    assert kernels.linear_bf16(x, w).shape == (0, 3)


@pytest.mark.parametrize("m,k,n", [
    (200, 1096, 300),     # 128 x 128 tiles, four LDS stages
    (2148, 1096, 5400),   # 256 x 256 tiles (198 of them)
    (2148, 1096, 2800),   # 256 x 128 tiles (198 of them)
])
def test_linear_ragged_long_k_bias_modes_repeatable(ncm, cuda, m, k, n):
    """Ragged M and N, K not a multiple of the 64-wide K tile (partial last
    tile), bias, every output mode against the D53 bound and each other, and
    identical bits over repeated launches; one shape per tile configuration
    the automatic choice uses."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(77 + m)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32))
    y32 = _run(xb, wb, cuda, bias_bits=bb)
    x64 = synth.bf16_to_f32(xb).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    ref = x64 @ w64.T + synth.bf16_to_f32(bb).astype(np.float64)
    asum = np.abs(x64) @ np.abs(w64).T + np.abs(synth.bf16_to_f32(bb))
    assert np.all(np.abs(y32 - ref) <= (k + 2) * 2.0**-24 * asum)
    assert np.array_equal(_run(xb, wb, cuda, bias_bits=bb, out_mode="bf16"), synth.bf16_bits(y32))
    ybf = _run(xb, wb, cuda, bias_bits=bb, out_mode="bf16_f32")
    assert np.array_equal(ybf, synth.bf16_to_f32(synth.bf16_bits(y32)))
    # Repeated launches give identical bits.
    x = _to_dev(xb, cuda)
    w = _to_dev(wb, cuda)
    b = _to_dev(bb, cuda)
    outs = [kernels.linear_bf16(x, w, bias=b) for _ in range(5)]
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    assert np.array_equal(outs[0].cpu().numpy(), y32)


@pytest.mark.parametrize("m,n,k", [(96, 512, 2048), (64, 128256, 2048)])
def test_linear_decoder_caller_shapes(ncm, oracle, cuda, m, n, k):
    """The other shapes the reference's callers pass (decoder.project k/v:
    out 512; the LM head tied to the 128256-row embedding, decoder.zig:219-227)
    at a few tokens: partial row tiles, wide grids."""
    rng = np.random.default_rng(n + m)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    y = _run(xb, wb, cuda)
    x64 = synth.bf16_to_f32(xb).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    ref = x64 @ w64.T
    asum = np.abs(x64) @ np.abs(w64).T
    assert np.all(np.abs(y - ref) <= (k + 1) * 2.0**-24 * asum)
    for r in (0, m - 1):
        _, s = oracle.matmul_bf16_u16_rows(xb[r:r + 1], wb, 0, 1)
        assert np.all(np.abs(y[r] - s[0]) <= ATOL + RTOL * np.abs(s[0]))


@pytest.mark.parametrize("m,n,k", [
    (4096, 8192, 8),      # 256 x 256 tiles, 512 of them (two rounds), one K tile
    (4096, 8192, 200),    # the same with a partial last K tile
    (2560, 3584, 64),     # 256 x 128 tiles (280): one K tile, fewer than the stages
    (2560, 3584, 136),    # 256 x 128 with three K tiles, the last partial
    (2560, 3584, 1024),
])
def test_linear_multi_round_grids(ncm, cuda, m, n, k):
    """Grids with more tiles than the CUs hold at once, short and partial K:
    rows from every row tile against the D53 bound; the bf16 modes and the
    residual-fused form against the fp32 output."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m + n + k)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32))
    x, w, b = _to_dev(xb, cuda), _to_dev(wb, cuda), _to_dev(bb, cuda)
    y = kernels.linear_bf16(x, w, bias=b)
    ybf = kernels.linear_bf16(x, w, bias=b, out_mode="bf16_f32")
    res = torch.from_numpy(rng.standard_normal((m, n)).astype(np.float32)).to(cuda)
    yres = kernels.linear_bf16_residual(x, w, res, bias=b, out_mode="f32")
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.arange(0, m, 37)
    x64 = synth.bf16_to_f32(xb[rows]).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    b64 = synth.bf16_to_f32(bb).astype(np.float64)
    ref = x64 @ w64.T + b64
    asum = np.abs(x64) @ np.abs(w64).T + np.abs(b64)
    assert np.all(np.abs(y[rows] - ref) <= (k + 2) * 2.0**-24 * asum)
    assert np.array_equal(ybf.cpu().numpy(), synth.bf16_to_f32(synth.bf16_bits(y)))
    assert np.array_equal(yres.cpu().numpy(), res.cpu().numpy() + y)


def _flush_f32(a):
    """Subnormal fp32 values to signed zero (packages/kernels/root.zig:144-148)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).copy()
    sub = (u & np.uint32(0x7F800000)) == 0
    u[sub] &= np.uint32(0x80000000)
    return u.view(np.float32)


def test_linear_bf16_modes_special_values(ncm, cuda):
    """The bf16 output modes on sums that are NaN, infinite, overflowing or
    subnormal: every output equals the reference's rounding of the fp32 sum
    (flush, RNE, NaN -> 0x7FC0), with and without the residual add, on a
    whole-tile shape (the paired-rounding epilogue) and a ragged one."""
    import torch
    from ncmorph_amd import kernels

    for m, n, k in [(512, 512, 256), (300, 200, 72)]:
        rng = np.random.default_rng(m + k)
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[1, 5] = np.nan
        x[2, 7] = np.inf
        x[3, :] = np.float32(3e38)            # sums overflow to +-inf
        x[4, :] = np.float32(1.2e-38)         # products and sums subnormal
        x[5, 0] = -np.inf
        xb = synth.bf16_bits(x)
        wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
        xd, wd = _to_dev(xb, cuda), _to_dev(wb, cuda)
        y32 = kernels.linear_bf16(xd, wd)
        ybf = kernels.linear_bf16(xd, wd, out_mode="bf16")
        yb32 = kernels.linear_bf16(xd, wd, out_mode="bf16_f32")
        res = rng.standard_normal((m, n)).astype(np.float32)
        res[6, :3] = [np.nan, np.inf, -np.inf]
        resd = torch.from_numpy(res).to(cuda)
        yres = kernels.linear_bf16_residual(xd, wd, resd, out_mode="bf16_f32")
        torch.cuda.synchronize()
        y = y32.cpu().numpy()
        want = synth.bf16_bits(_flush_f32(y))
        assert np.isnan(y[1]).any() and np.isinf(y[3]).any()
        assert np.array_equal(ybf.cpu().numpy().view(np.uint16), want)
        bits = lambda a: np.ascontiguousarray(a, np.float32).view(np.uint32)
        assert np.array_equal(bits(yb32.cpu().numpy()), bits(synth.bf16_to_f32(want)))
        with np.errstate(invalid="ignore"):
            want_res = synth.bf16_bits(res + synth.bf16_to_f32(want))
        assert np.array_equal(bits(yres.cpu().numpy()), bits(synth.bf16_to_f32(want_res)))
