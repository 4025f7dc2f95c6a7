"""GPU parity of the decoder ops around the linear against the oracle
(restatement of packages/kernels/root.zig:150-270, src/decoder.zig:168-211).

RMSNorm (bf16 mode): bit-identical to the oracle, which reproduces the
reference's pinned cascade KATs bit for bit. SiLU: the device's expf and the
reference's exp may differ in the last fp32 bit, so results may differ by
one bf16 step where the quotient sits next to a rounding boundary: the test
asks >= 99.9% identical bf16 results and no difference above one (silu) or
two (silu * up) bf16 steps.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _bf16_steps(a, b):
    """Distance in bf16 steps between two arrays of bf16-valued floats."""
    ai = a.astype(np.float32).view(np.int32) >> 16
    bi = b.astype(np.float32).view(np.int32) >> 16
    # map sign-magnitude to a monotone integer line
    ai = np.where(ai < 0, -(ai & 0x7FFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFF), bi)
    return np.abs(ai.astype(np.int64) - bi.astype(np.int64))


def test_rms_norm_dropin_kats_and_random(ncm, oracle, cuda):
    from ncmorph_amd import kernels

    # root.zig:789-797 constant vector.
    y = np.empty(4, np.float32)
    kernels.rms_norm_bf16(np.full(4, 3, np.float32), np.ones(4, np.float32), y, 0.0)
    assert y.tolist() == [1, 1, 1, 1]
    # The cascade KAT input (root.zig:799-812) through the full op, and
    # random vectors whose lengths reach every cascade level and tail.
    kat = ((np.arange(896) * 17) % 101 + 1).astype(np.float32) * np.float32(0.125)
    rng = np.random.default_rng(3)
    cases = [kat] + [rng.standard_normal(n).astype(np.float32)
                     for n in (1, 11, 17, 896, 2048, 8 * 4 * 256 + 11, 8 * 4 * 4096 + 37)]
    for x in cases:
        w = (rng.standard_normal(x.size) * 0.1 + 1).astype(np.float32)
        y = np.empty_like(x)
        kernels.rms_norm_bf16(x, w, y, 1e-5)
        ref = oracle.rms_norm(x, w, 1e-5, bf16=True)
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), x.size


@pytest.mark.parametrize("rows,width", [(64, 2048), (5, 11), (3, 2050), (4096, 2048),
                                        (3, 6144), (3, 8192), (2, 16384), (2, 8204),
                                        (8193, 2048), (8224, 4096), (8194, 11), (9, 1024),
                                        (8195, 1024)])
def test_rms_norm_rows_device(ncm, oracle, cuda, rows, width):
    """Every row bit-identical to the oracle, in both modes. Widths 1024,
    2048 and 4096 run one row per wavefront held in registers; the others
    read the row twice, and above 8192 rows run two rows per wavefront
    (8193: the last wavefront's second row absent)."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(rows * 31 + width)
    # Hidden states hold bf16 values in the decoder (bf16 mode).
    x = oracle.round_bf16(rng.standard_normal((rows, width)).astype(np.float32) * 3)
    w = oracle.round_bf16((rng.standard_normal(width) * 0.1 + 1).astype(np.float32))
    xd, wd = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
    y32 = kernels.rms_norm_rows(xd, wd, 1e-5)
    y16 = kernels.rms_norm_rows(xd, wd, 1e-5, out_mode="bf16")
    torch.cuda.synchronize()
    sample = range(rows) if rows <= 64 or rows > 8192 else [0, 1, rows // 2, rows - 1]
    y32n = y32.cpu().numpy()
    for r in sample:
        ref = oracle.rms_norm(x[r], w, 1e-5, bf16=True)
        assert np.array_equal(y32n[r].view(np.uint32), ref.view(np.uint32)), r
    bits = y16.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16
    assert np.array_equal(bits, y32n.view(np.uint32))
    # The f32 mode (rms_norm, root.zig:226-239) on unrounded inputs.
    xf = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
    yf = kernels.rms_norm_rows(torch.from_numpy(xf).to(cuda), wd, 1e-5, out_mode="f32")
    yfn = yf.cpu().numpy()
    for r in sample:
        ref = oracle.rms_norm(xf[r], w, 1e-5, bf16=False)
        assert np.array_equal(yfn[r].view(np.uint32), ref.view(np.uint32)), r


def test_silu_dropin(ncm, oracle, cuda):
    from ncmorph_amd import kernels

    y = np.empty(1, np.float32)
    kernels.silu_bf16(np.zeros(1, np.float32), y)  # root.zig:781-787
    assert y[0] == 0.0
    rng = np.random.default_rng(5)
    x = ((rng.random(1 << 16, dtype=np.float32) * 2 - 1) * 12).astype(np.float32)
    y = np.empty_like(x)
    kernels.silu_bf16(x, y)
    ref = oracle.silu_bf16(x)
    steps = _bf16_steps(y, ref)
    assert np.mean(steps == 0) >= 0.999 and steps.max() <= 1


def test_silu_mul_device(ncm, oracle, cuda):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(6)
    n = 4096 * 64 + 3
    g = oracle.round_bf16((rng.standard_normal(n) * 2).astype(np.float32))
    u = oracle.round_bf16(rng.standard_normal(n).astype(np.float32))
    gd, ud = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    y = kernels.silu_mul(gd, ud).cpu().numpy()
    yb = kernels.silu_mul(gd, ud, out_mode="bf16").cpu().view(torch.int16).numpy()
    ref = oracle.silu_mul_bf16(g, u)
    steps = _bf16_steps(y, ref)
    assert np.mean(steps == 0) >= 0.999 and steps.max() <= 2
    assert np.array_equal(yb.view(np.uint16).astype(np.uint32) << 16, y.view(np.uint32))


def _same_bits_or_both_nan(a, b):
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(nan | (a.view(np.uint32) == b.view(np.uint32))))


@pytest.mark.parametrize("width", [2048, 8192, 16384])
def test_rms_norm_rows_special_values(ncm, oracle, cuda, width):
    """Rows whose rounding inputs are subnormal (tiny x, tiny weights), and
    rows holding a NaN, an infinity or both signs of infinity, bit for bit
    against the oracle (NaN rows: NaN where the oracle has NaN), at widths
    from the decoder's to past the largest hidden size."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(width)
    base = rng.standard_normal(width).astype(np.float32)
    rows = [base * np.float32(1e-39),                      # x subnormal: sum of squares 0
            base * np.float32(1e-20),                      # squares subnormal
            base.copy(), base.copy(), base.copy(), base.copy()]
    rows[3][7] = np.nan
    rows[4][5] = np.inf
    rows[5][1], rows[5][2] = np.inf, -np.inf
    x = oracle.round_bf16(np.stack(rows).astype(np.float32))
    weights = [oracle.round_bf16((rng.standard_normal(width) * 0.1 + 1).astype(np.float32)),
               oracle.round_bf16((rng.standard_normal(width) * 1e-38).astype(np.float32))]
    for w in weights:
        xd, wd = torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda)
        y = kernels.rms_norm_rows(xd, wd, 1e-5).cpu().numpy()
        for r in range(x.shape[0]):
            ref = oracle.rms_norm(x[r], w, 1e-5, bf16=True)
            assert _same_bits_or_both_nan(y[r], ref), r


def test_silu_mul_special_values(ncm, oracle, cuda):
    """round(silu_bf16(gate) * up) with up around 1e-39 (subnormal products
    and roundings), gate at +-inf, large magnitudes and NaN: within the SiLU
    test's step bound of the oracle, NaN exactly where the oracle has NaN."""
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(8)
    n = 4096
    g = oracle.round_bf16((rng.standard_normal(n) * 3).astype(np.float32))
    u = oracle.round_bf16((rng.standard_normal(n) * 1e-39).astype(np.float32))
    g[:8] = [np.inf, -np.inf, np.nan, 1e30, -1e30, 0.0, -0.0, 88.0]
    u[8:16] = [np.inf, -np.inf, np.nan, 1e30, 0.0, -0.0, 1e-45, 3e-38]
    gd, ud = torch.from_numpy(g).to(cuda), torch.from_numpy(u).to(cuda)
    y = kernels.silu_mul(gd, ud).cpu().numpy()
    ref = oracle.silu_mul_bf16(g, u)
    assert np.array_equal(np.isnan(y), np.isnan(ref))
    ok = ~np.isnan(ref)
    steps = _bf16_steps(y[ok], ref[ok])
    assert steps.max() <= 2 and np.mean(steps == 0) >= 0.99
