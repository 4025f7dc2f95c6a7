"""Pins the oracle's linear (packages/kernels/root.zig:25-148) with the
reference's own known-answer tests, bit for bit, and the D53 bound
(PROJECT.md:506) against f64."""
import numpy as np


def kat_inputs():
    # root.zig:713-730: closed-form modular inputs, T=4, in=1536, out=576.
    T, K, N = 4, 1536, 576
    t = np.arange(T)[:, None]
    i = np.arange(K)[None, :]
    x = (((t * 29 + i * 37) % 251) - 125).astype(np.float32) / np.float32(128.0)
    o = np.arange(N)[:, None]
    w = (((o * 17 + i * 11) % 257) - 128).astype(np.float32) / np.float32(128.0)
    return x, w


def test_kat_digest_and_values(oracle):
    # root.zig:707-744
    x, w = kat_inputs()
    y = oracle.matmul_bf16(x, w)
    assert oracle.digest(y) == 0x547F69F667C8103F
    flat = y.ravel()
    assert flat[0] == np.float32(-0.466796875)
    assert flat[1] == np.float32(1.109375)
    assert flat[1793] == np.float32(-0.796875)


def test_kat_flush_subnormal_products(oracle):
    # root.zig:746-755
    v = np.float32(5.421010862427522e-20)
    y = oracle.matmul_bf16(np.array([[v, v]], np.float32), np.array([[v, v]], np.float32))
    assert y[0, 0] == 0.0


def test_kat_k_block_partials(oracle):
    # root.zig:757-770: 512-wide K blocks change the bf16 result.
    x = np.full((1, 576), 5.960464477539063e-8, np.float32)
    x[0, 0] = 1.0
    x[0, -1] = 0.00390625
    y = oracle.matmul_bf16(x, np.ones((1, 576), np.float32))
    assert y[0, 0] == np.float32(1.0078125)


def test_kat_hand_computed(oracle):
    # root.zig:684-695
    y = oracle.matmul_reference(np.array([[5, 6], [7, 8]], np.float32),
                                np.array([[1, 2], [3, 4]], np.float32))
    assert y.ravel().tolist() == [17, 39, 23, 53]


def test_matmul_reference_d53_bound(oracle):
    # root.zig:697-705 shapes; |got - f64| <= (in + 1) 2^-24 sum|x w|.
    rng = np.random.default_rng(0xB12026)
    for T, K, N in [(1, 35, 4), (3, 7, 5), (2, 1, 3), (33, 35, 34)]:
        x = (rng.random((T, K), dtype=np.float32) * 2 - 1).astype(np.float32)
        w = (rng.random((N, K), dtype=np.float32) * 2 - 1).astype(np.float32)
        got = oracle.matmul_reference(x, w)
        ref, asum = oracle.matmul_f64(x, w)
        assert np.all(np.abs(got - ref) <= (K + 1) * 2.0**-24 * asum)


def test_matmul_bf16_sum_d53_bound(oracle):
    # The pre-rounding fp32 sum of the pair-FMA emulation obeys the same bound
    # against f64 on the bf16-rounded operands (products of bf16 are exact).
    rng = np.random.default_rng(7)
    for T, K, N in [(3, 2048, 17), (2, 1100, 9), (5, 513, 4), (1, 7, 3)]:
        x = oracle.round_bf16(rng.standard_normal((T, K)).astype(np.float32))
        w = oracle.round_bf16((rng.standard_normal((N, K)) * 0.02).astype(np.float32))
        y, s = oracle.matmul_bf16(x, w, want_sum=True)
        ref, asum = oracle.matmul_f64(x, w)
        assert np.all(np.abs(s - ref) <= (K + 1) * 2.0**-24 * asum)
        assert np.array_equal(y, oracle.round_bf16(s))


def test_bias_added_before_rounding(oracle):
    # root.zig:138: round_bf16(bias) is added to the fp32 sum, then one rounding.
    x = np.array([[1.0, 2.0]], np.float32)
    w = np.array([[0.5, 0.25], [1.0, 1.0]], np.float32)
    b = np.array([0.00390625, 1.0000001], np.float32)
    y, s = oracle.matmul_bf16(x, w, bias=b, want_sum=True)
    assert s[0, 0] == np.float32(1.0 + 0.00390625)
    assert s[0, 1] == np.float32(3.0 + 1.0)
    assert y[0, 0] == np.float32(1.0)  # 1.00390625 is a tie -> even
    assert y[0, 1] == np.float32(4.0)


def test_u16_path_matches_f32_path(oracle):
    rng = np.random.default_rng(3)
    x = oracle.round_bf16(rng.standard_normal((4, 300)).astype(np.float32))
    w = oracle.round_bf16(rng.standard_normal((6, 300)).astype(np.float32))
    y, s = oracle.matmul_bf16(x, w, want_sum=True)
    y2, s2 = oracle.matmul_bf16_u16_rows(oracle.bf16_from_f32(x), oracle.bf16_from_f32(w), 0, 4)
    assert np.array_equal(y, y2) and np.array_equal(s, s2)


def test_threaded_matmul_is_bit_identical(oracle):
    """The column-split threaded matmul gives the single-threaded bits."""
    rng = np.random.default_rng(9)
    x = oracle.round_bf16(rng.standard_normal((7, 2050)).astype(np.float32))
    w = oracle.round_bf16(rng.standard_normal((301, 2050)).astype(np.float32))
    b = oracle.round_bf16(rng.standard_normal(301).astype(np.float32))
    one = oracle.matmul_bf16(x, w, b)
    prev = oracle.set_threads(5)
    try:
        many = oracle.matmul_bf16(x, w, b)
    finally:
        oracle.set_threads(prev)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32))
