"""GPU parity of the fp32 linear against the oracle (restatement of
`kernels.matmul` / `matmul_reference`, packages/kernels/root.zig:25-93).

The reference's own contract for `matmul` (root.zig:697-705 with the check
at :836-865) is |y - y_f64| <= (K + 1) 2^-24 sum|x w| per output; the GPU's
fp32 MFMA sums in another order and is held to the same bound. Against the
oracle (increasing-k fp32 sum) the two bounds add: |y - y_oracle| <=
2 (K + 1) 2^-24 sum|x w|. Small-integer products sum exactly in any order
(root.zig:684-695).
"""
import numpy as np
import pytest

from ncmorph_amd import NcmError

pytestmark = pytest.mark.gpu


def _uniform(rng, shape):
    return (rng.random(shape, dtype=np.float32) * 2 - 1).astype(np.float32)


def _host(x, w):
    from ncmorph_amd import kernels

    y = np.empty((x.shape[0], w.shape[0]), np.float32)
    kernels.matmul(x, w, y, x.shape[0], x.shape[1], w.shape[0])
    return y


def test_kat_hand_computed(ncm, cuda):
    # root.zig:684-695
    x = np.array([[5, 6], [7, 8]], np.float32)
    w = np.array([[1, 2], [3, 4]], np.float32)
    assert _host(x, w).ravel().tolist() == [17, 39, 23, 53]


def test_d53_bound_reference_shapes(ncm, oracle, cuda):
    # The reference's seeded shapes (root.zig:697-705), K not a multiple of 4
    # (the drop-in pads rows with zeros).
    rng = np.random.default_rng(0xB12026)
    for T, K, N in [(1, 35, 4), (3, 7, 5), (2, 1, 3), (33, 35, 34)]:
        x, w = _uniform(rng, (T, K)), _uniform(rng, (N, K))
        got = _host(x, w)
        ref, asum = oracle.matmul_f64(x, w)
        assert np.all(np.abs(got - ref) <= (K + 1) * 2.0**-24 * asum)
        seq = oracle.matmul_reference(x, w)
        assert np.all(np.abs(got - seq) <= 2 * (K + 1) * 2.0**-24 * asum)


@pytest.mark.parametrize("m,k,n", [(300, 520, 260), (129, 4, 257), (64, 2048, 1024),
                                   (1024, 1024, 1024)])
def test_device_linear_f32(ncm, oracle, cuda, m, k, n):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m * 7 + k * 3 + n)
    x, w = rng.standard_normal((m, k)).astype(np.float32), rng.standard_normal((n, k)).astype(np.float32)
    y = kernels.linear_f32(torch.from_numpy(x).to(cuda), torch.from_numpy(w).to(cuda))
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref, asum = oracle.matmul_f64(x, w)
    assert np.all(np.abs(got - ref) <= (k + 1) * 2.0**-24 * asum), float(
        np.max(np.abs(got - ref) / asum))
    rows = sorted({0, m // 2, m - 1})
    seq = oracle.matmul_reference(x[rows], w)
    assert np.all(np.abs(got[rows] - seq) <= 2 * (k + 1) * 2.0**-24 * asum[rows])


def test_drop_in_lengths_and_empty(ncm, cuda):
    from ncmorph_amd import kernels

    x = np.ones((2, 3), np.float32)
    w = np.ones((4, 3), np.float32)
    with pytest.raises(NcmError):
        kernels.matmul(x, w, np.empty((2, 5), np.float32), 2, 3, 4)
    # K = 0: every output is the empty sum.
    y = np.full((2, 4), 7.0, np.float32)
    kernels.matmul(np.empty((2, 0), np.float32), np.empty((4, 0), np.float32), y, 2, 0, 4)
    assert np.all(y == 0)


def test_device_rejects_unaligned_k(ncm, cuda):
    import torch
    from ncmorph_amd import kernels

    x = torch.zeros((4, 6), dtype=torch.float32, device=cuda)
    w = torch.zeros((3, 6), dtype=torch.float32, device=cuda)
    with pytest.raises(NcmError):
        kernels.linear_f32(x, w)
