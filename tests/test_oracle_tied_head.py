"""The NCM codebook-tied head restated in the oracle (PROJECT.md:222; the
reference has no code for it), pinned by what the mathematics fixes: a
closed form on an orthogonal codebook, argmax = the nearest code of the RVQ
oracle's exhaustive fixed-order search, and the scale / bias composition."""
import numpy as np

from ncmorph_amd import synth


def test_orthogonal_codebook_closed_form(oracle):
    d, v = 16, 8
    a = np.arange(1, v + 1, dtype=np.float64)
    E = np.zeros((v, d))
    E[np.arange(v), np.arange(v)] = a          # E_k = a_k e_k
    z = np.zeros((3, d))
    z[0, 2] = 5.0                              # along code 2
    z[1, 7] = -1.0
    z[2, 12] = 3.0                             # orthogonal to every code
    got, _ = oracle.tied_head_logits_f64(z, E, log_inv_t=np.log(2.0))
    mean = np.mean(a * a)
    want = (-a[None, :] ** 2) * np.ones((3, 1))
    want[0, 2] += 2 * 5.0 * a[2]
    want[1, 7] += 2 * -1.0 * a[7]
    assert np.allclose(got, want * 2.0 / mean, rtol=1e-14, atol=0)


def test_argmax_is_the_nearest_code(oracle):
    rng = np.random.default_rng(5)
    rows, d, v = 96, 64, 300
    x, cb_bits = synth.rvq_inputs(5, 1, rows, d, 1, v)
    zb = synth.bf16_bits(x.reshape(rows, d))
    z = synth.bf16_to_f32(zb)
    E = synth.bf16_to_f32(cb_bits[0])
    logits, _ = oracle.tied_head_logits_f64(z, E, log_inv_t=rng.standard_normal())
    enc = oracle.rvq_encode(z.reshape(1, rows, d), cb_bits, (1,), threads=4)
    codes = enc["codes"][0]
    top2 = np.sort(logits, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 1e-9 * np.abs(top2[:, 1])
    assert clear.mean() > 0.95
    assert np.array_equal(np.argmax(logits, axis=1)[clear], codes[clear])


def test_scale_and_bias_compose(oracle):
    rng = np.random.default_rng(6)
    z = rng.standard_normal((5, 24))
    E = rng.standard_normal((40, 24))
    b = rng.standard_normal(40)
    base, _ = oracle.tied_head_logits_f64(z, E)
    scaled, _ = oracle.tied_head_logits_f64(z, E, log_inv_t=0.5, bias=b)
    assert np.allclose(scaled, base * np.exp(0.5) + b, rtol=1e-13, atol=1e-13)
