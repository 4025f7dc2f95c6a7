"""Pins the oracle's RVQ restatement. The reference has no RVQ code or test
(ROADMAP.md:257-259), so every check here is fixed by the mathematics:
an independent f64 brute force over a materialized residual, planted codes
that must be recovered exactly, the lowest-index tie rule, exact pooling of
repeated blocks, error bounds of the fixed-order dot product, and the
decode / reconstruction identity."""
import os

import numpy as np
import pytest

from ncmorph_amd import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rvq_small.npz")


def _cb(rng, levels, v, d, scale=1.0):
    return synth.bf16_bits((rng.standard_normal((levels, v, d)) * scale / np.sqrt(d)).astype(
        np.float32))


def test_dot_fixed_error_bound(oracle):
    rng = np.random.default_rng(1)
    for d in (64, 192, 256, 320, 2048):
        u = rng.standard_normal(d).astype(np.float32)
        c = synth.bf16_bits(rng.standard_normal(d).astype(np.float32))
        cf = synth.bf16_to_f32(c).astype(np.float64)
        got = oracle.lib().ncmo_dot_fixed(u, c, d)
        ref = float(np.dot(u.astype(np.float64), cf))
        bound = (d // 64 + 7) * 2.0**-24 * float(np.sum(np.abs(u * cf)))
        assert abs(got - ref) <= bound


def test_dot_fixed_order_is_the_stated_one(oracle):
    # Lane j owns elements 4j..4j+3 (+256 m); lanes combine by a halving tree.
    # u[0] = 2^24 and u[1] = 1 share lane 0 (the 1 is absorbed: ties to even);
    # u[4] and u[12] sit in lanes 1 and 3, meet at tree offset 2 (sum 2) and
    # join lane 0 at offset 1: 2^24 + 2. A sequential sum gives 2^24, the
    # correctly rounded sum 2^24 + 4, and a lane-per-element (i mod 64)
    # assignment 2^24 + 4, so only the stated order yields 2^24 + 2.
    d = 256
    u = np.zeros(d, np.float32)
    c = synth.bf16_bits(np.ones(d, np.float32))
    u[0], u[1], u[4], u[12] = 2.0**24, 1.0, 1.0, 1.0
    got = oracle.lib().ncmo_dot_fixed(u, c, d)
    assert got == np.float32(2.0**24 + 2.0)
    assert np.float32(np.sum(u.astype(np.float64))) == np.float32(2.0**24 + 4.0)


def test_csq_matches_f64(oracle):
    rng = np.random.default_rng(2)
    cb = _cb(rng, 2, 33, 256)
    csq = oracle.rvq_csq(cb)
    ref = np.sum(synth.bf16_to_f32(cb).astype(np.float64) ** 2, axis=-1)
    assert np.allclose(csq, ref, rtol=2e-6, atol=0)


def _check_against_f64(oracle, x, cb, strides, tol=1e-6):
    """Codes equal the f64 brute force except where the f64 top-2 relative
    gap is below tol; the f64 run is teacher-forced with the oracle's codes so
    a near-tie cannot change later levels."""
    r = oracle.rvq_encode(x, cb, strides)
    codes64, gap64 = oracle.rvq_encode_f64(x, cb, strides, forced=r["codes"])
    diff = r["codes"] != codes64
    assert np.all(gap64[diff] < tol), (np.sum(diff), gap64[diff])
    # Gaps agree where they are not ties.
    ok = gap64 > 1e-3
    assert np.allclose(r["gap"][ok], gap64[ok], rtol=1e-3)
    return r, int(np.sum(diff)), int(np.sum(gap64 < 1e-5))


def test_small_config_matches_f64(oracle):
    c = synth.RVQ_SMALL
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    r, ndiff, nties = _check_against_f64(oracle, x, cb, c["strides"])
    assert ndiff == 0


def test_multiscale_matches_f64(oracle):
    rng = np.random.default_rng(3)
    strides = (16, 8, 4, 2, 1)
    x = rng.standard_normal((2, 64, 128)).astype(np.float32)
    cb = _cb(rng, len(strides), 96, 128)
    _check_against_f64(oracle, x, cb, strides)


def test_multiscale_skipping_strides_matches_f64(oracle):
    rng = np.random.default_rng(4)
    strides = (32, 32, 4, 1, 1)
    x = rng.standard_normal((3, 64, 64)).astype(np.float32)
    cb = _cb(rng, len(strides), 40, 64)
    _check_against_f64(oracle, x, cb, strides)


def test_planted_codes_recovered(oracle):
    # x = sum over levels of repeat(C_l[k_l]) with geometrically shrinking
    # codebooks; every level's code must come back exactly, and the
    # reconstruction equals x bit for bit (same summation order).
    rng = np.random.default_rng(5)
    strides = (8, 4, 2, 1)
    B, T, d, V = 2, 32, 64, 50
    cb = np.stack([_cb(rng, 1, V, d, scale=4.0 ** -l)[0] for l in range(4)])
    cbf = synth.bf16_to_f32(cb)
    total = sum(T // s for s in strides)
    planted = np.zeros((B, total), np.int32)
    x = np.zeros((B, T, d), np.float32)
    off = 0
    for l, s in enumerate(strides):
        k = rng.integers(0, V, size=(B, T // s)).astype(np.int32)
        planted[:, off:off + T // s] = k
        x = x + cbf[l][np.repeat(k, s, axis=1)]
        off += T // s
    r = oracle.rvq_encode(x, cb, strides)
    assert np.array_equal(r["codes"], planted)
    assert np.array_equal(r["recon"], x)


def test_tie_breaks_to_lowest_index(oracle):
    rng = np.random.default_rng(6)
    d, V = 64, 16
    cb = _cb(rng, 1, V, d)
    cb[0, 9] = cb[0, 3]
    cb[0, 12] = cb[0, 3]
    x = synth.bf16_to_f32(cb[0, 3])[None, None, :].astype(np.float32)
    r = oracle.rvq_encode(x, cb, (1,))
    assert r["codes"][0, 0] == 3
    assert r["gap"][0, 0] == 0.0


def test_pooling_of_repeated_blocks_is_exact(oracle):
    # A residual that is constant over each stride block pools to itself, so
    # with a zero second level the level-0 input equals the block value.
    rng = np.random.default_rng(7)
    d, V = 64, 8
    blocks = rng.standard_normal((1, 4, d)).astype(np.float32)
    x = np.repeat(blocks, 16, axis=1)
    cb = _cb(rng, 1, V, d)
    rows = np.arange(4, dtype=np.int64)
    csq = oracle.rvq_csq(cb)
    _, _, u = oracle.rvq_level_rows(x, cb, (16,), csq, np.zeros((1, 4), np.int32), 0, rows,
                                    want_u=True)
    assert np.array_equal(u, blocks[0])


def test_pyramid_mean_close_to_exact_mean(oracle):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((1, 128, 64)).astype(np.float32)
    cb = _cb(rng, 1, 4, 64)
    csq = oracle.rvq_csq(cb)
    _, _, u = oracle.rvq_level_rows(x, cb, (128,), csq, np.zeros((1, 1), np.int32), 0,
                                    np.array([0], np.int64), want_u=True)
    ref = x[0].astype(np.float64).mean(axis=0)
    assert np.all(np.abs(u[0] - ref) <= 8 * 2.0**-24 * np.abs(x[0]).max() * 1.0)


def test_decode_matches_encode_recon(oracle):
    rng = np.random.default_rng(9)
    strides = (4, 2, 1)
    x = rng.standard_normal((2, 16, 64)).astype(np.float32)
    cb = _cb(rng, 3, 20, 64)
    r = oracle.rvq_encode(x, cb, strides)
    rec = oracle.rvq_decode(r["codes"], cb, strides, 16)
    assert np.array_equal(rec, r["recon"])
    # Residual energy never increases across levels for this data.
    assert np.linalg.norm(x - r["recon"]) < np.linalg.norm(x)


def test_level_rows_agrees_with_encode(oracle):
    rng = np.random.default_rng(10)
    strides = (8, 4, 2, 1)
    x = rng.standard_normal((2, 32, 64)).astype(np.float32)
    cb = _cb(rng, 4, 24, 64)
    r = oracle.rvq_encode(x, cb, strides)
    csq = oracle.rvq_csq(cb)
    off = 0
    for l, s in enumerate(strides):
        n = 2 * (32 // s)
        rows = np.arange(n, dtype=np.int64)
        codes, gap = oracle.rvq_level_rows(x, cb, strides, csq, r["codes"], l, rows)
        want = r["codes"][:, off:off + 32 // s].ravel()
        assert np.array_equal(codes, want)
        off += 32 // s


def test_teacher_forcing_uses_forced_codes(oracle):
    rng = np.random.default_rng(11)
    strides = (2, 1)
    x = rng.standard_normal((1, 8, 64)).astype(np.float32)
    cb = _cb(rng, 2, 12, 64)
    r = oracle.rvq_encode(x, cb, strides)
    forced = r["codes"].copy()
    forced[0, :4] = (forced[0, :4] + 1) % 12
    f = oracle.rvq_encode(x, cb, strides, forced=forced)
    assert np.array_equal(f["codes"][0, :4], r["codes"][0, :4])  # level 0 unchanged
    codes64, _ = oracle.rvq_encode_f64(x, cb, strides, forced=forced)
    assert np.array_equal(f["codes"], codes64)


def test_invalid_strides_rejected(oracle):
    x = np.zeros((1, 8, 64), np.float32)
    cb = np.zeros((2, 4, 64), np.uint16)
    for bad in [(1, 2), (3, 1), (16, 1), (0, 1)]:
        with pytest.raises(ValueError):
            oracle.rvq_encode(x, cb, bad)


def test_golden_fixture(oracle):
    import hashlib

    g = np.load(GOLDEN)
    c = synth.RVQ_SMALL
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    assert hashlib.sha256(x.tobytes()).digest() == g["x_sha256"].tobytes()
    assert hashlib.sha256(cb.tobytes()).digest() == g["cb_sha256"].tobytes()
    r = oracle.rvq_encode(x, cb, c["strides"])
    assert np.array_equal(r["codes"].reshape(4, 128), g["codes"])
    assert hashlib.sha256(r["recon"].tobytes()).digest() == g["recon_sha256"].tobytes()
