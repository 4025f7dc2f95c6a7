"""Pins of the oracle's NCM level-parallel body (src/ncm_model.zig:89-250)
and its helpers (src/ncm_position.zig, src/ncm_norm.zig, the post-upsample
Conv1d): the reference's own tests restated, closed forms, and an
independent f64 forward whose bound tells the right composition from
planted mistakes."""
import numpy as np
import pytest

from .ncm_f64 import ncm_forward_f64, random_ncm


def _reference_case():
    """The configuration and weights of the reference's test "NCM forward
    uses EOS prefix, level embeddings and learned level-0 queries"
    (src/ncm_model.zig:332-429)."""
    cfg = dict(hidden_size=4, vq_width=2, num_attention_heads=2, num_key_value_heads=1,
               head_dim=2, intermediate_size=3, rms_norm_epsilon=1e-5, rope="default",
               rope_theta=10000.0, level_lengths=[1, 2], prefix_length=1, query_level0=True)
    f = lambda v: np.asarray(v, np.float32)
    fused = f([((i % 9) - 4) * 0.025 for i in range(32)])
    layer = dict(
        fused_qkv_weight=fused.reshape(8, 4),
        output_weight=f([0.1, 0.2, -0.1, 0.05, -0.2, 0.1, 0.15, -0.05,
                         0.05, -0.1, 0.2, 0.1, -0.1, 0.05, 0.1, 0.2]).reshape(4, 4),
        query_norm_weight=f([1, 1]), key_norm_weight=f([1, 1]),
        ln_1_weight=f([1, 1, 1, 1]), ln_2_weight=f([1, 1, 1, 1]),
        gate_weight=f([0.1, -0.1, 0.2, 0.05, -0.05, 0.1, -0.2, 0.15, 0.05, 0.2, 0.1,
                       -0.1]).reshape(3, 4),
        up_weight=f([0.1, 0.05, -0.1, 0.15, -0.2, 0.1, 0.1, 0.2, -0.05, 0.1, -0.1,
                     0.05]).reshape(3, 4),
        down_weight=f([0.1, -0.1, 0.05, 0.2, 0.1, -0.05, -0.2, 0.15, 0.1, -0.1, 0.05,
                       0.1]).reshape(4, 3),
    )
    weights = dict(
        prefix_token_embedding=f([0.1, -0.2, 0.3, 0.2, -0.4, 0.5]).reshape(3, 2),
        prefix_vocab_size=3,
        input_projection=f([0.2, -0.1, -0.3, 0.4, 0.1, 0.2, -0.2, 0.3]).reshape(4, 2),
        input_projection_bias=f([0.01, -0.02, 0.03, -0.04]),
        level_embedding=f([0.01, 0.02, -0.02, 0.03, -0.03, 0.01, 0.02, -0.01]).reshape(2, 4),
        l0_queries=f([0.4, -0.3]).reshape(1, 2),
        final_norm_weight=f([1, 1, 1, 1]),
        layers=[layer, layer],
    )
    return cfg, weights


@pytest.mark.parametrize("bf16", [False, True])
def test_reference_ncm_forward_invariants(oracle, bf16):
    """src/ncm_model.zig:332-429: level-0 inputs are replaced by the learned
    queries; the queries, the level embeddings and the prefix table each
    change the output; a fully padded prefix still gives finite values."""
    cfg, w = _reference_case()
    ids, pad = [2], [False]
    target = np.asarray([99, -99, 0.1, 0.2, -0.3, 0.4], np.float32)
    changed_l0 = np.asarray([-33, 44, 0.1, 0.2, -0.3, 0.4], np.float32)
    run = lambda ww, tgt, p=pad: oracle.ncm_forward(cfg, ww, ids, p, tgt, bf16=bf16)
    out = run(w, target)
    assert out.shape == (4, 4)
    assert np.array_equal(out, run(w, changed_l0))
    w2 = dict(w, l0_queries=w["l0_queries"] + np.float32([[0.5, 0]]))
    assert not np.array_equal(out, run(w2, target))
    emb = w["level_embedding"].copy()
    emb.flat[4] += 0.5
    assert not np.array_equal(out, run(dict(w, level_embedding=emb), target))
    table = w["prefix_token_embedding"].copy()
    table.flat[4] += 1
    assert not np.array_equal(out, run(dict(w, prefix_token_embedding=table), target))
    assert np.all(np.isfinite(run(w, target, [True])))


def test_reference_errors(oracle):
    cfg, w = _reference_case()
    t = np.zeros(6, np.float32)
    with pytest.raises(ValueError, match="InvalidPrefixLength"):
        oracle.ncm_forward(cfg, w, [1, 2], [], t)
    with pytest.raises(ValueError, match="InvalidPrefixMask"):
        oracle.ncm_forward(cfg, w, [1], [False, True], t)
    with pytest.raises(ValueError, match="InvalidNcmTensorSize"):
        oracle.ncm_forward(cfg, w, [1], [], t[:4])
    with pytest.raises(ValueError, match="PrefixTokenOutOfRange"):
        oracle.ncm_forward(cfg, w, [3], [], t)
    with pytest.raises(ValueError, match="InvalidNcmDimensions"):
        oracle.ncm_forward(dict(cfg, head_dim=3), w, [1], [], t)


def test_level_positions_restart(oracle):
    # src/ncm_position.zig:152-158
    assert list(oracle.fill_level_positions(2, [1, 2, 3])) == [0, 1, 0, 0, 1, 0, 1, 2]


def test_llama3_tables_at_restarting_positions(oracle):
    # src/ncm_position.zig:120-150: every gathered row is the row of the
    # 3-position table at its position.
    positions = [0, 1, 2, 0, 1, 0]
    inv = oracle.rope_llama3(64, 500000.0, 32.0, 1.0, 4.0, 8192)
    c_ref, s_ref = oracle.rope_tables(inv, 3)
    c, s = oracle.tables_at_positions(inv, positions)
    for i, p in enumerate(positions):
        assert np.array_equal(c[i], c_ref[p]) and np.array_equal(s[i], s_ref[p])


def test_norm_rows_match_per_row_kernel(oracle):
    # src/ncm_norm.zig:51-75 (rows of 17, two epsilons), plus the bias add.
    rng = np.random.default_rng(0x4E434D32)
    x = (rng.random((3, 17)) * 2 - 1).astype(np.float32)
    w = (rng.random(17) * 2 - 1).astype(np.float32)
    b = (rng.random(17) * 2 - 1).astype(np.float32)
    for eps in (1e-5, 1e-6):
        got = oracle.rms_norm_rows_with_bias(x, w, None, eps, bf16=False)
        want = np.stack([oracle.rms_norm(x[r], w, eps, bf16=False) for r in range(3)])
        assert np.array_equal(got, want)
        got_b = oracle.rms_norm_rows_with_bias(x, w, b, eps, bf16=False)
        assert np.array_equal(got_b, (want + b[None, :]).astype(np.float32))
        got_bf = oracle.rms_norm_rows_with_bias(x, w, b, eps, bf16=True)
        want_bf = oracle.round_bf16(oracle.rms_norm(x, w, eps, bf16=True) + b[None, :])
        assert np.array_equal(got_bf, want_bf)


def test_post_upsample_conv(oracle):
    # Zero kernel: output = input + bias, exactly.
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 4)).astype(np.float32)
    b = rng.standard_normal(4).astype(np.float32)
    got = oracle.post_upsample_conv(x, np.zeros((4, 4, 3), np.float32), b)
    assert np.array_equal(got, (x + b[None, :]).astype(np.float32))
    # One channel, small integers: value[p] = w0 x[p-1] + w1 x[p] + w2 x[p+1]
    # with the edge taps skipped (exact in fp32).
    x1 = np.asarray([[1], [2], [3], [4]], np.float32)
    w1 = np.asarray([[[2, 3, 5]]], np.float32)
    got = oracle.post_upsample_conv(x1, w1, np.zeros(1, np.float32))
    want = [1 + (3 * 1 + 5 * 2), 2 + (2 * 1 + 3 * 2 + 5 * 3), 3 + (2 * 2 + 3 * 3 + 5 * 4),
            4 + (2 * 3 + 3 * 4)]
    assert got.ravel().tolist() == want
    # Random case against f64 of the same formula, within the fp32 bound of
    # a (3 width + 1)-term sum; a transposed kernel layout fails it.
    x = rng.standard_normal((9, 16)).astype(np.float32)
    w = rng.standard_normal((16, 16, 3)).astype(np.float32) * np.float32(0.1)
    got = oracle.post_upsample_conv(x, w, b[:1].repeat(16))

    def f64(wk):
        xp = np.concatenate([np.zeros((1, 16)), x, np.zeros((1, 16))]).astype(np.float64)
        v = float(b[0]) + sum(xp[k:k + 9] @ wk[:, :, k].T.astype(np.float64) for k in range(3))
        mag = abs(float(b[0])) + sum(np.abs(xp[k:k + 9]) @ np.abs(wk[:, :, k]).T for k in range(3))
        return x + v, mag

    want, mag = f64(w)
    assert np.all(np.abs(got - want) <= (3 * 16 + 2) * 2.0 ** -24 * (mag + np.abs(x)))
    wrong, _ = f64(np.ascontiguousarray(w.transpose(1, 0, 2)))
    assert np.max(np.abs(got - wrong)) > 1e-3


def test_block_causal_mask(oracle):
    levels, P = [2, 3, 1], 3
    pad = [False, True, False]
    m = oracle.block_causal_mask(P, levels, pad)
    d = oracle.block_diagonal_mask(P, levels, pad)
    level_of = np.concatenate([np.full(P, -1)] + [np.full(n, l) for l, n in enumerate(levels)])
    S = P + sum(levels)
    for q in range(S):
        for k in range(S):
            if k < P:
                want = not pad[k]
            else:
                want = level_of[q] >= 0 and level_of[k] <= level_of[q]
            assert m[q, k] == want, (q, k)
    # It contains the block-diagonal mask, and differs only below the diagonal blocks.
    assert np.all(m >= d)
    assert np.all((m > d) <= (level_of[None, :] < level_of[:, None]))


def _cfg(levels, P, hidden, vq, hq, hkv, hd, inter):
    return dict(hidden_size=hidden, vq_width=vq, num_attention_heads=hq, num_key_value_heads=hkv,
                head_dim=hd, intermediate_size=inter, rms_norm_epsilon=1e-5,
                level_lengths=levels, prefix_length=P, query_level0=True, rope="default",
                rope_theta=10000.0)


@pytest.mark.parametrize("bf16,mask,extras", [
    (False, "block_diagonal", {}),
    (True, "block_diagonal", {}),
    (True, "block_causal", dict(biases=True)),
    (True, "block_diagonal", dict(qk_norm=True, convs=True)),
    (False, "block_causal", dict(qk_norm=True, convs=True, biases=True)),
])
def test_oracle_ncm_against_f64(oracle, bf16, mask, extras):
    """f32 mode (the reference's arithmetic) within 1e-4 of f64 and bf16
    mode within 2% (bf16 roundings through two layers); the bounds separate
    the composition from planted mistakes (restarting positions only in f32
    mode, where their effect is above the bound at these lengths)."""
    rng = np.random.default_rng(41 + 3 * bf16 + len(extras))
    levels, P = [4, 8, 16], 5
    hidden, vq, hq, hkv, hd, inter = 128, 64, 4, 2, 32, 256
    cfg = _cfg(levels, P, hidden, vq, hq, hkv, hd, inter)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, 2, levels, P, 11,
                   **extras)
    ids = rng.integers(0, 11, P)
    pad = [False, False, True, False, True]
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    got = oracle.ncm_forward(cfg, w, ids, pad, tgt, bf16=bf16, mask=mask)
    mk = (oracle.block_causal_mask if mask == "block_causal" else oracle.block_diagonal_mask)(
        P, levels, pad).astype(bool)
    cfg64 = dict(cfg, inv_freq=oracle.rope_default_frequencies(hd, 10000.0))
    ref = ncm_forward_f64(cfg64, w, ids, tgt, mk)
    scale = np.max(np.abs(ref))
    tol = (0.02 if bf16 else 1e-4) * scale
    assert np.max(np.abs(got - ref)) <= tol, np.max(np.abs(got - ref)) / scale
    for mistake in ("level", "l0") + (() if bf16 else ("positions",)):
        wrong = ncm_forward_f64(cfg64, w, ids, tgt, mk, skip=mistake)
        assert np.max(np.abs(wrong - ref)) > 2 * tol, mistake
    other = (oracle.block_diagonal_mask if mask == "block_causal" else oracle.block_causal_mask)(
        P, levels, pad).astype(bool)
    assert np.max(np.abs(ncm_forward_f64(cfg64, w, ids, tgt, other) - ref)) > 2 * tol


def test_oracle_ncm_trace_layout(oracle):
    cfg, w = _reference_case()
    tgt = np.asarray([99, -99, 0.1, 0.2, -0.3, 0.4], np.float32)
    out, states = oracle.ncm_forward(cfg, w, [2], [False], tgt, trace=True)
    # [layers + 1] states: the input stage, each layer but the last, then
    # the final-normalized output (src/ncm_model.zig:169-172, 242-249).
    assert len(states) == 3 and np.array_equal(states[-1], out)
    assert not np.array_equal(states[0], states[1])


@pytest.mark.parametrize("bf16", [False, True])
def test_oracle_ncm_stages_compose_to_the_body(oracle, bf16):
    """ncm_input_stage, ncm_layer on each state and ncm_final_norm (the
    stages the device replay tests call one at a time) reproduce
    ncm_forward's traced states bit for bit, in both arithmetic modes."""
    rng = np.random.default_rng(7 + bf16)
    levels, P = [4, 8, 16], 5
    hidden, vq, hq, hkv, hd, inter = 128, 64, 4, 2, 32, 256
    cfg = _cfg(levels, P, hidden, vq, hq, hkv, hd, inter)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, 3, levels, P, 11,
                   biases=True, qk_norm=True, convs=True)
    ids = rng.integers(0, 11, P)
    pad = [False, True, False, False, True]
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    out, states = oracle.ncm_forward(cfg, w, ids, pad, tgt, bf16=bf16, mask="block_causal",
                                     trace=True)
    assert np.array_equal(oracle.ncm_input_stage(cfg, w, ids, tgt, bf16=bf16), states[0])
    cos, sin, m = oracle.ncm_tables_and_mask(cfg, pad, "block_causal")
    h = states[0]
    for l, layer in enumerate(w["layers"]):
        h = oracle.ncm_layer(cfg, layer, h, cos, sin, m, bf16=bf16)
        if l + 1 < len(w["layers"]):
            assert np.array_equal(h, states[l + 1]), l
    assert np.array_equal(oracle.ncm_final_norm(cfg, w, h, bf16=bf16), out)
