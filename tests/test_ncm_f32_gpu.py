"""GPU NCM level-parallel body in the reference's own f32 arithmetic
(ncm_ncm_forward_f32_dev) against the oracle's f32 composition
(oracle.ncm_forward with bf16=False: kernels.matmul + bias, f32 RMSNorm with
the norm biases, RoPE at the restarting positions, f32 attention with the
level mask, silu(gate) * up, unrounded adds), which the reference's own
invariant test (src/ncm_model.zig:332-429) and an f64 forward pin.

Bar: the final states within 1e-4 of their largest magnitude: the device
sums the projections on the fp32 MFMA in its own order (the oracle in
increasing k), and its expf differs from Zig's exp in the last bits; the
attention adds in the reference's dimension and key order. The reference's
invariants hold bit for bit on the device."""
import numpy as np
import pytest

from .ncm_f64 import random_ncm

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _ident(a):
    return np.asarray(a, np.float32)


def _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, layers, mask, vocab, window=0,
          query_level0=True):
    return N.NcmSpec(hidden=hidden, vq_width=vq, intermediate=inter, q_heads=hq, kv_heads=hkv,
                     head_dim=hd, layers=layers, level_lengths=tuple(levels), prefix_length=P,
                     prefix_vocab=vocab, query_level0=query_level0, mask=mask, window=window,
                     rope_theta=10000.0, rope_llama3=None)


def _cfg(spec):
    return dict(hidden_size=spec.hidden, vq_width=spec.vq_width,
                num_attention_heads=spec.q_heads, num_key_value_heads=spec.kv_heads,
                head_dim=spec.head_dim, intermediate_size=spec.intermediate,
                rms_norm_epsilon=spec.rms_eps, level_lengths=list(spec.level_lengths),
                prefix_length=spec.prefix_length, query_level0=spec.query_level0,
                rope="default", rope_theta=spec.rope_theta,
                source_causal=spec.mask == "causal", sliding_window=spec.window or None)


def _run(N, torch, cuda, spec, dw, ids, tgt, pad=None):
    cos, sin = N.rope_tables(spec)
    out = N.forward_f32(spec, dw, ids, torch.from_numpy(tgt).to(cuda),
                        torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda),
                        prefix_pad_mask=pad)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = [
    # (mask, head_dim, extras, window, query_level0, pad)
    ("block_diagonal", 64, {}, 0, True, True),
    ("block_causal", 64, dict(biases=True), 0, True, True),
    ("block_diagonal", 128, dict(qk_norm=True, biases=True), 0, False, False),
    ("block_diagonal", 32, dict(convs=True, qk_norm=True, biases=True), 0, True, True),
    ("causal", 64, {}, 0, True, False),
    ("causal", 96, dict(biases=True), 24, True, False),
]


@pytest.mark.parametrize("mask,hd,extras,window,ql0,use_pad", CASES)
def test_ncm_f32_body_matches_oracle(cuda, ncm, oracle, mask, hd, extras, window, ql0, use_pad):
    import torch
    from ncmorph_amd import ncm as N

    print(f"ncm f32 case mask={mask} hd={hd} extras={extras} window={window}", flush=True)
    rng = np.random.default_rng(3 * hd + len(extras) + window)
    levels, P = [8, 16, 32, 64], 12
    hidden, vq, hq, hkv, inter, nl, vocab = 192, 96, 4, 2, 384, 2, 50
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, mask, vocab, window, ql0)
    w = random_ncm(rng, _ident, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   query_level0=ql0, **extras)
    ids = rng.integers(0, vocab, P)
    pad = (rng.random(P) < 0.3) if use_pad else None
    tgt = rng.standard_normal((sum(levels), vq)).astype(np.float32)
    dw = N.device_weights_f32(spec, w, cuda)
    got = _run(N, torch, cuda, spec, dw, ids, tgt, pad)
    ref = oracle.ncm_forward(_cfg(spec), w, ids, pad, tgt, bf16=False,
                             mask="block_diagonal" if mask == "causal" else mask)
    scale = np.max(np.abs(ref))
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    print("max error relative to max|ref|:", err.max() / scale)
    assert err.max() <= TOL * scale, err.max() / scale


def test_ncm_f32_hidden_states_match_oracle(cuda, ncm, oracle):
    """hidden_states in the reference's own arithmetic (forward_with_trace,
    src/ncm_model.zig:169-171, :243-249): [layers + 1, S, hidden], the
    input stage, every layer but the last, then the final-normalized output
    (equal to the body's output bit for bit); each state within TOL of the
    largest magnitude of the oracle's."""
    import torch
    from ncmorph_amd import ncm as N

    rng = np.random.default_rng(29)
    levels, P = [8, 16, 32], 10
    hidden, vq, hq, hkv, hd, inter, nl, vocab = 192, 96, 4, 2, 64, 384, 3, 40
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, "block_diagonal", vocab)
    w = random_ncm(rng, _ident, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   biases=True)
    ids = rng.integers(0, vocab, P)
    tgt = rng.standard_normal((sum(levels), vq)).astype(np.float32)
    dw = N.device_weights_f32(spec, w, cuda)
    cos, sin = N.rope_tables(spec)
    args = (spec, dw, ids, torch.from_numpy(tgt).to(cuda), torch.from_numpy(cos).to(cuda),
            torch.from_numpy(sin).to(cuda))
    plain = N.forward_f32(*args)
    out, states = N.forward_f32(*args, hidden_states=True)
    torch.cuda.synchronize()
    assert states.shape == (nl + 1, spec.seq_len, hidden)
    assert torch.equal(plain, out)
    assert torch.equal(states[nl], out)
    _, ref_states = oracle.ncm_forward(_cfg(spec), w, ids, None, tgt, bf16=False,
                                       mask="block_diagonal", trace=True)
    got = states.cpu().numpy()
    for i, r in enumerate(ref_states):
        scale = np.max(np.abs(r))
        assert np.max(np.abs(got[i] - r)) <= TOL * scale, i


def test_ncm_f32_reference_invariants(cuda, ncm, oracle):
    """src/ncm_model.zig:332-429 in the reference's arithmetic on the device:
    level-0 inputs do not reach the output when query_level0 (bit for bit);
    the queries, the level embeddings and the prefix table do; a fully padded
    prefix stays finite (its queries see no key: zero context). With the
    block-diagonal mask a change of one level's inputs leaves every other
    position bit-identical; with the block-causal mask, every earlier one."""
    import torch
    from ncmorph_amd import ncm as N

    rng = np.random.default_rng(11)
    levels, P = [4, 8, 16, 32], 6
    hidden, vq, hd, inter, vocab = 128, 64, 32, 256, 20
    for mask in ("block_diagonal", "block_causal"):
        spec = _spec(N, levels, P, hidden, vq, 4, 2, hd, inter, 2, mask, vocab)
        w = random_ncm(rng, _ident, hidden, vq, inter, 4, 2, hd, 2, levels, P, vocab)
        dw = N.device_weights_f32(spec, w, cuda)
        ids = rng.integers(0, vocab, P)
        tgt = rng.standard_normal((sum(levels), vq)).astype(np.float32)
        out = _run(N, torch, cuda, spec, dw, ids, tgt)
        t2 = tgt.copy()
        t2[:levels[0]] += 5.0
        assert np.array_equal(out, _run(N, torch, cuda, spec, dw, ids, t2))
        begin = np.cumsum([P] + levels)
        t3 = tgt.copy()
        t3[begin[2] - P:begin[3] - P] *= -1
        o3 = _run(N, torch, cuda, spec, dw, ids, t3)
        changed = np.any(o3 != out, axis=1)
        assert changed[begin[2]:begin[3]].all()
        assert not changed[:begin[2]].any()
        if mask == "block_diagonal":
            assert not changed[begin[3]:].any()
        else:
            assert changed[begin[3]:].all()
        w2 = dict(w, l0_queries=w["l0_queries"] + np.float32(0.5))
        assert not np.array_equal(out, _run(N, torch, cuda, spec,
                                            N.device_weights_f32(spec, w2, cuda), ids, tgt))
        w3 = dict(w, level_embedding=w["level_embedding"] + np.float32(0.25))
        assert not np.array_equal(out, _run(N, torch, cuda, spec,
                                            N.device_weights_f32(spec, w3, cuda), ids, tgt))
        ids2 = ids.copy()
        ids2[0] = (ids2[0] + 1) % vocab
        assert not np.array_equal(out, _run(N, torch, cuda, spec, dw, ids2, tgt))
        full = _run(N, torch, cuda, spec, dw, ids, tgt, np.ones(P, bool))
        assert np.all(np.isfinite(full))
        ref = oracle.ncm_forward(_cfg(spec), w, ids, np.ones(P, bool), tgt, bf16=False, mask=mask)
        assert np.abs(full - ref).max() <= TOL * np.abs(ref).max()

