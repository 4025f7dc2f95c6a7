"""GPU NCM level-parallel body (ncm_ncm_forward_dev) against the oracle's
bf16-mode composition (oracle.ncm_forward, pinned by the reference's
invariant test and an f64 forward), and the reference's invariants on the
device, at small shapes and at the Llama-3-8B shape with 8 levels of a
4096-position sequence.

Bar: the final-normalized states agree with the oracle within 3% of their
largest magnitude (max) and 0.3% (mean): the GPU sums projections, scores
and P V in MFMA order, so intermediate bf16 roundings differ from the
oracle's now and then and the differences travel through the layers. The
reference's invariants hold bit for bit on the device."""
import numpy as np
import pytest

from .ncm_f64 import random_ncm

pytestmark = pytest.mark.gpu


def _spec(ncm, levels, P, hidden, vq, hq, hkv, hd, inter, layers, mask, vocab, window=0,
          query_level0=True):
    return ncm.NcmSpec(hidden=hidden, vq_width=vq, intermediate=inter, q_heads=hq,
                       kv_heads=hkv, head_dim=hd, layers=layers, level_lengths=tuple(levels),
                       prefix_length=P, prefix_vocab=vocab, query_level0=query_level0,
                       mask=mask, window=window, rope_theta=10000.0, rope_llama3=None)


def _oracle_cfg(spec):
    return dict(hidden_size=spec.hidden, vq_width=spec.vq_width,
                num_attention_heads=spec.q_heads, num_key_value_heads=spec.kv_heads,
                head_dim=spec.head_dim, intermediate_size=spec.intermediate,
                rms_norm_epsilon=spec.rms_eps, level_lengths=list(spec.level_lengths),
                prefix_length=spec.prefix_length, query_level0=spec.query_level0,
                rope="default", rope_theta=spec.rope_theta,
                source_causal=spec.mask == "causal", sliding_window=spec.window or None)


def _run(ncm, torch, cuda, spec, dw, ids, tgt, pad=None):
    cos, sin = ncm.rope_tables(spec)
    out = ncm.forward(spec, dw, ids, torch.from_numpy(tgt).to(cuda),
                      torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda),
                      prefix_pad_mask=pad)
    torch.cuda.synchronize()
    return out.cpu().numpy()


CASES = [
    # (mask, head_dim, extras, window, query_level0, pad)
    ("block_diagonal", 64, {}, 0, True, True),
    ("block_causal", 64, dict(biases=True), 0, True, True),
    ("block_diagonal", 128, dict(qk_norm=True), 0, False, False),
    ("block_causal", 128, dict(convs=True, qk_norm=True, biases=True), 0, True, True),
    ("causal", 64, {}, 0, True, False),
    ("causal", 128, dict(biases=True), 24, True, False),
]


@pytest.mark.parametrize("mask,hd,extras,window,ql0,use_pad", CASES)
def test_ncm_body_matches_oracle(cuda, ncm, oracle, mask, hd, extras, window, ql0, use_pad):
    import torch
    from ncmorph_amd import ncm as N

    print(f"ncm case mask={mask} hd={hd} extras={extras} window={window}", flush=True)
    rng = np.random.default_rng(hd + len(extras) + window)
    levels, P = [8, 16, 32, 64], 12
    hidden, vq, hq, hkv, inter, nl, vocab = 256, 128, 4, 2, 512, 2, 50
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, mask, vocab, window, ql0)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   query_level0=ql0, **extras)
    ids = rng.integers(0, vocab, P)
    pad = (rng.random(P) < 0.3) if use_pad else None
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    dw = N.device_weights(spec, w, cuda)
    got = _run(N, torch, cuda, spec, dw, ids, tgt, pad)
    ref = oracle.ncm_forward(_oracle_cfg(spec), w, ids, pad, tgt, bf16=True,
                             mask="block_diagonal" if mask == "causal" else mask)
    scale = np.max(np.abs(ref))
    err = np.abs(got - ref)
    assert np.all(np.isfinite(got))
    assert err.max() <= 0.03 * scale, err.max() / scale
    assert err.mean() <= 0.003 * scale, err.mean() / scale
    print("max / mean error relative to max|ref|:", err.max() / scale, err.mean() / scale)


@pytest.mark.parametrize("mask", ["block_causal", "block_diagonal"])
def test_ncm_hidden_states_match_oracle(cuda, ncm, oracle, mask):
    """hidden_states (forward_with_trace, src/ncm_model.zig:169-171, :243-249):
    [layers + 1, S, hidden] = the input stage, the output of every layer but
    the last, then the final-normalized output (equal to the body's output
    bit for bit); with the states the output is the same bits as without;
    every state agrees with the oracle's within the body's bound."""
    import torch
    from ncmorph_amd import ncm as N

    rng = np.random.default_rng(23)
    levels, P = [8, 16, 32], 10
    hidden, vq, hq, hkv, hd, inter, nl, vocab = 256, 128, 4, 2, 64, 512, 3, 40
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, mask, vocab)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   biases=True)
    ids = rng.integers(0, vocab, P)
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    dw = N.device_weights(spec, w, cuda)
    cos, sin = N.rope_tables(spec)
    args = (spec, dw, ids, torch.from_numpy(tgt).to(cuda), torch.from_numpy(cos).to(cuda),
            torch.from_numpy(sin).to(cuda))
    plain = N.forward(*args)
    out, states = N.forward(*args, hidden_states=True)
    torch.cuda.synchronize()
    assert states.shape == (nl + 1, spec.seq_len, hidden)
    assert torch.equal(plain, out)
    assert torch.equal(states[nl], out)
    ref, ref_states = oracle.ncm_forward(_oracle_cfg(spec), w, ids, None, tgt, bf16=True,
                                         mask=mask, trace=True)
    got = states.cpu().numpy()
    for i, r in enumerate(ref_states):
        scale = np.max(np.abs(r))
        err = np.abs(got[i] - r)
        assert err.max() <= 0.03 * scale, (i, err.max() / scale)
        assert err.mean() <= 0.003 * scale, (i, err.mean() / scale)
    # The input stage has no summation-order freedom beyond the input
    # projection: it is bf16-valued.
    assert np.array_equal(got[0], oracle.round_bf16(got[0]))


# Layer-replay bars: one layer of the body from the device's own input state
# (the oracle's ncm_layer) against the device's next state. Inside a layer
# the MFMA's summation order moves a projection's bf16 output by one step
# for a few percent of the elements, and such steps pass through the
# attention, the MLP and both residual adds of that layer only.
# A flip of the largest element is one bf16 step, up to 2^-7 of it.
LAYER_SAME, LAYER_ERR = 0.85, 2.0 ** -6
INPUT_SAME = 0.95


def _layer_close(dev, ref, min_same=LAYER_SAME):
    same = float(np.mean(dev == ref))
    err = float(np.max(np.abs(dev - ref))) / max(float(np.max(np.abs(ref))), 1e-30)
    return same >= min_same and err <= LAYER_ERR, (round(same, 4), round(err, 5))


@pytest.mark.parametrize("mask,hd,extras", [("block_diagonal", 64, dict(biases=True)),
                                             ("block_causal", 128, dict(qk_norm=True,
                                                                        convs=True))])
def test_ncm_layers_replayed_against_oracle(cuda, ncm, oracle, mask, hd, extras):
    """Every stage of the bf16 body against the oracle applied to the
    device's own input of that stage (hidden_states): the input stage
    (prefix rows, queries, convs, input projection, level embeddings) at
    least 95% identical and within 2^-6 of its largest magnitude (two bf16
    steps of the largest element); each layer (oracle.ncm_layer on the
    device's state before it) at least 85% identical and within 2^-6; the
    last layer with the final norm likewise (measured 91-100% identical,
    errors up to 0.55%). The whole-body comparison allows 3%, because it
    carries differences through every layer. Planted mistakes in the
    replay (the other level mask; positions that do not restart at each
    level; two heads' output-projection columns exchanged) fail them."""
    import torch
    from ncmorph_amd import ncm as N

    print(f"ncm replay mask={mask} hd={hd} extras={extras}", flush=True)
    rng = np.random.default_rng(41 + hd)
    levels, P = [8, 16, 32, 64], 12
    hidden, vq, hq, hkv, inter, nl, vocab = 256, 128, 4, 2, 512, 3, 50
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, mask, vocab)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   **extras)
    ids = rng.integers(0, vocab, P)
    pad = rng.random(P) < 0.3
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    dw = N.device_weights(spec, w, cuda)
    cos, sin = N.rope_tables(spec)
    out, states = N.forward(spec, dw, ids, torch.from_numpy(tgt).to(cuda),
                            torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda),
                            prefix_pad_mask=pad, hidden_states=True)
    torch.cuda.synchronize()
    st = states.cpu().numpy()
    cfg = _oracle_cfg(spec)
    report = {}
    inp = oracle.ncm_input_stage(cfg, w, ids, tgt, bf16=True)
    ok, report["input"] = _layer_close(st[0], inp, INPUT_SAME)
    assert ok, report
    ocos, osin, m = oracle.ncm_tables_and_mask(cfg, pad, mask)
    for l in range(nl):
        ref = oracle.ncm_layer(cfg, w["layers"][l], st[l], ocos, osin, m, bf16=True)
        if l == nl - 1:
            ref = oracle.ncm_final_norm(cfg, w, ref, bf16=True)
        ok, report[f"layer{l}"] = _layer_close(st[l + 1], ref)
        assert ok, (l, report)
    print("stage (identical fraction, max error / max|ref|):", report, flush=True)

    # Planted mistakes, in the oracle's replay of layer 0 only.
    other = "block_causal" if mask == "block_diagonal" else "block_diagonal"
    _, _, m_other = oracle.ncm_tables_and_mask(cfg, pad, other)
    bad = oracle.ncm_layer(cfg, w["layers"][0], st[0], ocos, osin, m_other, bf16=True)
    assert not _layer_close(st[1], bad)[0]
    inv = oracle.rope_default_frequencies(hd, spec.rope_theta)
    lin_cos, lin_sin = oracle.rope_tables(inv, spec.seq_len)
    bad = oracle.ncm_layer(cfg, w["layers"][0], st[0], lin_cos, lin_sin, m, bf16=True)
    assert not _layer_close(st[1], bad)[0]
    L0 = dict(w["layers"][0])
    wo = np.array(L0["output_weight"], np.float32)
    wo[:, :hd], wo[:, hd:2 * hd] = wo[:, hd:2 * hd].copy(), wo[:, :hd].copy()
    L0["output_weight"] = wo
    bad = oracle.ncm_layer(cfg, L0, st[0], ocos, osin, m, bf16=True)
    assert not _layer_close(st[1], bad)[0]


def test_ncm_rejects_misaligned_conv_weight(cuda, ncm, oracle):
    """The convolutions read their weights with 16-byte loads: a conv weight
    that is not 16-byte aligned is refused (NCM_E_ARG) before any launch, as
    the f32 body does."""
    import torch
    from ncmorph_amd import ncm as N
    from ncmorph_amd._lib import NCM_E_ARG, NcmError

    rng = np.random.default_rng(31)
    levels, P = [8, 16], 4
    hidden, vq, hq, hkv, hd, inter, nl, vocab = 128, 64, 2, 1, 64, 256, 1, 20
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, "block_causal", vocab)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   convs=True)
    dw = N.device_weights(spec, w, cuda)
    buf = torch.empty(vq * vq * 3 + 1, dtype=torch.float32, device=cuda)
    odd = buf[1:].view(vq, vq, 3)
    odd.copy_(dw.convs[0]["weight"])
    assert odd.data_ptr() % 16 != 0
    dw.convs[0]["weight"] = odd
    cos, sin = N.rope_tables(spec)
    tgt = torch.zeros((sum(levels), vq), dtype=torch.float32, device=cuda)
    with pytest.raises(NcmError) as e:
        N.forward(spec, dw, rng.integers(0, vocab, P), tgt, torch.from_numpy(cos).to(cuda),
                  torch.from_numpy(sin).to(cuda))
    assert e.value.status == NCM_E_ARG


def test_ncm_body_reference_invariants(cuda, ncm, oracle):
    """src/ncm_model.zig:332-429 on the device: level-0 inputs do not reach
    the output when query_level0 (bit for bit), the queries, the level
    embeddings and the prefix table do; a padded prefix stays finite. With
    the block-diagonal mask a change of one level's inputs leaves every other
    position bit-identical; with the block-causal mask, every earlier one."""
    import torch
    from ncmorph_amd import ncm as N

    rng = np.random.default_rng(7)
    levels, P = [4, 8, 16, 32], 6
    hidden, vq, hd, inter, vocab = 256, 128, 64, 512, 20
    for mask in ("block_diagonal", "block_causal"):
        spec = _spec(N, levels, P, hidden, vq, 4, 2, hd, inter, 2, mask, vocab)
        w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, 4, 2, hd, 2, levels, P, vocab)
        dw = N.device_weights(spec, w, cuda)
        ids = rng.integers(0, vocab, P)
        tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
        out = _run(N, torch, cuda, spec, dw, ids, tgt)
        t2 = tgt.copy()
        t2[:levels[0]] += 5.0                       # level 0 is replaced by the queries
        assert np.array_equal(out, _run(N, torch, cuda, spec, dw, ids, t2))
        begin = np.cumsum([P] + levels)
        t3 = tgt.copy()
        t3[begin[2] - P:begin[3] - P] *= -1        # level 2's inputs
        o3 = _run(N, torch, cuda, spec, dw, ids, t3)
        changed = np.any(o3 != out, axis=1)
        assert changed[begin[2]:begin[3]].all()
        assert not changed[:begin[2]].any()
        if mask == "block_diagonal":
            assert not changed[begin[3]:].any()
        else:
            assert changed[begin[3]:].all()
        w2 = dict(w, l0_queries=w["l0_queries"] + np.float32(0.5))
        assert not np.array_equal(out, _run(N, torch, cuda, spec, N.device_weights(spec, w2, cuda),
                                            ids, tgt))
        w3 = dict(w, level_embedding=w["level_embedding"] + np.float32(0.25))
        assert not np.array_equal(out, _run(N, torch, cuda, spec, N.device_weights(spec, w3, cuda),
                                            ids, tgt))
        ids2 = ids.copy()
        ids2[0] = (ids2[0] + 1) % vocab
        assert not np.array_equal(out, _run(N, torch, cuda, spec, dw, ids2, tgt))
        assert np.all(np.isfinite(_run(N, torch, cuda, spec, dw, ids, tgt, np.ones(P, bool))))


def test_ncm_code_heads_match_oracle(cuda, ncm, oracle):
    """Per-level z projection of the body's output and the tied heads: z
    agrees with the oracle's matmul_bf16 within one bf16 step (summation
    order), and every logit is within the tied head's fp32 bound (see
    test_tied_head_gpu.py) of the f64 head formula on that z, with each
    level's rows, codebook and log_inv_T."""
    import torch
    from ncmorph_amd import kernels, ncm as N, vq

    rng = np.random.default_rng(3)
    levels, P, hidden, d, V = [4, 8, 16], 3, 256, 128, 300
    spec = _spec(N, levels, P, hidden, 128, 4, 2, 64, 512, 1, "block_diagonal", 10)
    h = oracle.round_bf16(rng.standard_normal((spec.seq_len, hidden)).astype(np.float32))
    zw = oracle.round_bf16((rng.standard_normal((3, d, hidden)) * 0.05).astype(np.float32))
    cb = oracle.round_bf16((rng.standard_normal((3, V, d)) / np.sqrt(d)).astype(np.float32))
    to_bf = lambda a: torch.from_numpy((a.view(np.uint32) >> 16).astype(np.uint16).view(
        np.int16)).to(cuda).view(torch.bfloat16)
    cbd, zwd = to_bf(cb), to_bf(zw)
    hd_ = torch.from_numpy(h).to(cuda)
    csq = vq.prepare(cbd)
    lit = np.asarray([0.0, 0.3, -0.2], np.float32)
    got = N.code_head_logits(spec, hd_, zwd, cbd, csq, log_inv_t=lit).cpu().numpy()
    h16 = kernels.bf16_from_f32(hd_[P:])
    off = 0
    for l, n in enumerate(levels):
        zg = kernels.linear_bf16(h16[off:off + n], zwd[l], out_mode="bf16_f32").cpu().numpy()
        zo = oracle.matmul_bf16(h[P + off:P + off + n], zw[l])
        ulp = np.abs(zo).view(np.uint32) & 0x7F800000
        step = (ulp.astype(np.uint32) >> 23).astype(np.int32)
        assert np.all(np.abs(zg - zo) <= np.ldexp(1.0, step - 127 - 7) + 1e-30)
        ref, mag = oracle.tied_head_logits_f64(zg, cb[l], log_inv_t=float(lit[l]))
        esq = np.sum(cb[l].astype(np.float64) ** 2, axis=1)
        scale = np.exp(float(lit[l])) / esq.mean()
        t = np.abs(ref) / scale
        bound = (scale * ((d + 4) * 2.0**-24 * mag + d * 2.0**-24 * esq[None, :] + 2.0**-22 * t)
                 + 2.0**-21 * np.abs(ref) + 1e-30)
        err = np.abs(got[off:off + n].astype(np.float64) - ref)
        assert np.all(err <= bound), (l, float(np.max(err / bound)))
        off += n


def test_ncm_body_8b_layer_shape_against_oracle(cuda, ncm, oracle):
    """Two layers at the Llama-3-8B layer shape (hidden 4096, 32 / 8 heads of
    128, FFN 14336, vq width 4096) over an 8-token prefix and levels of 1, 2,
    4 and 8 positions, block-causal, against the oracle's bf16 body (its
    matmuls threaded over the host's cores, bit-identical to one thread):
    the body's bar of 3% (max) and 0.3% (mean) of max|ref|, on the output and
    on every hidden state."""
    import os

    import torch
    from ncmorph_amd import ncm as N

    rng = np.random.default_rng(84)
    levels, P = [1, 2, 4, 8], 8
    hidden, vq, hq, hkv, hd, inter, nl, vocab = 4096, 4096, 32, 8, 128, 14336, 2, 64
    spec = _spec(N, levels, P, hidden, vq, hq, hkv, hd, inter, nl, "block_causal", vocab)
    w = random_ncm(rng, oracle.round_bf16, hidden, vq, inter, hq, hkv, hd, nl, levels, P, vocab,
                   std=0.02, biases=True)
    ids = rng.integers(0, vocab, P)
    tgt = oracle.round_bf16(rng.standard_normal((sum(levels), vq)).astype(np.float32))
    dw = N.device_weights(spec, w, cuda)
    cos, sin = N.rope_tables(spec)
    out, states = N.forward(spec, dw, ids, torch.from_numpy(tgt).to(cuda),
                            torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda),
                            hidden_states=True)
    torch.cuda.synchronize()
    got_states = states.cpu().numpy()
    del dw, states
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    prev = oracle.set_threads(threads)
    try:
        ref, ref_states = oracle.ncm_forward(_oracle_cfg(spec), w, ids, None, tgt, bf16=True,
                                             mask="block_causal", trace=True)
    finally:
        oracle.set_threads(prev)
    for i, (g, r) in enumerate(list(zip(got_states, ref_states)) + [(out.cpu().numpy(), ref)]):
        scale = np.max(np.abs(r))
        err = np.abs(g - r)
        assert np.all(np.isfinite(g)), i
        assert err.max() <= 0.03 * scale, (i, err.max() / scale)
        assert err.mean() <= 0.003 * scale, (i, err.mean() / scale)


def test_ncm_body_8b_shape_properties(cuda, ncm):
    """The Llama-3-8B-shaped body (32 layers, hidden 4096, 32/8 heads of 128,
    FFN 14336) over a 64-token prefix and the 8 levels of a 4096-position
    sequence (8160 target positions), block-causal mask: finite output,
    identical bits on a second run, level-0 inputs without effect (learned
    queries), and a change of the last level's inputs confined to its rows."""
    import torch
    from ncmorph_amd import ncm as N

    spec = N.LLAMA_3_8B_NCM
    dw = N.random_weights(spec, cuda, seed=5)
    g = torch.Generator(device=cuda).manual_seed(6)
    T = sum(spec.level_lengths)
    tgt = torch.randn(T, spec.vq_width, generator=g, device=cuda)
    ids = np.random.default_rng(6).integers(0, spec.prefix_vocab, spec.prefix_length)
    cos, sin = N.rope_tables(spec)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    out = N.forward(spec, dw, ids, tgt, cd, sd)
    again = N.forward(spec, dw, ids, tgt, cd, sd)
    torch.cuda.synchronize()
    assert out.shape == (spec.seq_len, spec.hidden)
    assert bool(torch.isfinite(out).all())
    assert torch.equal(out, again)
    t2 = tgt.clone()
    t2[:spec.level_lengths[0]] += 3.0
    assert torch.equal(out, N.forward(spec, dw, ids, t2, cd, sd))
    last = spec.seq_len - spec.level_lengths[-1]
    t3 = tgt.clone()
    t3[last - spec.prefix_length:] *= -1
    o3 = N.forward(spec, dw, ids, t3, cd, sd)
    torch.cuda.synchronize()
    changed = (o3 != out).any(dim=1).cpu().numpy()
    assert not changed[:last].any() and changed[last:].all()
