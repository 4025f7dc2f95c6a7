"""Benchmark of the ncmorph hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only linear|rvq|decoder]

A step is one pass of the bf16-weight linear over the three Llama-3.2-1B
shapes: x bf16 [2048, K] ~N(0,1) times W^T with W bf16 [N, K] ~N(0, 0.02^2),
(N, K) in {(2048, 2048), (8192, 2048), (2048, 8192)}, fp32 accumulation and
fp32 output. `value` is the whole step's TFLOP/s (algorithmic 2*M*N*K per
linear) with inputs resident in HBM.

The same JSON line carries the multiscale RVQ encode at 16 x 2048 positions,
d = 2048, 8 levels (strides 128..1), 4096 codes per level (input seed 1),
timed separately and reported as tokens/s (input positions per second of a
full encode including the reconstruction), and the bf16 decoder prefill
forward of a random-init Llama-3.2-1B over 4 x 1024 tokens (tokens/s), each
with its roofline fraction and CPU baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0
METRIC = "RVQ-encode tokens/s & bf16-linear TFLOP/s (1B shape), % of MI355X roofline"
LINEAR_M = 2048
LINEAR_NK = [(2048, 2048), (8192, 2048), (2048, 8192)]
# HBM-side bytes measured with rocprofv3 FETCH_SIZE / WRITE_SIZE (each in its
# own run, fetch scaled by the factor a plain copy shows): the linear figure is
# the mean over the step's three launches (466.1 MB per step), the RVQ figure
# one whole encode (3521 MB fetched, 1049 MB written); the summaries and
# commands are in profiles/linear_bf16_1b_shapes.md and
# profiles/rvq_encode_b16_t2048_d2048_l8_v4096.md.
LINEAR_TRAFFIC_BYTES_PER_LAUNCH = 155.4e6
RVQ_TRAFFIC_BYTES_PER_ENCODE = 4570e6
NEAR_TIE_REL = 1e-5  # relative top-2 distance gap under which a code is a near-tie


def cpu_threads():
    """Host threads for the N-core CPU baselines: the cores this process may
    use, capped at 16 (the GPU box's share of the host)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def linear_inputs(torch, dev):
    from ncmorph_amd import synth

    xs, ws = {}, {}
    for (n, k) in LINEAR_NK:
        if k not in xs:
            xb = synth.normal_bf16(synth.LINEAR_SEED_X + k, (LINEAR_M, k))
            xs[k] = torch.from_numpy(xb.view(np.int16)).to(dev).view(torch.bfloat16)
        wb = synth.normal_bf16(synth.LINEAR_SEED_W + n * 7 + k, (n, k), std=0.02)
        ws[(n, k)] = torch.from_numpy(wb.view(np.int16)).to(dev).view(torch.bfloat16)
    ys = {nk: torch.empty((LINEAR_M, nk[0]), dtype=torch.float32, device=dev) for nk in LINEAR_NK}
    return xs, ws, ys


# Untimed clock-settling run before every timed loop, ours and hipBLASLt's
# alike: the GPU raises its engine clock over roughly 100 ms of sustained
# load, so a loop timed right after set-up, host-only work (a CPU baseline)
# or a short warmup measures the ramp instead of the steady clock.
RAMP_MS = 200.0
SHAPE_RAMP_MS = 50.0


def _ramp(torch, fn, ms=RAMP_MS):
    """Runs fn, untimed, until about `ms` of wall time has passed."""
    t0 = time.perf_counter()
    n = 1
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        n *= 2


def _queue_ahead(torch, cycles=5_000_000):
    """Occupies the GPU for about 2 ms (one spinning wavefront) so that the
    host queues the launches of a timed region behind it: the region's start
    event then fires with its first kernels already queued, and the timing
    holds the GPU's work rather than the host's first launch calls."""
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(cycles)


def _queued_launch_time(torch, run, reps=20):
    """Seconds per launch of `run` with its launches queued behind a GPU
    spin: a 2048^3 launch takes less time than one host-side launch call,
    so an unqueued loop would time the host. Used for ours and hipBLASLt's
    per-shape figures alike."""
    e0, e1 = _events(torch)
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(2_000_000)  # about 1 ms of GPU cycles
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps * 1e-3


def run_linear(torch, steps, warmup):
    from ncmorph_amd import kernels

    dev = torch.device("cuda", 0)
    xs, ws, ys = linear_inputs(torch, dev)

    def step():
        for (n, k) in LINEAR_NK:
            kernels.linear_bf16(xs[k], ws[(n, k)], out=ys[(n, k)])

    # Per-shape launch durations (events on the launch stream), each shape
    # after the same 50 ms ramp that the hipBLASLt shapes get below.
    per_shape = {}
    for (n, k) in LINEAR_NK:
        run = lambda: kernels.linear_bf16(xs[k], ws[(n, k)], out=ys[(n, k)])  # noqa: E731
        _ramp(torch, run, ms=SHAPE_RAMP_MS)
        per_shape[(n, k)] = _queued_launch_time(torch, run)
    # Clock ramp, then `warmup` untimed steps, then the timed region:
    # exactly `steps` steps, synchronized on both sides.
    _ramp(torch, step)
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    t0 = time.perf_counter()
    _queue_ahead(torch)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_s = e0.elapsed_time(e1) * 1e-3
    flops = sum(2.0 * LINEAR_M * n * k for (n, k) in LINEAR_NK)
    # Sanity: one output against torch's fp32 product.
    n, k = LINEAR_NK[0]
    ref = xs[k].float() @ ws[(n, k)].float().T
    err = float((ys[(n, k)] - ref).abs().max())
    # Same-box reference point, outside the timed region: torch's bf16
    # linear (hipBLASLt; bf16 output, half of this path's output bytes).
    # Also torch.mm with out_dtype=float32 (hipBLASLt with this path's fp32
    # output), where this torch build has it.
    def vendor_times(fn):
        out = {}
        for (n, k) in LINEAR_NK:
            run = lambda: fn(xs[k], ws[(n, k)])  # noqa: E731
            _ramp(torch, run, ms=SHAPE_RAMP_MS)
            out[(n, k)] = _queued_launch_time(torch, run)
        return out

    vendor = vendor_times(torch.nn.functional.linear)
    try:
        vendor_f32 = vendor_times(lambda a, b: torch.mm(a, b.t(), out_dtype=torch.float32))
    except (RuntimeError, TypeError):
        vendor_f32 = None
    return {"step_s": gpu_s / steps, "wall_s": wall, "flops_per_step": flops,
            "per_shape_s": per_shape, "max_abs_err_vs_fp32": err, "vendor_per_shape_s": vendor,
            "vendor_f32_per_shape_s": vendor_f32}


def run_rvq(torch, reps, warmup):
    from ncmorph_amd import synth, vq

    dev = torch.device("cuda", 0)
    c = synth.RVQ_LARGE
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    xd = torch.from_numpy(x).to(dev)
    cbd = torch.from_numpy(cb.view(np.int16)).to(dev).view(torch.bfloat16)
    del x
    csq = vq.prepare(cbd)
    out = {}
    r = vq.encode(xd, cbd, c["strides"], csq=csq, want_gap=False, level_counts=True)
    n_flagged = r["n_flagged"]
    level_rows = [c["b"] * c["t"] // s for s in c["strides"]]
    rescored = [{"rows": n, "scored": sc, "share": round(sc / n, 4), "flagged": fl}
                for n, sc, fl in zip(level_rows, r["scored"], r["flagged"])]
    out = {"codes": r["codes"], "recon": r["recon"]}

    def enc():
        vq.encode(xd, cbd, c["strides"], csq=csq, want_gap=False, out=out)

    _ramp(torch, enc)
    for _ in range(warmup):
        enc()
    torch.cuda.synchronize()
    e0, e1 = _events(torch)
    _queue_ahead(torch)
    e0.record()
    for _ in range(reps):
        vq.encode(xd, cbd, c["strides"], csq=csq, want_gap=False, out=out)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) * 1e-3 / reps
    # Untimed: one encode with the per-code relative top-2 gap, for the
    # near-tie count (gap < 1e-5: the rows where any fp32 order could pick
    # another code).
    g = vq.encode(xd, cbd, c["strides"], csq=csq, want_recon=False, want_gap=True)["gap"]
    torch.cuda.synchronize()
    near = int((g < NEAR_TIE_REL).sum())
    rows = sum(c["b"] * c["t"] // s for s in c["strides"])
    flops = 2.0 * c["v"] * c["d"] * rows
    # x read once, codebooks read once, codes and reconstruction written once.
    bytes_alg = (c["b"] * c["t"] * c["d"] * 4 + c["levels"] * c["v"] * c["d"] * 2 +
                 rows * 4 + c["b"] * c["t"] * c["d"] * 4)
    return {"encode_s": t, "tokens": c["b"] * c["t"], "flops": flops, "bytes": bytes_alg,
            "n_flagged": n_flagged, "near_ties": near, "codes": rows, "rescored": rescored}


def run_decoder_ops(torch, reps=20):
    """The bf16 decoder's ops around the linear at the Llama-3.2-1B layer shape
    (4096 tokens, hidden 2048, intermediate 8192): RMSNorm rows (f32 in, bf16
    out) and the MLP activation round_bf16(silu(gate) * up) (f32 in, bf16
    out). HBM-bound: bytes = inputs read once + output written once."""
    from ncmorph_amd import kernels

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(7)
    t, h, inter = 4096, 2048, 8192
    x = torch.randn(t, h, device=dev, generator=g)
    w = torch.randn(h, device=dev, generator=g) * 0.1 + 1
    gate = torch.randn(t, inter, device=dev, generator=g)
    up = torch.randn(t, inter, device=dev, generator=g)
    y_n = torch.empty(t, h, dtype=torch.bfloat16, device=dev)
    y_m = torch.empty(t, inter, dtype=torch.bfloat16, device=dev)
    out = {}
    for name, fn, nbytes in (
            ("rms_norm_bf16_rows", lambda: kernels.rms_norm_rows(x, w, 1e-5, "bf16", out=y_n),
             t * h * 4 + h * 4 + t * h * 2),
            ("silu_mul_bf16", lambda: kernels.silu_mul(gate, up, "bf16", out=y_m),
             2 * t * inter * 4 + t * inter * 2)):
        _ramp(torch, fn)
        e0, e1 = _events(torch)
        # Kernels of about 10 us: the launches are queued behind a GPU spin so
        # that the events time the kernels, not the host's launch calls.
        _queue_ahead(torch)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        gbs = nbytes / sec / 1e9
        out[name] = {"shape": [t, h] if "norm" in name else [t, inter], "us": round(sec * 1e6, 2),
                     "bytes": nbytes,
                     "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                                  "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    return out


DECODER_BATCH, DECODER_SEQ = 4, 1024


def decoder_flops(spec, batch, seq):
    """Algorithmic FLOPs of one bf16 prefill forward: 2 per multiply-add of
    every projection and the LM head, plus the causal attention's QK^T and
    PV over the allowed (query, key) pairs."""
    t = batch * seq
    per_layer = (spec.qkv_width * spec.hidden + spec.hidden * spec.q_heads * spec.head_dim
                 + 2 * spec.intermediate * spec.hidden + spec.hidden * spec.intermediate)
    linear = 2.0 * t * (spec.layers * per_layer + spec.vocab * spec.hidden)
    pairs = batch * seq * (seq + 1) / 2
    attention = spec.layers * spec.q_heads * 2 * (2.0 * pairs * spec.head_dim)
    return linear, attention


def run_decoder(torch, reps=10, warmup=3):
    """Random-init Llama-3.2-1B bf16 prefill forward over 4 x 1024 token ids
    (16 layers, hidden 2048, 32/8 heads of 64, SwiGLU 8192, vocab 128256,
    weights ~N(0, 0.02), Llama 3 RoPE theta 500000), logits to HBM."""
    from ncmorph_amd import decoder

    dev = torch.device("cuda", 0)
    spec = decoder.LLAMA_3_2_1B
    w = decoder.random_weights(spec, dev, seed=11)
    cos, sin = decoder.rope_tables(spec, DECODER_SEQ)
    cd, sd = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    ids = np.random.default_rng(12).integers(0, spec.vocab, (DECODER_BATCH, DECODER_SEQ))
    logits = torch.empty((DECODER_BATCH * DECODER_SEQ, spec.vocab), dtype=torch.float32,
                         device=dev)
    for _ in range(warmup):
        decoder.forward(spec, w, ids, cd, sd, logits=logits)
    _ramp(torch, lambda: decoder.forward(spec, w, ids, cd, sd, logits=logits))
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        decoder.forward(spec, w, ids, cd, sd, logits=logits)
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    lin, att = decoder_flops(spec, DECODER_BATCH, DECODER_SEQ)
    tf = (lin + att) / sec / 1e12
    tokens = DECODER_BATCH * DECODER_SEQ
    return {"metric": "bf16 decoder prefill tokens/s", "value": round(tokens / sec, 1),
            "unit": "tokens/s", "ms_per_forward": round(sec * 1e3, 3),
            "config": {"workload": "random-init Llama-3.2-1B bf16 prefill forward, logits out",
                       "batch": DECODER_BATCH, "seq_len": DECODER_SEQ, "layers": spec.layers,
                       "hidden": spec.hidden, "heads": [spec.q_heads, spec.kv_heads],
                       "head_dim": spec.head_dim, "intermediate": spec.intermediate,
                       "vocab": spec.vocab},
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                         "flops_linear": lin, "flops_attention_causal": att}}


def ncm_step_flops(spec, d, v):
    """Algorithmic FLOPs of one NCM level-parallel step: 2 per multiply-add
    of the input projection and every layer projection over all S
    positions, 4 head_dim per allowed (query, key) pair and query head for
    QK^T and P V, and per target position the level's z projection (hidden
    -> d) and tied head (d -> v codes)."""
    S = spec.seq_len
    T = sum(spec.level_lengths)
    qw, kvw = spec.q_heads * spec.head_dim, spec.kv_heads * spec.head_dim
    per_layer = spec.hidden * (qw + 2 * kvw) + qw * spec.hidden + 3 * spec.hidden * spec.intermediate
    linear = 2.0 * S * (spec.vq_width * spec.hidden + spec.layers * per_layer)
    P = spec.prefix_length
    pairs = P * P
    seen = 0
    for n in spec.level_lengths:
        own = seen + n if spec.mask == "block_causal" else n
        pairs += n * (P + own)
        seen += n
    attention = spec.layers * spec.q_heads * 4.0 * spec.head_dim * pairs
    heads = 2.0 * T * (spec.hidden * d + d * v)
    return linear, attention, heads


def run_ncm_step(torch, reps=5, warmup=2):
    """The NCM level-parallel step at the Llama-3-8B shape: the bf16 body
    (32 layers, hidden 4096, 32 / 8 heads of 128, FFN 14336, input
    projection from vq width 4096) over a 64-token prefix and the 8 levels
    of one 4096-position sequence (32 ... 4096 positions, 8160 in all),
    then the level's z projection (4096 -> 4096) and codebook-tied head
    (8192 codes) at every target position. Random-init weights ~N(0, 0.02),
    code heads' projections ~N(0, 0.02), codebooks ~N(0, 1/4096)."""
    import dataclasses

    from ncmorph_amd import ncm, vq

    dev = torch.device("cuda", 0)
    d, v = 4096, 8192
    out = {}
    base = ncm.LLAMA_3_8B_NCM
    w = ncm.random_weights(base, dev, seed=21)
    g = torch.Generator(device=dev).manual_seed(22)
    L = len(base.level_lengths)
    zw = (torch.randn(L, d, base.hidden, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    cb = (torch.randn(L, v, d, generator=g, device=dev) / d ** 0.5).to(torch.bfloat16)
    csq = vq.prepare(cb)
    T = sum(base.level_lengths)
    tgt = torch.randn(T, base.vq_width, generator=g, device=dev)
    ids = np.random.default_rng(23).integers(0, base.prefix_vocab, base.prefix_length)
    cos, sin = ncm.rope_tables(base)
    cd, sd = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    hidden = torch.empty((base.seq_len, base.hidden), dtype=torch.float32, device=dev)
    for mask in ("block_causal", "block_diagonal"):
        spec = dataclasses.replace(base, mask=mask)

        def step():
            ncm.forward(spec, w, ids, tgt, cd, sd, out=hidden)
            return ncm.code_head_logits(spec, hidden, zw, cb, csq)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = _events(torch)
        e0.record()
        for _ in range(reps):
            step()
        e1.record()
        torch.cuda.synchronize()
        sec = e0.elapsed_time(e1) * 1e-3 / reps
        lin, att, heads = ncm_step_flops(spec, d, v)
        tf = (lin + att + heads) / sec / 1e12
        out[mask] = {"ms_per_step": round(sec * 1e3, 3),
                     "positions_per_s": round(spec.seq_len / sec, 1),
                     "flops": {"linear": lin, "attention": att, "code_heads": heads},
                     "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                                  "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                                  "frac": round(tf / BF16_PEAK_TFLOPS, 4)}}
    del w, zw, cb
    res = out["block_causal"]
    res.update({"metric": "NCM level-parallel step positions/s", "value":
                res["positions_per_s"], "unit": "positions/s",
                "config": {"workload": "random-init Llama-3-8B-shaped bf16 NCM body + tied code "
                                       "heads, one 4096-position sequence",
                           "layers": base.layers, "hidden": base.hidden,
                           "heads": [base.q_heads, base.kv_heads], "head_dim": base.head_dim,
                           "intermediate": base.intermediate, "prefix": base.prefix_length,
                           "levels": list(base.level_lengths), "codebook": v, "d": d,
                           "mask": "block_causal"},
                "block_diagonal": out["block_diagonal"]})
    return res


PCIE_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction
NCM_PREFIX, NCM_LEVELS = 64, [32, 64, 128, 256, 512, 1024, 2048, 4096]


def run_ncm_attention(torch, reps=10):
    """Attention of the NCM level-parallel step at the Llama-3-8B head shape
    (32 query / 8 key-value heads of 128): a 64-token prefix and 8 levels of
    one 4096-position sequence (4096 / 2^(7 - l) positions at level l), under
    the block-diagonal level mask. Flops: 4 hd per allowed (query, key) pair
    and query head (QK^T and PV)."""
    from ncmorph_amd import kernels

    dev = torch.device("cuda", 0)
    hq, hkv, hd = 32, 8, 128
    lo, hi, bits = kernels.block_diagonal_segments(NCM_PREFIX, NCM_LEVELS)
    seq = lo.size
    g = torch.Generator(device=dev).manual_seed(15)
    qkv = torch.randn(seq, (hq + 2 * hkv) * hd, device=dev, generator=g).to(torch.bfloat16)
    q, k, v = qkv[:, :hq * hd], qkv[:, hq * hd:(hq + hkv) * hd], qkv[:, (hq + hkv) * hd:]
    dl, dh = torch.from_numpy(lo).to(dev), torch.from_numpy(hi).to(dev)
    out = torch.empty(seq, hq * hd, dtype=torch.bfloat16, device=dev)

    def run():
        kernels.attention_bf16_seg(q, k, v, 1, seq, hq, hkv, hd, NCM_PREFIX, dl, dh, None,
                                   out_mode="bf16", out=out)

    _ramp(torch, run)
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    pairs = NCM_PREFIX * NCM_PREFIX + sum(n * (NCM_PREFIX + n) for n in NCM_LEVELS)
    flops = 4.0 * hd * hq * pairs
    tf = flops / sec / 1e12
    return {"positions": seq, "us": round(sec * 1e6, 1), "flops": flops,
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4)}}


def run_ncm_tied_head(torch, reps=5):
    """Codebook-tied code heads of the NCM level-parallel step at the 8B shape
    (PROJECT.md:222): for each of the 8 levels (the level lengths of
    run_ncm_attention), logits [n_l, 8192] = (2 z E_l^T - ||E_l||^2) *
    exp(log_inv_T) / mean ||E_l||^2 with z bf16 [n_l, 4096] and the level's
    bf16 codebook E_l [8192, 4096] ~N(0, 1/4096), all levels in one call
    (ncm_tied_head_logits_levels). Flops: 2 V d per row."""
    from ncmorph_amd import kernels, vq

    dev = torch.device("cuda", 0)
    v, d = 8192, 4096
    g = torch.Generator(device=dev).manual_seed(17)
    rows = sum(NCM_LEVELS)
    z = torch.randn(rows, d, device=dev, generator=g).to(torch.bfloat16)
    cb = (torch.randn(len(NCM_LEVELS), v, d, device=dev, generator=g) / d ** 0.5).to(torch.bfloat16)
    csq = vq.prepare(cb)
    out = torch.empty(rows, v, dtype=torch.float32, device=dev)

    def run():
        kernels.tied_head_logits_levels(z, cb, csq, NCM_LEVELS, out=out)

    _ramp(torch, run)
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        run()
    e1.record()
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3 / reps
    flops = 2.0 * v * d * rows
    tf = flops / sec / 1e12
    return {"rows": rows, "codes": v, "d": d, "levels": len(NCM_LEVELS),
            "us": round(sec * 1e6, 1), "flops": flops,
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4)}}


VQ_TOK_BATCH = 1024
VQ_TOK_DECODE_BATCH = 64
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def run_vq_tokenizer(torch, reps=20):
    """The upstream VQ-VAE tokenizer at the released WMT14 configuration
    (D 384, 64 positions, 11 levels 1..64 of 4096 codes, learned level-0
    cascade of three stride-4 stages with GroupNorms, Phi blend convs),
    random-init float32 weights: encode (token ids -> codes + zhat) of 1024
    sequences, and the decoder (zhat -> logits over 151680 tokens) of 64.
    Flops: 2 per multiply-add of the code searches, Phi convs and cascade
    (encode) and of the decoder's linears and attention (decode)."""
    from ncmorph_amd import vq_tokenizer as vt

    dev = torch.device("cuda", 0)
    cfg = vt.WMT14
    tok = vt.Tokenizer(cfg, vt.random_state(cfg, dev, seed=31))
    ids = np.random.default_rng(32).integers(0, cfg.in_vocab, (VQ_TOK_BATCH, cfg.seq_len))
    B = VQ_TOK_BATCH
    codes = torch.empty((B, cfg.codes_per_sequence), dtype=torch.int32, device=dev)
    zhat = torch.empty((B, cfg.seq_len, cfg.embed_dim), dtype=torch.float32, device=dev)
    latent = tok.encode(ids, want_latent=True)["latent"]

    def enc():
        tok.quantize(latent)

    _ramp(torch, enc)
    e0, e1 = _events(torch)
    e0.record()
    for _ in range(reps):
        enc()
    e1.record()
    torch.cuda.synchronize()
    q_sec = e0.elapsed_time(e1) * 1e-3 / reps
    e0.record()
    for _ in range(reps):
        tok.encode(ids)
    e1.record()
    torch.cuda.synchronize()
    e_sec = e0.elapsed_time(e1) * 1e-3 / reps
    del codes, zhat
    fl = vt.flops_per_sequence(cfg)
    tf = fl["total"] * B / q_sec / 1e12
    # decoder
    Bd = VQ_TOK_DECODE_BATCH
    zd = latent[:Bd].contiguous()
    logits = torch.empty((Bd, cfg.seq_len, cfg.in_vocab), dtype=torch.float32, device=dev)
    tok.decode(zd, logits)
    _ramp(torch, lambda: tok.decode(zd, logits))
    e0.record()
    for _ in range(reps):
        tok.decode(zd, logits)
    e1.record()
    torch.cuda.synchronize()
    d_sec = e0.elapsed_time(e1) * 1e-3 / reps
    d, L, c = cfg.embed_dim, cfg.seq_len, cfg.in_vocab
    d_flops = Bd * (2 * L * d * (3 * d + d + 8 * d + c) + 4 * L * L * d)
    d_tf = d_flops / d_sec / 1e12
    tokens = B * L
    return {"metric": "VQ tokenizer quantize tokens/s", "value": round(tokens / q_sec, 1),
            "unit": "tokens/s", "ms_per_quantize": round(q_sec * 1e3, 4),
            "encode_with_ids_tokens_per_s": round(tokens / e_sec, 1),
            "config": {"workload": "upstream VQ-VAE tokenizer, WMT14 configuration, fp32",
                       "batch": B, "seq_len": L, "d": d, "levels": list(cfg.levels),
                       "codes": cfg.vocab_sizes[0], "cascade": cfg.cascade_strides()},
            "flops_per_sequence": fl,
            "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": FP32_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tf / FP32_PEAK_TFLOPS, 4)},
            "decode": {"batch": Bd, "ms": round(d_sec * 1e3, 4),
                       "tokens_per_s": round(Bd * L / d_sec, 1), "flops": d_flops,
                       "roofline": {"bound": "mfma", "achieved": round(d_tf, 2),
                                    "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                                    "frac": round(d_tf / FP32_PEAK_TFLOPS, 4)}}}


def cpu_vq_tokenizer_baseline(seqs=24):
    """The float64 oracle's quantizer (numpy, BLAS held to one thread) on
    `seqs` sequences of the WMT14 configuration with random weights."""
    from threadpoolctl import threadpool_limits

    from oracle import vq_tokenizer as vo

    cfg = vo.WMT14
    enc, qw, _ = vo.random_weights(cfg, seed=31, vocab_cap=1024)
    ids = np.random.default_rng(32).integers(0, 1024, (seqs, cfg.seq_len))
    z = vo.encode_front(cfg, ids, enc["wte"], enc["wpe"])
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        vo.quantize(cfg, qw, z)
        dt = time.perf_counter() - t0
    return {"value": seqs * cfg.seq_len / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"{seqs} sequences of 64 tokens, all 11 levels, float64 numpy oracle, "
                      "1 BLAS thread"}


def run_weight_upload(torch, mib=512):
    """Device weight path: one bf16 tensor of `mib` MiB in a safetensors file
    (written first, so it is in the page cache) copied to HBM as stored
    through the pinned staging of ncm_st_upload; host-to-device GB/s."""
    import tempfile

    from ncmorph_amd import safetensors as st

    n = mib * 2**20 // 2
    raw = np.random.default_rng(14).integers(0, 2**16, n, dtype=np.uint16).tobytes()
    dev = torch.device("cuda", 0)
    out = torch.empty(n, dtype=torch.int16, device=dev)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "w.safetensors")
        st.write_file(path, {"w": ("BF16", (n,), raw)})
        with st.SafetensorsFile(path) as f:
            f.upload("w", out)
            torch.cuda.synchronize()
            reps = 3
            t0 = time.perf_counter()
            for _ in range(reps):
                f.upload("w", out)
            torch.cuda.synchronize()
            sec = (time.perf_counter() - t0) / reps
    gbs = n * 2 / sec / 1e9
    return {"bytes": n * 2, "ms": round(sec * 1e3, 2),
            "roofline": {"bound": "pcie", "achieved": round(gbs, 1), "peak": PCIE_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / PCIE_PEAK_GBS, 4)}}


def cpu_decoder_baseline():
    """Oracle decoder (scalar restatements, 1 thread) of the same model shape
    on 4 tokens: once with no layers and an LM head of 8192 vocabulary rows,
    once with one layer added. The 16-layer, 128256-row forward is
    extrapolated from the two (attention grows with the sequence and is
    undercounted at 4 tokens; it is under 6% of the FLOPs at 1024)."""
    from ncmorph_amd import decoder
    from oracle import pyoracle

    spec = decoder.LLAMA_3_2_1B
    rng = np.random.default_rng(13)
    rb = pyoracle.round_bf16

    def w(*shape):
        return rb((rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)))

    tok, vocab_rows = 4, 8192
    layer = dict(input_norm=np.ones(spec.hidden, np.float32),
                 qkv_weight=w(spec.qkv_width, spec.hidden), qkv_bias=None,
                 o_weight=w(spec.hidden, spec.q_heads * spec.head_dim), o_bias=None,
                 post_attention_norm=np.ones(spec.hidden, np.float32),
                 gate_up_weight=w(2 * spec.intermediate, spec.hidden), gate_up_bias=None,
                 down_weight=w(spec.hidden, spec.intermediate), down_bias=None)
    embed = w(vocab_rows, spec.hidden)
    fn = np.ones(spec.hidden, np.float32)
    cos, sin = decoder.rope_tables(spec, tok)
    ids = rng.integers(0, vocab_rows, tok)
    args = (spec.q_heads, spec.kv_heads, spec.head_dim, spec.rms_eps)
    t0 = time.perf_counter()
    pyoracle.decoder_forward(ids, embed, [], fn, None, cos, sin, *args)
    t_head = time.perf_counter() - t0
    t0 = time.perf_counter()
    pyoracle.decoder_forward(ids, embed, [layer], fn, None, cos, sin, *args)
    t_layer = max(time.perf_counter() - t0 - t_head, 0.0)
    per_forward = t_head * spec.vocab / vocab_rows + spec.layers * t_layer
    return {"value": round(tok / per_forward, 4), "unit": "tokens/s", "cores": 1,
            "kind": "port",
            "sample": f"{tok} tokens through the oracle decoder of the 1B shape with 0 and 1 "
                      f"layers and an LM head of {vocab_rows} rows, 1 thread; 16 layers and "
                      f"{spec.vocab} rows extrapolated"}


def cpu_linear_baseline():
    """Oracle (scalar restatement of matmul_bf16, 1 thread) on a 24-row slice
    of each shape, extrapolated linearly in M."""
    from ncmorph_amd import synth
    from oracle import pyoracle

    rows = 24
    t_total = 0.0
    for (n, k) in LINEAR_NK:
        xb = synth.normal_bf16(synth.LINEAR_SEED_X + k, (rows, k))
        wb = synth.normal_bf16(synth.LINEAR_SEED_W + n * 7 + k, (n, k), std=0.02)
        t0 = time.perf_counter()
        pyoracle.matmul_bf16_u16_rows(xb, wb, 0, rows)
        t_total += (time.perf_counter() - t0) * (LINEAR_M / rows)
    flops = sum(2.0 * LINEAR_M * n * k for (n, k) in LINEAR_NK)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"first {rows} rows of x for each of the 3 shapes, oracle matmul_bf16 "
                      "(pair-FMA, FTZ, K-blocks), 1 thread, extrapolated to M=2048"}


def cpu_linear_baseline_ncores():
    """The same oracle on a 384-row slice of each shape, rows split over
    cpu_threads() host threads (rows are independent, so the outputs are the
    1-thread ones), extrapolated linearly in M."""
    from concurrent.futures import ThreadPoolExecutor

    from ncmorph_amd import synth
    from oracle import pyoracle

    nt = cpu_threads()
    rows = 24 * nt
    t_total = 0.0
    for (n, k) in LINEAR_NK:
        xb = synth.normal_bf16(synth.LINEAR_SEED_X + k, (rows, k))
        wb = synth.normal_bf16(synth.LINEAR_SEED_W + n * 7 + k, (n, k), std=0.02)
        step = rows // nt
        t0 = time.perf_counter()
        with ThreadPoolExecutor(nt) as ex:
            list(ex.map(lambda i: pyoracle.matmul_bf16_u16_rows(xb, wb, i * step, (i + 1) * step),
                        range(nt)))
        t_total += (time.perf_counter() - t0) * (LINEAR_M / rows)
    flops = sum(2.0 * LINEAR_M * n * k for (n, k) in LINEAR_NK)
    return {"value": flops / t_total / 1e12, "unit": "TFLOP/s", "cores": nt, "kind": "port",
            "sample": f"first {rows} rows of x for each of the 3 shapes, oracle matmul_bf16 "
                      f"rows split over {nt} threads, extrapolated to M=2048"}


def cpu_rvq_baseline_ncores():
    """Oracle encode of one whole sequence (2048 positions, all 8 levels)
    with each level's rows split over cpu_threads() host threads."""
    from ncmorph_amd import synth
    from oracle import pyoracle

    c = synth.RVQ_LARGE
    nt = cpu_threads()
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    xs = np.ascontiguousarray(x[:1])
    del x
    csq = pyoracle.rvq_csq(cb)
    t0 = time.perf_counter()
    pyoracle.rvq_encode(xs, cb, c["strides"], csq=csq, want_gap=False, threads=nt)
    dt = time.perf_counter() - t0
    return {"value": c["t"] / dt, "unit": "tokens/s", "cores": nt, "kind": "port",
            "sample": f"sequence 0 (2048 positions), all 8 levels, 4096 codes/level, d=2048, "
                      f"oracle exhaustive search, each level's rows over {nt} threads"}


def cpu_rvq_baseline():
    """Oracle encode (exhaustive fp32 search, 1 thread) of the first 256
    positions of sequence 0, all 8 levels."""
    from ncmorph_amd import synth
    from oracle import pyoracle

    c = synth.RVQ_LARGE
    t = 256
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    xs = np.ascontiguousarray(x[:1, :t])
    del x
    csq = pyoracle.rvq_csq(cb)
    t0 = time.perf_counter()
    pyoracle.rvq_encode(xs, cb, c["strides"], csq=csq, want_gap=False, threads=1)
    dt = time.perf_counter() - t0
    return {"value": t / dt, "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": f"sequence 0, positions 0..{t - 1}, all 8 levels (strides 128..1), "
                      "4096 codes/level, d=2048, oracle exhaustive search, 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Every timed section first runs its own work untimed for RAMP_MS (the
    # engine clock's ramp), then its warmup, then exactly its timed steps.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", choices=["linear", "rvq", "decoder", "ncm", "attention", "vqtok", "all",
                                       "copy"],
                    default="all",
                    help="copy: a plain 256 MiB device copy, the reference point for "
                         "the FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1"}))
        sys.exit(2)

    import torch

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    import ncmorph_amd  # noqa: F401  (raises if the HIP library is missing)

    torch.cuda.init()
    if args.only == "copy":
        n = 64 * 1024 * 1024
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_per_launch": n * 4, "launches": 5}))
        return
    res = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (SplitMix64 + Box-Muller normals, fixed seeds)"}
    if args.only in ("linear", "all"):
        lin = run_linear(torch, args.steps, args.warmup)
        tflops = lin["flops_per_step"] / lin["step_s"] / 1e12
        res.update({"value": round(tflops, 2), "unit": "TFLOP/s",
                    "ms_per_step": round(lin["step_s"] * 1e3, 4)})
        res["config"] = {"workload": "bf16-weight linear y = x W^T at Llama-3.2-1B shapes",
                         "m": LINEAR_M, "nk": [list(nk) for nk in LINEAR_NK],
                         "accumulate": "fp32", "output": "fp32"}
        res["roofline"] = {"bound": "mfma", "achieved": round(tflops, 2),
                           "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                           "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                           "traffic": LINEAR_TRAFFIC_BYTES_PER_LAUNCH,
                           "flops_per_launch": lin["flops_per_step"] / len(LINEAR_NK),
                           "avg_launch_us": round(lin["step_s"] / len(LINEAR_NK) * 1e6, 3)}
        res["linear_per_shape"] = {
            f"{LINEAR_M}x{n}x{k}": {
                "us": round(t * 1e6, 2),
                "tflops": round(2.0 * LINEAR_M * n * k / t / 1e12, 2),
                "frac": round(2.0 * LINEAR_M * n * k / t / 1e12 / BF16_PEAK_TFLOPS, 4)}
            for (n, k), t in lin["per_shape_s"].items()}
        res["linear_max_abs_err_vs_fp32"] = lin["max_abs_err_vs_fp32"]
        res["linear_hipblaslt_bf16_out_per_shape_us"] = {
            f"{LINEAR_M}x{n}x{k}": round(t * 1e6, 2) for (n, k), t in
            lin["vendor_per_shape_s"].items()}
        res["linear_hipblaslt_f32_out_per_shape_us"] = None if lin["vendor_f32_per_shape_s"] is None \
            else {f"{LINEAR_M}x{n}x{k}": round(t * 1e6, 2) for (n, k), t in
                  lin["vendor_f32_per_shape_s"].items()}
        if not args.no_cpu:
            res["cpu_baseline"] = cpu_linear_baseline()
            res["cpu_baseline_ncores"] = cpu_linear_baseline_ncores()
    if args.only in ("linear", "all"):
        res["decoder_ops"] = run_decoder_ops(torch)
    if args.only in ("rvq", "all"):
        rv = run_rvq(torch, max(10, args.steps // 2), max(1, args.warmup // 5))
        tps = rv["tokens"] / rv["encode_s"]
        tf = rv["flops"] / rv["encode_s"] / 1e12
        gbs = rv["bytes"] / rv["encode_s"] / 1e9
        rvq = {"metric": "RVQ-encode tokens/s", "value": round(tps, 1), "unit": "tokens/s",
               "ms_per_encode": round(rv["encode_s"] * 1e3, 4),
               "config": {"workload": "multiscale RVQ encode + reconstruction",
                          "b": 16, "t": 2048, "d": 2048, "levels": 8, "v": 4096,
                          "strides": [128, 64, 32, 16, 8, 4, 2, 1]},
               "roofline": {"bound": "mfma", "achieved": round(tf, 2),
                            "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                            "traffic": RVQ_TRAFFIC_BYTES_PER_ENCODE,
                            "hbm_gbs_algorithmic": round(gbs, 1),
                            "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
               "flagged_rows": rv["n_flagged"],
               # Per level: rows that needed any exact distance (the rest had
               # one candidate under the error bound) and rows with an
               # incomplete candidate chunk.
               "rescored_rows_per_level": rv["rescored"],
               "near_ties": {"count": rv["near_ties"], "codes": rv["codes"],
                             "rel_gap_below": NEAR_TIE_REL}}
        if not args.no_cpu:
            rvq["cpu_baseline"] = cpu_rvq_baseline()
            rvq["cpu_baseline_ncores"] = cpu_rvq_baseline_ncores()
        res["rvq_encode"] = rvq
        if "value" not in res:
            res.update({"value": rvq["value"], "unit": "tokens/s",
                        "ms_per_step": rvq["ms_per_encode"], "config": rvq["config"],
                        "roofline": rvq["roofline"]})
            if "cpu_baseline" in rvq:
                res["cpu_baseline"] = rvq["cpu_baseline"]
    if args.only == "ncm":
        res["ncm_level_step"] = run_ncm_step(torch)
    if args.only == "attention":
        res["ncm_level_attention"] = run_ncm_attention(torch)
    if args.only in ("vqtok", "all"):
        vq = run_vq_tokenizer(torch)
        if not args.no_cpu:
            vq["cpu_baseline"] = cpu_vq_tokenizer_baseline()
        res["vq_tokenizer"] = vq
    if args.only in ("decoder", "all"):
        dec = run_decoder(torch)
        dec["weight_upload"] = run_weight_upload(torch)
        dec["ncm_level_attention"] = run_ncm_attention(torch)
        dec["ncm_tied_head"] = run_ncm_tied_head(torch)
        res["ncm_level_step"] = run_ncm_step(torch)
        if not args.no_cpu:
            dec["cpu_baseline"] = cpu_decoder_baseline()
        res["decoder_prefill"] = dec
        if "value" not in res:
            res.update({"value": dec["value"], "unit": "tokens/s",
                        "ms_per_step": dec["ms_per_forward"], "config": dec["config"],
                        "roofline": dec["roofline"]})
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
