"""NCM level-parallel step on the GPU: the body of src/ncm_model.zig:89-250
(ncm_ncm_forward_dev) and the codebook-tied code heads that read its level
positions (PROJECT.md:222).

The body is one C-ABI call in the bf16 mode of the source decoder; this
module holds the model description (the reference's config_t / weights_t
field names), device weights in the layout that call reads (q|k|v rows
fused as the reference's fused_qkv_weight, gate and up rows interleaved in
groups of 32), random initialisation for synthetic runs, the positions
that restart at every level (src/ncm_position.zig:11-22) and the RoPE
tables gathered at them, built on the host with the system libm as the
reference does (src/ncm_position.zig:73-118).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import _check as _ck
from . import decoder as _dec
from ._lib import NcmError, check, lib
from .context import default_context

MAX_LEVELS = 32
MASK_MODES = {"block_diagonal": 0, "block_causal": 1, "causal": 2}


@dataclass
class NcmSpec:
    """config_t (src/ncm_model.zig:15-35) of the level-parallel body."""

    hidden: int
    vq_width: int
    intermediate: int
    q_heads: int
    kv_heads: int
    head_dim: int
    layers: int
    level_lengths: tuple
    prefix_length: int
    prefix_vocab: int
    query_level0: bool = True
    use_level_encoding: bool = True
    mask: str = "block_diagonal"
    window: int = 0
    rms_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_llama3: tuple | None = (8.0, 1.0, 4.0, 8192)

    @property
    def seq_len(self) -> int:
        return self.prefix_length + int(sum(self.level_lengths))

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


def multiscale_levels(positions: int, levels: int) -> tuple:
    """Level lengths of a multiscale RVQ over `positions` positions: level l
    has positions / 2^(levels - 1 - l) (coarsest first)."""
    return tuple(positions >> (levels - 1 - l) for l in range(levels))


# Llama-3-8B-shaped body predicting 8 RVQ levels (codebook 8192, d = 4096)
# of one 4096-position sequence after a 64-token prefix.
LLAMA_3_8B_NCM = NcmSpec(hidden=4096, vq_width=4096, intermediate=14336, q_heads=32,
                         kv_heads=8, head_dim=128, layers=32,
                         level_lengths=multiscale_levels(4096, 8), prefix_length=64,
                         prefix_vocab=128256, mask="block_causal")


class _Shape(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("vq_width", C.c_int64), ("intermediate", C.c_int64),
                ("q_heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("layers", C.c_int32), ("prefix_length", C.c_int64),
                ("prefix_vocab", C.c_int64), ("n_levels", C.c_int32),
                ("mask_mode", C.c_int32), ("query_level0", C.c_int32),
                ("use_level_encoding", C.c_int32), ("window", C.c_int64),
                ("rms_eps", C.c_float), ("reserved", C.c_int32),
                ("level_lengths", C.c_int64 * MAX_LEVELS)]


class _Weights(C.Structure):
    _fields_ = [("prefix_token_embedding", C.c_void_p), ("input_projection", C.c_void_p),
                ("input_projection_bias", C.c_void_p), ("level_embedding", C.c_void_p),
                ("l0_queries", C.c_void_p), ("final_norm", C.c_void_p),
                ("final_norm_bias", C.c_void_p), ("conv_weight", C.c_void_p),
                ("conv_bias", C.c_void_p)]


@dataclass
class NcmWeights:
    """Device weights: bf16 tensors for tables and projections, float32 for
    norm scales, biases of norms and the fp32 convolutions. layers[i] maps
    the decoder's layer field names (ncmorph_amd.decoder._LAYER_FIELDS) to
    tensors; convs: [] or one dict(weight [vq, vq, 3] f32, bias [vq] f32) per
    level."""

    prefix_token_embedding: object
    input_projection: object
    input_projection_bias: object
    level_embedding: object
    l0_queries: object
    final_norm: object
    final_norm_bias: object = None
    layers: list = field(default_factory=list)
    convs: list = field(default_factory=list)


def random_weights(spec: NcmSpec, device, seed: int = 0, std: float = 0.02) -> NcmWeights:
    """Random-init bf16 weights of spec's shape (~N(0, std); tables and level
    queries ~N(0, 1)), norm scales 1, no biases, QK-norm or convolutions."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def w(*shape, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s).to(torch.bfloat16)

    base = _dec.DecoderSpec(hidden=spec.hidden, intermediate=spec.intermediate, vocab=1,
                            q_heads=spec.q_heads, kv_heads=spec.kv_heads,
                            head_dim=spec.head_dim, layers=spec.layers)
    layers = _dec.random_weights(base, device, seed=seed + 1, std=std).layers
    return NcmWeights(
        prefix_token_embedding=w(spec.prefix_vocab, spec.vq_width, s=1.0),
        input_projection=w(spec.hidden, spec.vq_width),
        input_projection_bias=w(spec.hidden),
        level_embedding=w(len(spec.level_lengths), spec.hidden),
        l0_queries=w(spec.level_lengths[0], spec.vq_width, s=1.0) if spec.query_level0 else None,
        final_norm=torch.ones(spec.hidden, device=device),
        layers=layers)


def device_weights(spec: NcmSpec, ref: dict, device) -> NcmWeights:
    """Device form of weights in the reference's weights_t layout (numpy
    float32 arrays holding bf16 values, per-layer dicts with the
    layer_weights_t names): fused q|k|v rows kept, gate and up rows
    interleaved, bf16 tensors as bit patterns."""
    import torch

    from . import kernels

    def bf(a):
        if a is None:
            return None
        bits = np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32) >> 16
        return torch.from_numpy(bits.astype(np.uint16).view(np.int16)).to(device).view(
            torch.bfloat16)

    def f32(a):
        return None if a is None else torch.from_numpy(
            np.ascontiguousarray(a, np.float32)).to(device)

    layers = []
    for L in ref["layers"]:
        gb, ub = L.get("gate_bias"), L.get("up_bias")
        layers.append({
            "input_norm": f32(L["ln_1_weight"]),
            "qkv_weight": bf(L["fused_qkv_weight"]),
            "qkv_bias": bf(L.get("fused_qkv_bias")),
            "o_weight": bf(L["output_weight"]),
            "o_bias": bf(L.get("output_bias")),
            "post_attention_norm": f32(L["ln_2_weight"]),
            "gate_up_weight": bf(kernels.interleave_gate_up(np.asarray(L["gate_weight"]),
                                                             np.asarray(L["up_weight"]))),
            "gate_up_bias": None if gb is None else bf(kernels.interleave_gate_up(
                np.asarray(gb).reshape(-1, 1), np.asarray(ub).reshape(-1, 1)).ravel()),
            "down_weight": bf(L["down_weight"]),
            "down_bias": bf(L.get("down_bias")),
            "q_norm": f32(L.get("query_norm_weight")),
            "k_norm": f32(L.get("key_norm_weight")),
            "input_norm_bias": f32(L.get("ln_1_bias")),
            "post_attention_norm_bias": f32(L.get("ln_2_bias")),
        })
    convs = [dict(weight=f32(c["weight"]), bias=f32(c["bias"]))
             for c in (ref.get("post_upsample_convs") or [])]
    return NcmWeights(
        prefix_token_embedding=bf(ref["prefix_token_embedding"]),
        input_projection=bf(ref["input_projection"]),
        input_projection_bias=bf(ref["input_projection_bias"]),
        level_embedding=bf(ref["level_embedding"]),
        l0_queries=bf(ref.get("l0_queries")),
        final_norm=f32(ref["final_norm_weight"]),
        final_norm_bias=f32(ref.get("final_norm_bias")),
        layers=layers, convs=convs)


def level_positions(spec: NcmSpec) -> np.ndarray:
    """fill_level_positions (src/ncm_position.zig:11-22)."""
    return np.concatenate([np.arange(spec.prefix_length)] +
                          [np.arange(n) for n in spec.level_lengths]).astype(np.int64)


def rope_tables(spec: NcmSpec):
    """cosine, sine float32 [S, head_dim]: the tables over 0 .. max position
    (system libm, as the reference), gathered at the restarting positions
    (src/ncm_position.zig:73-118)."""
    pos = level_positions(spec)
    cos, sin = _dec.rope_tables(spec, int(pos.max()) + 1)
    return np.ascontiguousarray(cos[pos]), np.ascontiguousarray(sin[pos])


def forward(spec: NcmSpec, weights: NcmWeights, prefix_ids, target_inputs, cosine, sine,
            prefix_pad_mask=None, out=None, ctx=None, hidden_states: bool = False):
    """Final-normalized hidden states float32 [S, hidden] (bf16 values) of
    the NCM body for one prefix (host ints [prefix_length]) and the target
    inputs (float32 device [sum level_lengths, vq_width]); cosine / sine:
    float32 device [S, head_dim] (rope_tables). Runs on torch's current
    stream. hidden_states=True also returns forward_with_trace's states
    (src/ncm_model.zig:89-250) float32 [layers + 1, S, hidden]: (out,
    states)."""
    import torch

    W = "ncm_forward"
    if len(spec.level_lengths) > MAX_LEVELS or spec.mask not in MASK_MODES:
        raise NcmError(-2, W, "too many levels or an unknown mask")
    ids = np.ascontiguousarray(prefix_ids, dtype=np.int64).ravel()
    if ids.size != spec.prefix_length:
        raise NcmError(-3, W, "prefix_ids must hold prefix_length ids")
    pad = None if prefix_pad_mask is None else np.ascontiguousarray(prefix_pad_mask, np.uint8)
    S, T = spec.seq_len, int(sum(spec.level_lengths))
    a = _ck.Args(W)
    a.dev(target_inputs, "target_inputs", _ck.F32, (T, spec.vq_width))
    a.dev(cosine, "cosine", _ck.F32, (S, spec.head_dim))
    a.dev(sine, "sine", _ck.F32, (S, spec.head_dim))
    nl = len(spec.level_lengths)
    a.dev(weights.prefix_token_embedding, "prefix_token_embedding", _ck.BF16,
          (spec.prefix_vocab, spec.vq_width))
    a.dev(weights.input_projection, "input_projection", _ck.BF16, (spec.hidden, spec.vq_width))
    a.dev(weights.input_projection_bias, "input_projection_bias", _ck.BF16, (spec.hidden,))
    a.dev(weights.level_embedding, "level_embedding", _ck.BF16, (nl, spec.hidden))
    a.dev(weights.l0_queries, "l0_queries", _ck.BF16, (spec.level_lengths[0], spec.vq_width),
          optional=not spec.query_level0)
    a.dev(weights.final_norm, "final_norm", _ck.F32, (spec.hidden,))
    a.dev(weights.final_norm_bias, "final_norm_bias", _ck.F32, (spec.hidden,), optional=True)
    if len(weights.layers) != spec.layers:
        raise NcmError(-3, W, "one weight dict per layer")
    for i, L in enumerate(weights.layers):
        _dec.check_layer(a, L, spec, f"layers[{i}].")
    if weights.convs and len(weights.convs) != nl:
        raise NcmError(-3, W, "one convolution per level, or none")
    for i, c in enumerate(weights.convs):
        a.dev(c["weight"], f"convs[{i}].weight", _ck.F32, (spec.vq_width, spec.vq_width, 3))
        a.dev(c["bias"], f"convs[{i}].bias", _ck.F32, (spec.vq_width,))
    if out is None:
        out = torch.empty((S, spec.hidden), dtype=torch.float32, device=target_inputs.device)
    po = a.dev(out, "out", _ck.F32, (S, spec.hidden))
    states = (torch.empty((spec.layers + 1, S, spec.hidden), dtype=torch.float32,
                          device=target_inputs.device) if hidden_states else None)
    a.done()

    ptr = lambda t: None if t is None else t.data_ptr()
    shape = _Shape(spec.hidden, spec.vq_width, spec.intermediate, spec.q_heads, spec.kv_heads,
                   spec.head_dim, spec.layers, spec.prefix_length, spec.prefix_vocab, nl,
                   MASK_MODES[spec.mask], int(spec.query_level0), int(spec.use_level_encoding),
                   spec.window, spec.rms_eps, 0)
    for l, n in enumerate(spec.level_lengths):
        shape.level_lengths[l] = int(n)
    cw = cb = None
    if weights.convs:
        cw = (C.c_void_p * nl)(*[ptr(c["weight"]) for c in weights.convs])
        cb = (C.c_void_p * nl)(*[ptr(c["bias"]) for c in weights.convs])
    wts = _Weights(ptr(weights.prefix_token_embedding), ptr(weights.input_projection),
                   ptr(weights.input_projection_bias), ptr(weights.level_embedding),
                   ptr(weights.l0_queries), ptr(weights.final_norm),
                   ptr(weights.final_norm_bias), C.cast(cw, C.c_void_p) if cw else None,
                   C.cast(cb, C.c_void_p) if cb else None)
    arr = (_dec._Layer * spec.layers)()
    for i, L in enumerate(weights.layers):
        arr[i] = _dec._Layer(*[ptr(L.get(n)) for n in _dec._LAYER_FIELDS])
    ctx = ctx or default_context(target_inputs.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_ncm_forward_dev(
        ctx.handle, C.byref(shape), arr, C.byref(wts), ids.ctypes.data_as(C.c_void_p),
        None if pad is None else pad.ctypes.data_as(C.c_void_p), 0 if pad is None else pad.size,
        C.c_void_p(target_inputs.data_ptr()), C.c_void_p(cosine.data_ptr()),
        C.c_void_p(sine.data_ptr()), po,
        None if states is None else C.c_void_p(states.data_ptr())), W)
    return (out, states) if hidden_states else out


def code_head_logits(spec: NcmSpec, hidden, z_weights, codebooks, csq, log_inv_t=None,
                     bias=None, ctx=None):
    """The codebook-tied code heads (PROJECT.md:222, upstream
    _TiedCodebookHead) of every level from the body's output: per level l,
    z = bf16(h_l W_z,l^T) over that level's rows of `hidden` (float32 [S,
    hidden] from forward), then logits = (2 z E_l^T - |E_l|^2) *
    exp(log_inv_t[l]) / mean |E_l|^2 (+ bias[l]), all levels in one launch.
    z_weights: bf16 [levels, d, hidden]; codebooks: bf16 [levels, v, d];
    csq: float32 [levels, v]. Returns float32 [sum level_lengths, v]."""
    import torch

    from . import kernels

    nl = len(spec.level_lengths)
    L, d, H = _ck.dims(z_weights, "z_weights", "code_head_logits", 3)
    if L != nl or H != spec.hidden:
        raise NcmError(-2, "code_head_logits", "z_weights must be [levels, d, hidden]")
    T = int(sum(spec.level_lengths))
    h16 = kernels.bf16_from_f32(hidden[spec.prefix_length:], ctx=ctx)
    z = torch.empty((T, d), dtype=torch.bfloat16, device=hidden.device)
    off = 0
    for l, n in enumerate(spec.level_lengths):
        if n:
            kernels.linear_bf16(h16[off:off + n], z_weights[l], out=z[off:off + n],
                                out_mode="bf16", ctx=ctx)
        off += n
    return kernels.tied_head_logits_levels(z, codebooks, csq, list(spec.level_lengths),
                                           log_inv_t=log_inv_t, bias=bias, ctx=ctx)


class _WeightsF32(C.Structure):
    _fields_ = [("prefix_token_embedding", C.c_void_p), ("input_projection", C.c_void_p),
                ("input_projection_bias", C.c_void_p), ("level_embedding", C.c_void_p),
                ("l0_queries", C.c_void_p), ("final_norm", C.c_void_p),
                ("final_norm_bias", C.c_void_p), ("conv_weight", C.c_void_p),
                ("conv_bias", C.c_void_p)]


def device_weights_f32(spec: NcmSpec, ref: dict, device) -> NcmWeights:
    """Float32 device weights for forward_f32 from the reference's weights_t
    layout (numpy float32 arrays, per-layer dicts with the layer_weights_t
    names): fused q|k|v rows, gate / up / down as stored, the ln biases as
    the norm biases."""
    import torch

    def f32(a):
        return None if a is None else torch.from_numpy(
            np.ascontiguousarray(a, np.float32)).to(device)

    layers = []
    for L in ref["layers"]:
        layers.append({
            "input_norm": f32(L["ln_1_weight"]), "qkv_weight": f32(L["fused_qkv_weight"]),
            "qkv_bias": f32(L.get("fused_qkv_bias")), "o_weight": f32(L["output_weight"]),
            "o_bias": f32(L.get("output_bias")), "post_attention_norm": f32(L["ln_2_weight"]),
            "gate_weight": f32(L["gate_weight"]), "gate_bias": f32(L.get("gate_bias")),
            "up_weight": f32(L["up_weight"]), "up_bias": f32(L.get("up_bias")),
            "down_weight": f32(L["down_weight"]), "down_bias": f32(L.get("down_bias")),
            "q_norm": f32(L.get("query_norm_weight")), "k_norm": f32(L.get("key_norm_weight")),
            "input_norm_bias": f32(L.get("ln_1_bias")),
            "post_attention_norm_bias": f32(L.get("ln_2_bias")),
        })
    convs = [dict(weight=f32(c["weight"]), bias=f32(c["bias"]))
             for c in (ref.get("post_upsample_convs") or [])]
    return NcmWeights(
        prefix_token_embedding=f32(ref["prefix_token_embedding"]),
        input_projection=f32(ref["input_projection"]),
        input_projection_bias=f32(ref.get("input_projection_bias")),
        level_embedding=f32(ref["level_embedding"]),
        l0_queries=f32(ref.get("l0_queries")),
        final_norm=f32(ref["final_norm_weight"]),
        final_norm_bias=f32(ref.get("final_norm_bias")),
        layers=layers, convs=convs)


def forward_f32(spec: NcmSpec, weights: NcmWeights, prefix_ids, target_inputs, cosine, sine,
                prefix_pad_mask=None, out=None, ctx=None, hidden_states: bool = False):
    """The NCM body in the reference's f32 arithmetic (forward_with_trace,
    src/ncm_model.zig:89-250): final-normalized hidden states float32 [S,
    hidden]. Arguments as forward, with float32 weights (device_weights_f32;
    layers[i] maps the names of decoder._LAYER_F32_FIELDS); hidden_states as
    forward."""
    import torch

    W = "ncm_forward_f32"
    if len(spec.level_lengths) > MAX_LEVELS or spec.mask not in MASK_MODES:
        raise NcmError(-2, W, "too many levels or an unknown mask")
    ids = np.ascontiguousarray(prefix_ids, dtype=np.int64).ravel()
    if ids.size != spec.prefix_length:
        raise NcmError(-3, W, "prefix_ids must hold prefix_length ids")
    pad = None if prefix_pad_mask is None else np.ascontiguousarray(prefix_pad_mask, np.uint8)
    S, T = spec.seq_len, int(sum(spec.level_lengths))
    H, I, hd, vq = spec.hidden, spec.intermediate, spec.head_dim, spec.vq_width
    qkv, qw = (spec.q_heads + 2 * spec.kv_heads) * hd, spec.q_heads * hd
    nl = len(spec.level_lengths)
    a = _ck.Args(W)
    a.dev(target_inputs, "target_inputs", _ck.F32, (T, vq))
    a.dev(cosine, "cosine", _ck.F32, (S, hd))
    a.dev(sine, "sine", _ck.F32, (S, hd))
    a.dev(weights.prefix_token_embedding, "prefix_token_embedding", _ck.F32,
          (spec.prefix_vocab, vq))
    a.dev(weights.input_projection, "input_projection", _ck.F32, (H, vq))
    a.dev(weights.input_projection_bias, "input_projection_bias", _ck.F32, (H,), optional=True)
    a.dev(weights.level_embedding, "level_embedding", _ck.F32, (nl, H),
          optional=not spec.use_level_encoding)
    a.dev(weights.l0_queries, "l0_queries", _ck.F32, (spec.level_lengths[0], vq),
          optional=not spec.query_level0)
    a.dev(weights.final_norm, "final_norm", _ck.F32, (H,))
    a.dev(weights.final_norm_bias, "final_norm_bias", _ck.F32, (H,), optional=True)
    if len(weights.layers) != spec.layers:
        raise NcmError(-3, W, "one weight dict per layer")
    shapes = {"input_norm": (H,), "qkv_weight": (qkv, H), "qkv_bias": (qkv,), "o_weight": (H, qw),
              "o_bias": (H,), "post_attention_norm": (H,), "gate_weight": (I, H),
              "gate_bias": (I,), "up_weight": (I, H), "up_bias": (I,), "down_weight": (H, I),
              "down_bias": (H,), "q_norm": (hd,), "k_norm": (hd,), "input_norm_bias": (H,),
              "post_attention_norm_bias": (H,)}
    required = {"input_norm", "qkv_weight", "o_weight", "post_attention_norm", "gate_weight",
                "up_weight", "down_weight"}
    for i, L in enumerate(weights.layers):
        for f in _dec._LAYER_F32_FIELDS:
            a.dev(L.get(f), f"layers[{i}].{f}", _ck.F32, shapes[f], optional=f not in required)
    if weights.convs and len(weights.convs) != nl:
        raise NcmError(-3, W, "one convolution per level, or none")
    for i, c in enumerate(weights.convs):
        a.dev(c["weight"], f"convs[{i}].weight", _ck.F32, (vq, vq, 3))
        a.dev(c["bias"], f"convs[{i}].bias", _ck.F32, (vq,))
    if out is None:
        out = torch.empty((S, H), dtype=torch.float32, device=target_inputs.device)
    po = a.dev(out, "out", _ck.F32, (S, H))
    states = (torch.empty((spec.layers + 1, S, H), dtype=torch.float32,
                          device=target_inputs.device) if hidden_states else None)
    a.done()

    ptr = lambda t: None if t is None else t.data_ptr()
    shape = _Shape(H, vq, I, spec.q_heads, spec.kv_heads, hd, spec.layers, spec.prefix_length,
                   spec.prefix_vocab, nl, MASK_MODES[spec.mask], int(spec.query_level0),
                   int(spec.use_level_encoding), spec.window, spec.rms_eps, 0)
    for l, n in enumerate(spec.level_lengths):
        shape.level_lengths[l] = int(n)
    cw = cb = None
    if weights.convs:
        cw = (C.c_void_p * nl)(*[ptr(c["weight"]) for c in weights.convs])
        cb = (C.c_void_p * nl)(*[ptr(c["bias"]) for c in weights.convs])
    wts = _WeightsF32(ptr(weights.prefix_token_embedding), ptr(weights.input_projection),
                      ptr(weights.input_projection_bias), ptr(weights.level_embedding),
                      ptr(weights.l0_queries), ptr(weights.final_norm),
                      ptr(weights.final_norm_bias), C.cast(cw, C.c_void_p) if cw else None,
                      C.cast(cb, C.c_void_p) if cb else None)
    arr = (_dec._LayerF32 * spec.layers)()
    for i, L in enumerate(weights.layers):
        arr[i] = _dec._LayerF32(*[ptr(L.get(n)) for n in _dec._LAYER_F32_FIELDS])
    ctx = ctx or default_context(target_inputs.device.index or 0)
    ctx.bind_stream()
    check(lib().ncm_ncm_forward_f32_dev(
        ctx.handle, C.byref(shape), arr, C.byref(wts), ids.ctypes.data_as(C.c_void_p),
        None if pad is None else pad.ctypes.data_as(C.c_void_p), 0 if pad is None else pad.size,
        C.c_void_p(target_inputs.data_ptr()), C.c_void_p(cosine.data_ptr()),
        C.c_void_p(sine.data_ptr()), po,
        None if states is None else C.c_void_p(states.data_ptr())), W)
    return (out, states) if hidden_states else out
