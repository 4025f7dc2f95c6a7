"""Bf16 decoder prefill forward on the GPU (src/decoder.zig:62-228).

The forward itself is one C-ABI call (ncm_decoder_forward_dev) that
stream-orders the device kernels; this module holds the model description,
device weights in the layout that call reads (q|k|v and gate|up rows
concatenated), random initialisation for synthetic runs, and the RoPE
tables, which the reference builds on the host with the system libm
(packages/kernels/root.zig:305-348, 636-682) and which are built the same
way here.
"""
from __future__ import annotations

import ctypes as C
import ctypes.util
import math
from dataclasses import dataclass, field

import numpy as np

from . import _check as _ck
from ._lib import NcmError, check, lib
from .context import default_context


@dataclass
class DecoderSpec:
    """The config.spec_t fields the bf16 forward reads."""

    hidden: int
    intermediate: int
    vocab: int
    q_heads: int
    kv_heads: int
    head_dim: int
    layers: int
    rms_eps: float = 1e-5
    window: int = 0
    rope_theta: float = 500000.0
    # Llama 3 RoPE scaling (factor, low_freq_factor, high_freq_factor,
    # original_max_position_embeddings); None = default RoPE.
    rope_llama3: tuple | None = (32.0, 1.0, 4.0, 8192)
    tie_word_embeddings: bool = True

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


LLAMA_3_2_1B = DecoderSpec(hidden=2048, intermediate=8192, vocab=128256, q_heads=32, kv_heads=8,
                           head_dim=64, layers=16)


class _Shape(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("intermediate", C.c_int64), ("vocab", C.c_int64),
                ("q_heads", C.c_int32), ("kv_heads", C.c_int32), ("head_dim", C.c_int32),
                ("layers", C.c_int32), ("window", C.c_int64), ("rms_eps", C.c_float)]


_LAYER_FIELDS = ("input_norm", "qkv_weight", "qkv_bias", "o_weight", "o_bias",
                 "post_attention_norm", "gate_up_weight", "gate_up_bias", "down_weight",
                 "down_bias", "q_norm", "k_norm", "input_norm_bias",
                 "post_attention_norm_bias")


class _Layer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _LAYER_FIELDS]


def check_layer(a, L, spec, prefix=""):
    """Name one layer's tensors on the argument checker `a` (dtype and exact
    shape from spec: hidden, intermediate, q_heads, kv_heads, head_dim)."""
    H, I, hd = spec.hidden, spec.intermediate, spec.head_dim
    qkv, qw = (spec.q_heads + 2 * spec.kv_heads) * hd, spec.q_heads * hd
    n = lambda f: prefix + f
    a.dev(L.get("input_norm"), n("input_norm"), _ck.F32, (H,))
    a.dev(L.get("qkv_weight"), n("qkv_weight"), _ck.BF16, (qkv, H))
    a.dev(L.get("qkv_bias"), n("qkv_bias"), _ck.BF16, (qkv,), optional=True)
    a.dev(L.get("o_weight"), n("o_weight"), _ck.BF16, (H, qw))
    a.dev(L.get("o_bias"), n("o_bias"), _ck.BF16, (H,), optional=True)
    a.dev(L.get("post_attention_norm"), n("post_attention_norm"), _ck.F32, (H,))
    a.dev(L.get("gate_up_weight"), n("gate_up_weight"), _ck.BF16, (2 * I, H))
    a.dev(L.get("gate_up_bias"), n("gate_up_bias"), _ck.BF16, (2 * I,), optional=True)
    a.dev(L.get("down_weight"), n("down_weight"), _ck.BF16, (H, I))
    a.dev(L.get("down_bias"), n("down_bias"), _ck.BF16, (H,), optional=True)
    if (L.get("q_norm") is None) != (L.get("k_norm") is None):
        raise NcmError(-1, a.where, n("q_norm and k_norm come together"))
    a.dev(L.get("q_norm"), n("q_norm"), _ck.F32, (hd,), optional=True)
    a.dev(L.get("k_norm"), n("k_norm"), _ck.F32, (hd,), optional=True)
    a.dev(L.get("input_norm_bias"), n("input_norm_bias"), _ck.F32, (H,), optional=True)
    a.dev(L.get("post_attention_norm_bias"), n("post_attention_norm_bias"), _ck.F32, (H,),
          optional=True)


@dataclass
class DecoderWeights:
    """Device weights: bf16 tensors for projections and embeddings, float32
    for norm scales. layers[i] maps the _LAYER_FIELDS names to tensors (the
    bias entries may be None): qkv_weight = rows of q, k, v concatenated;
    gate_up_weight = gate and up rows interleaved in groups of 32
    (kernels.interleave_gate_up)."""

    embed: object
    final_norm: object
    layers: list = field(default_factory=list)
    lm_head: object = None
    # "bf16": the layout above (forward); "f32": float32 tensors with the
    # layer names of _LAYER_F32_FIELDS (forward_f32).
    mode: str = "bf16"


def random_weights(spec: DecoderSpec, device, seed: int = 0, std: float = 0.02,
                   norm_std: float = 0.0, bias_std: float = 0.0) -> DecoderWeights:
    """Random-init weights of spec's shape, ~N(0, std) in bf16, on device.
    Norm scales are 1 (+ N(0, norm_std)); biases are present when bias_std > 0."""
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)

    def w(*shape, s=std):
        return (torch.randn(*shape, generator=g, device=device) * s).to(torch.bfloat16)

    def norm():
        v = torch.ones(spec.hidden, device=device)
        if norm_std:
            v = v + torch.randn(spec.hidden, generator=g, device=device) * norm_std
        return v.contiguous()

    layers = []
    for _ in range(spec.layers):
        layer = {
            "input_norm": norm(),
            "qkv_weight": w(spec.qkv_width, spec.hidden),
            "qkv_bias": w(spec.qkv_width, s=bias_std) if bias_std else None,
            "o_weight": w(spec.hidden, spec.q_heads * spec.head_dim),
            "o_bias": w(spec.hidden, s=bias_std) if bias_std else None,
            "post_attention_norm": norm(),
            "gate_up_weight": w(2 * spec.intermediate, spec.hidden),
            "gate_up_bias": w(2 * spec.intermediate, s=bias_std) if bias_std else None,
            "down_weight": w(spec.hidden, spec.intermediate),
            "down_bias": w(spec.hidden, s=bias_std) if bias_std else None,
        }
        layers.append(layer)
    embed = w(spec.vocab, spec.hidden)
    lm_head = None if spec.tie_word_embeddings else w(spec.vocab, spec.hidden)
    return DecoderWeights(embed=embed, final_norm=norm(), layers=layers, lm_head=lm_head)


_libm = None


def _math_lib():
    global _libm
    if _libm is None:
        m = C.CDLL(ctypes.util.find_library("m") or "libm.so.6")
        for name, args in (("powf", [C.c_float, C.c_float]), ("cosf", [C.c_float]),
                           ("sinf", [C.c_float])):
            fn = getattr(m, name)
            fn.restype = C.c_float
            fn.argtypes = args
        _libm = m
    return _libm


def rope_inverse_frequencies(spec: DecoderSpec) -> np.ndarray:
    """Inverse frequencies in the reference's f32 operation order with the
    system powf (root.zig:305-326, 636-682)."""
    m = _math_lib()
    f32 = np.float32
    hd = spec.head_dim
    inv = np.array([f32(1.0) / f32(m.powf(f32(spec.rope_theta), f32(2 * i) / f32(hd)))
                    for i in range(hd // 2)], np.float32)
    if spec.rope_llama3 is None:
        return inv
    factor, low, high, orig = (f32(spec.rope_llama3[0]), f32(spec.rope_llama3[1]),
                               f32(spec.rope_llama3[2]), int(spec.rope_llama3[3]))
    old_len = f32(orig)
    low_wl = f32(orig / float(low))
    high_wl = f32(orig / float(high))
    two_pi = f32(2.0 * math.pi)
    out = np.empty_like(inv)
    for i, f in enumerate(inv):
        wl = two_pi / f
        llama = f / factor if wl > low_wl else f
        smooth = (old_len / wl - low) / (high - low)
        smoothed = (f32(1.0) - smooth) * llama / factor + smooth * llama
        medium = not (wl < high_wl) and not (wl > low_wl)
        out[i] = smoothed if medium else llama
    return out


def rope_tables(spec: DecoderSpec, positions: int):
    """cosine, sine float32 [positions, head_dim] (root.zig:328-348), system
    cosf / sinf of the f32 angle position * inverse frequency."""
    m = _math_lib()
    inv = rope_inverse_frequencies(spec)
    half = inv.size
    ang = np.arange(positions, dtype=np.float32)[:, None] * inv[None, :]
    flat = ang.ravel()
    c = np.fromiter((m.cosf(a) for a in flat.tolist()), np.float32, flat.size).reshape(ang.shape)
    s = np.fromiter((m.sinf(a) for a in flat.tolist()), np.float32, flat.size).reshape(ang.shape)
    return np.concatenate([c, c], axis=1), np.concatenate([s, s], axis=1)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def forward(spec: DecoderSpec, weights: DecoderWeights, token_ids, cosine, sine, logits=None,
            ctx=None, trace: bool = False):
    """Logits [batch * seq, vocab] (float32 holding bf16 values) of the bf16
    prefill forward of every row of token_ids (int [batch, seq]); cosine and
    sine: float32 device tensors [seq, head_dim]. Runs on torch's current
    stream. trace=True also returns the stages of decoder_trace_t
    (decoder.zig:30-47) as a dict of float32 tensors [layers, batch * seq,
    width] (block_input [batch * seq, hidden]) holding bf16 values:
    (logits, trace)."""
    import torch

    ids = np.ascontiguousarray(token_ids, dtype=np.int64)
    if ids.ndim != 2:
        raise ValueError("token_ids must be [batch, seq]")
    batch, seq = ids.shape
    dev = weights.embed.device
    W = "decoder_forward"
    a = _ck.Args(W)
    a.dev(cosine, "cosine", _ck.F32, (seq, spec.head_dim))
    a.dev(sine, "sine", _ck.F32, (seq, spec.head_dim))
    if logits is None:
        logits = torch.empty((batch * seq, spec.vocab), dtype=torch.float32, device=dev)
    a.dev(logits, "logits", _ck.F32, (batch * seq, spec.vocab))
    a.dev(weights.embed, "embed", _ck.BF16, (spec.vocab, spec.hidden))
    a.dev(weights.lm_head, "lm_head", _ck.BF16, (spec.vocab, spec.hidden), optional=True)
    a.dev(weights.final_norm, "final_norm", _ck.F32, (spec.hidden,))
    if len(weights.layers) != spec.layers:
        raise NcmError(-3, W, "one weight dict per layer")
    for i, layer in enumerate(weights.layers):
        check_layer(a, layer, spec, f"layers[{i}].")
    shape = _Shape(spec.hidden, spec.intermediate, spec.vocab, spec.q_heads, spec.kv_heads,
                   spec.head_dim, spec.layers, spec.window, spec.rms_eps)
    arr = (_Layer * max(1, spec.layers))()
    for i, layer in enumerate(weights.layers):
        arr[i] = _Layer(*[_ptr(layer.get(n)) for n in _LAYER_FIELDS])
    tr = _trace_buffers(torch, spec, batch * seq, dev) if trace else None
    a.done()
    ctx = ctx or default_context(dev.index or 0)
    ctx.bind_stream()
    check(lib().ncm_decoder_forward_dev(ctx.handle, C.byref(shape), arr, _ptr(weights.embed),
                                        _ptr(weights.final_norm), _ptr(weights.lm_head),
                                        _ptr(cosine), _ptr(sine),
                                        ids.ctypes.data_as(C.c_void_p), batch, seq,
                                        _ptr(logits),
                                        C.byref(_Trace(*[_ptr(tr[f]) for f in TRACE_FIELDS]))
                                        if tr else None),
          "decoder_forward")
    return (logits, tr) if trace else logits


def _trace_buffers(torch, spec, T, dev):
    """float32 [layers, T, width] per stage of decoder_trace_t (block_input
    [T, hidden])."""
    widths = {"attention_context": spec.q_heads * spec.head_dim,
              "gate_projection": spec.intermediate, "up_projection": spec.intermediate,
              "gate_up_product": spec.intermediate}
    return {f: torch.empty((T, spec.hidden) if f == "block_input" else
                           (spec.layers, T, widths.get(f, spec.hidden)),
                           dtype=torch.float32, device=dev)
            for f in TRACE_FIELDS}


_LAYER_F32_FIELDS = ("input_norm", "qkv_weight", "qkv_bias", "o_weight", "o_bias",
                     "post_attention_norm", "gate_weight", "gate_bias", "up_weight", "up_bias",
                     "down_weight", "down_bias", "q_norm", "k_norm", "input_norm_bias",
                     "post_attention_norm_bias")
TRACE_FIELDS = ("block_input", "input_norm", "attention_context", "attention_output",
                "attention_residual", "post_attention_norm", "gate_projection",
                "up_projection", "gate_up_product", "mlp_output", "block_output")


class _LayerF32(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in _LAYER_F32_FIELDS]


class _Trace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in TRACE_FIELDS]


def forward_f32(spec: DecoderSpec, weights: DecoderWeights, token_ids, cosine, sine,
                logits=None, trace: bool = False, ctx=None):
    """The f32-mode prefill forward (forward_with_trace with bf16_compute
    false, src/decoder.zig:62-228) of every row of token_ids (int [batch,
    seq]): logits float32 [batch * seq, vocab], and with trace=True also a
    dict of the stages of decoder_trace_t (decoder.zig:30-47), each float32
    [layers, batch * seq, width] (block_input [batch * seq, hidden]).
    weights: float32 device tensors; layers[i] maps the names of
    _LAYER_F32_FIELDS (qkv_weight = q, k and v rows concatenated; gate, up
    and down as stored; biases and q_norm / k_norm may be None)."""
    import torch

    ids = np.ascontiguousarray(token_ids, dtype=np.int64)
    if ids.ndim != 2:
        raise ValueError("token_ids must be [batch, seq]")
    batch, seq = ids.shape
    dev = weights.embed.device
    H, I, hd = spec.hidden, spec.intermediate, spec.head_dim
    qkv, qw = (spec.q_heads + 2 * spec.kv_heads) * hd, spec.q_heads * hd
    W = "decoder_forward_f32"
    a = _ck.Args(W)
    a.dev(cosine, "cosine", _ck.F32, (seq, hd))
    a.dev(sine, "sine", _ck.F32, (seq, hd))
    if logits is None:
        logits = torch.empty((batch * seq, spec.vocab), dtype=torch.float32, device=dev)
    a.dev(logits, "logits", _ck.F32, (batch * seq, spec.vocab))
    a.dev(weights.embed, "embed", _ck.F32, (spec.vocab, H))
    a.dev(weights.lm_head, "lm_head", _ck.F32, (spec.vocab, H), optional=True)
    a.dev(weights.final_norm, "final_norm", _ck.F32, (H,))
    if len(weights.layers) != spec.layers:
        raise NcmError(-3, W, "one weight dict per layer")
    shapes = {"input_norm": (H,), "qkv_weight": (qkv, H), "qkv_bias": (qkv,), "o_weight": (H, qw),
              "o_bias": (H,), "post_attention_norm": (H,), "gate_weight": (I, H),
              "gate_bias": (I,), "up_weight": (I, H), "up_bias": (I,), "down_weight": (H, I),
              "down_bias": (H,), "q_norm": (hd,), "k_norm": (hd,), "input_norm_bias": (H,),
              "post_attention_norm_bias": (H,)}
    optional = {"qkv_bias", "o_bias", "gate_bias", "up_bias", "down_bias", "q_norm", "k_norm",
                "input_norm_bias", "post_attention_norm_bias"}
    for i, layer in enumerate(weights.layers):
        for f in _LAYER_F32_FIELDS:
            a.dev(layer.get(f), f"layers[{i}].{f}", _ck.F32, shapes[f], optional=f in optional)
    tr = _trace_buffers(torch, spec, batch * seq, dev) if trace else None
    a.done()
    shape = _Shape(H, I, spec.vocab, spec.q_heads, spec.kv_heads, hd, spec.layers, spec.window,
                   spec.rms_eps)
    arr = (_LayerF32 * max(1, spec.layers))()
    for i, layer in enumerate(weights.layers):
        arr[i] = _LayerF32(*[_ptr(layer.get(n)) for n in _LAYER_F32_FIELDS])
    ctr = _Trace(*[_ptr(tr[f]) for f in TRACE_FIELDS]) if tr else None
    ctx = ctx or default_context(dev.index or 0)
    ctx.bind_stream()
    check(lib().ncm_decoder_forward_f32_dev(ctx.handle, C.byref(shape), arr, _ptr(weights.embed),
                                            _ptr(weights.final_norm), _ptr(weights.lm_head),
                                            _ptr(cosine), _ptr(sine),
                                            ids.ctypes.data_as(C.c_void_p), batch, seq,
                                            _ptr(logits), C.byref(ctr) if ctr else None), W)
    return (logits, tr) if trace else logits


def _hf_names(i: int) -> dict:
    p = f"model.layers.{i}."
    return {"input_norm": p + "input_layernorm.weight",
            "q": p + "self_attn.q_proj", "k": p + "self_attn.k_proj", "v": p + "self_attn.v_proj",
            "o": p + "self_attn.o_proj", "post_attention_norm": p + "post_attention_layernorm.weight",
            "gate": p + "mlp.gate_proj", "up": p + "mlp.up_proj", "down": p + "mlp.down_proj",
            "q_norm": p + "self_attn.q_norm.weight", "k_norm": p + "self_attn.k_norm.weight"}


class CheckpointError(ValueError):
    """A checkpoint the loader refuses, with the reference's rejection kind
    (src/loader.zig:41-49, 225-276): InvalidConfig, InvalidManifest or
    UnsupportedPickleWeights before any tensor data is read, and
    TiedHeadMismatch (a stored lm_head.weight that differs from tied
    embeddings) after. `problems` holds (feature, message) pairs."""

    def __init__(self, kind: str, problems: list):
        self.kind = kind
        self.problems = problems
        shown = "; ".join(f"{f}: {m}" for f, m in problems[:5])
        more = f" (+{len(problems) - 5} more)" if len(problems) > 5 else ""
        super().__init__(f"{kind}: {shown}{more}")


# Weight files in a pickle format that the loader names instead of reading
# (src/loader.zig:204-223).
_PICKLE_WEIGHTS = ("pytorch_model.bin", "pytorch_model.bin.index.json", "model.bin",
                   "model.bin.index.json", "pytorch_model.pt")


def load_checkpoint(path: str, device, read_count: list | None = None, mode: str = "auto"):
    """(ConfigSpec, DecoderSpec, DecoderWeights) of a Transformers checkpoint
    directory: config.json, then model.safetensors or a sharded
    model.safetensors.index.json (load_checkpoint_report_impl,
    src/loader.zig:95-202). config.json is parsed with the reference's rules
    (hf_config.parse_config) and every shard header is checked against the
    spec's tensor manifest and the index before the first tensor data read;
    any problem raises CheckpointError. mode "auto" picks the reference's
    arithmetic (bf16_compute when every tensor is BF16, src/loader.zig:
    191-199, else the f32 mode); "bf16" or "f32" forces one. read_count: a
    one-element list that counts tensor data reads."""
    import os

    from . import hf_config

    try:
        text = open(os.path.join(path, "config.json"), "rb").read()
        cfg, problems = hf_config.parse_config(text)
    except hf_config.ConfigError:
        raise CheckpointError("InvalidConfig", [(
            "config.json", "invalid JSON; provide a valid supported decoder configuration")])
    if cfg is None:
        raise CheckpointError("InvalidConfig", problems)
    spec = cfg.decoder_spec()
    return cfg, spec, _load(spec, cfg, path, device, read_count, mode)


def _manifest_spec(spec: DecoderSpec, present) -> "hf_config.ConfigSpec":
    """The manifest of a DecoderSpec given without config.json: the optional
    tensors (biases, QK-norm) are those that layer 0 of the checkpoint holds."""
    from . import hf_config

    names = {t.name for t in present}
    has = lambda suffix: f"model.layers.0.{suffix}" in names  # noqa: E731
    return hf_config.ConfigSpec(
        family="", vocab_size=spec.vocab, hidden_size=spec.hidden,
        intermediate_size=spec.intermediate, num_hidden_layers=spec.layers,
        num_attention_heads=spec.q_heads, num_key_value_heads=spec.kv_heads,
        head_dim=spec.head_dim, rms_norm_eps=spec.rms_eps, rope_theta=spec.rope_theta,
        rope_scaling=None, qkv_bias=has("self_attn.q_proj.bias"),
        o_bias=has("self_attn.o_proj.bias"), mlp_bias=has("mlp.gate_proj.bias"),
        qk_norm=has("self_attn.q_norm.weight"), tie_word_embeddings=spec.tie_word_embeddings,
        sliding_window=None)


def load_safetensors(spec: DecoderSpec, path: str, device,
                     read_count: list | None = None, mode: str = "bf16") -> DecoderWeights:
    """Device weights of a Llama-layout checkpoint (Transformers names:
    model.embed_tokens, model.layers.N.{input_layernorm, self_attn.{q,k,v,o}_proj,
    self_attn.{q,k}_norm, post_attention_layernorm, mlp.{gate,up,down}_proj},
    model.norm, lm_head) for a spec given without config.json, from one
    .safetensors file or a directory with model.safetensors or a sharded
    model.safetensors.index.json. The manifest is checked before any data
    read as in load_checkpoint, with the optional tensors that layer 0
    holds; mode as load_checkpoint's (default "bf16")."""
    return _load(spec, None, path, device, read_count, mode)


def run(spec: DecoderSpec, weights: DecoderWeights, token_ids, cosine, sine, logits=None,
        ctx=None):
    """Logits of the forward that matches the weights' mode: forward (bf16)
    or forward_f32."""
    if weights.mode == "f32":
        return forward_f32(spec, weights, token_ids, cosine, sine, logits=logits, ctx=ctx)
    return forward(spec, weights, token_ids, cosine, sine, logits=logits, ctx=ctx)


def _load(spec: DecoderSpec, cfg, path: str, device, read_count, mode="bf16"):
    """Manifest first, then the reads (src/loader.zig:95-202, 225-276).

    Every shard header is parsed, then checked against the manifest of
    `cfg` (hf_config.check) and the index (hf_config.check_index); any
    problem raises CheckpointError("InvalidManifest") before the first
    tensor read. BF16 tensors are copied to HBM as stored (ncm_st_upload);
    F32 and F16 projection weights are widened to f32 on the device and
    rounded to bf16 (RNE, the operand rounding of matmul_bf16); norm scales
    are widened to f32. q|k|v rows are concatenated and gate/up rows
    interleaved in place. Rotary inv_freq buffers are not read. A stored
    lm_head with tied embeddings must decode to the same f32 values
    (TiedHeadMismatch, src/loader.zig:259-267)."""
    import os

    import torch

    from . import hf_config, kernels
    from .safetensors import SafetensorsFile, parse_index

    entries, shard_names, base = None, [], path
    if os.path.isdir(path):
        idx = os.path.join(path, "model.safetensors.index.json")
        if os.path.exists(idx):
            try:
                entries, _ = parse_index(open(idx).read())
            except NcmError as e:
                raise CheckpointError("InvalidManifest", [(
                    "model.safetensors.index.json",
                    f"invalid safetensors index: {e.detail or e}")]) from None
            for _, shard in entries:
                if shard not in shard_names:
                    shard_names.append(shard)
        else:
            shard_names = ["model.safetensors"]
    else:
        base, name = os.path.split(path)
        shard_names = [name]

    files, shards, present, where = {}, {}, [], {}
    try:
        for shard in shard_names:
            p = os.path.join(base, shard)
            if not os.path.exists(p):
                if entries is None:
                    for cand in _PICKLE_WEIGHTS:
                        if os.path.exists(os.path.join(base, cand)):
                            raise CheckpointError("UnsupportedPickleWeights", [(
                                cand, "pickle-based weights are not supported; convert the "
                                "checkpoint to safetensors, then retry")])
                raise FileNotFoundError(p)
            files[shard] = SafetensorsFile(p)
            tensors = files[shard].tensors()
            shards[shard] = [t.name for t in tensors]
            present += tensors
            for t in tensors:
                where.setdefault(t.name, shard)
        mspec = cfg if cfg is not None else _manifest_spec(spec, present)
        problems, _notes = hf_config.check(mspec, present)
        if entries is not None:
            problems += hf_config.check_index(entries, shards)
        if problems:
            raise CheckpointError("InvalidManifest", problems)
        if mode not in ("auto", "bf16", "f32"):
            raise ValueError(f"mode must be auto, bf16 or f32, not {mode!r}")
        if mode == "auto":
            all_bf16 = all(t.dtype == "BF16" for t in present
                           if not t.name.endswith(hf_config.INV_FREQ))
            mode = "bf16" if all_bf16 else "f32"
        weights = _read_weights(spec, mspec, files, where, device, read_count, torch, kernels,
                                mode)
        torch.cuda.current_stream(device).synchronize()
        return weights
    finally:
        for f in files.values():
            f.close()


def _read_weights(spec, mspec, files, where, device, read_count, torch, kernels, mode):
    """The tensor reads of a checkpoint whose manifest passed, into the
    bf16 layout or (mode "f32") float32 tensors decoded as the reference's
    decode_chunk does (src/loader.zig:323-345)."""

    def handle(name):
        f = files[where[name]]
        return f, f.find(name)

    def raw(name, info, f):
        """Tensor `name` as a flat f32 (F32, F16) or bf16 (BF16) device tensor."""
        n = 1
        for d in info.shape:
            n *= d
        if read_count is not None:
            read_count[0] += 1
        if info.dtype == "BF16":
            return f.upload(name, torch.empty(n, dtype=torch.int16, device=device)).view(
                torch.bfloat16)
        if info.dtype == "F16":
            return f.upload(name, torch.empty(n, dtype=torch.float16, device=device)).float()
        return f.upload(name, torch.empty(n, dtype=torch.float32, device=device))

    def load_into(name, out):
        """Tensor `name` into the bf16 device tensor `out` (same element count)."""
        f, info = handle(name)
        n = 1
        for d in info.shape:
            n *= d
        if n != out.numel():
            raise ValueError(f"{name}: {info.shape} does not fit {tuple(out.shape)}")
        if info.dtype == "BF16":
            if read_count is not None:
                read_count[0] += 1
            f.upload(name, out)
        else:
            out.view(-1).copy_(kernels.bf16_from_f32(raw(name, info, f)).view(-1))
        return out

    def as_f32(name):
        f, info = handle(name)
        v = raw(name, info, f)
        return v.float() if v.dtype == torch.bfloat16 else v

    def bf16(*shape):
        return torch.empty(*shape, dtype=torch.bfloat16, device=device)

    def norm(name):
        return as_f32(name)

    def optional_bias(name, out):
        return load_into(name, out) if name in where else None

    qw, kw = spec.q_heads * spec.head_dim, spec.kv_heads * spec.head_dim

    def tied_check():
        # The reference compares the decoded f32 values bit for bit.
        same = torch.equal(as_f32("lm_head.weight").view(torch.int32),
                           as_f32("model.embed_tokens.weight").view(torch.int32))
        if not same:
            raise CheckpointError("TiedHeadMismatch", [(
                "lm_head.weight", "differs from model.embed_tokens.weight although the "
                "embeddings are tied")])

    if mode == "f32":
        def f32(name, *shape):
            return as_f32(name).view(*shape)

        def opt(name, *shape):
            return f32(name, *shape) if name in where else None

        layers = []
        for i in range(spec.layers):
            n = _hf_names(i)
            qkv_b = None
            if n["q"] + ".bias" in where:
                qkv_b = torch.cat([as_f32(n[p] + ".bias") for p in ("q", "k", "v")])
            layers.append({
                "input_norm": norm(n["input_norm"]),
                "qkv_weight": torch.cat([f32(n["q"] + ".weight", qw, spec.hidden),
                                         f32(n["k"] + ".weight", kw, spec.hidden),
                                         f32(n["v"] + ".weight", kw, spec.hidden)]),
                "qkv_bias": qkv_b,
                "o_weight": f32(n["o"] + ".weight", spec.hidden, qw),
                "o_bias": opt(n["o"] + ".bias", spec.hidden),
                "post_attention_norm": norm(n["post_attention_norm"]),
                "gate_weight": f32(n["gate"] + ".weight", spec.intermediate, spec.hidden),
                "gate_bias": opt(n["gate"] + ".bias", spec.intermediate),
                "up_weight": f32(n["up"] + ".weight", spec.intermediate, spec.hidden),
                "up_bias": opt(n["up"] + ".bias", spec.intermediate),
                "down_weight": f32(n["down"] + ".weight", spec.hidden, spec.intermediate),
                "down_bias": opt(n["down"] + ".bias", spec.hidden),
                "q_norm": norm(n["q_norm"]) if mspec.qk_norm else None,
                "k_norm": norm(n["k_norm"]) if mspec.qk_norm else None,
            })
        embed = f32("model.embed_tokens.weight", spec.vocab, spec.hidden)
        lm_head = None
        if not spec.tie_word_embeddings:
            lm_head = f32("lm_head.weight", spec.vocab, spec.hidden)
        elif "lm_head.weight" in where:
            tied_check()
        return DecoderWeights(embed=embed, final_norm=norm("model.norm.weight"), layers=layers,
                              lm_head=lm_head, mode="f32")

    layers = []
    for i in range(spec.layers):
        n = _hf_names(i)
        qkv = bf16(spec.qkv_width, spec.hidden)
        load_into(n["q"] + ".weight", qkv[:qw])
        load_into(n["k"] + ".weight", qkv[qw:qw + kw])
        load_into(n["v"] + ".weight", qkv[qw + kw:])
        qkv_b = None
        if n["q"] + ".bias" in where:
            qkv_b = bf16(spec.qkv_width)
            load_into(n["q"] + ".bias", qkv_b[:qw])
            load_into(n["k"] + ".bias", qkv_b[qw:qw + kw])
            load_into(n["v"] + ".bias", qkv_b[qw + kw:])
        gate = load_into(n["gate"] + ".weight", bf16(spec.intermediate, spec.hidden))
        up = load_into(n["up"] + ".weight", bf16(spec.intermediate, spec.hidden))
        gu_b = None
        if n["gate"] + ".bias" in where:
            gb = load_into(n["gate"] + ".bias", bf16(spec.intermediate))
            ub = load_into(n["up"] + ".bias", bf16(spec.intermediate))
            gu_b = kernels.interleave_gate_up(gb, ub)
        layers.append({
            "input_norm": norm(n["input_norm"]),
            "qkv_weight": qkv, "qkv_bias": qkv_b,
            "o_weight": load_into(n["o"] + ".weight", bf16(spec.hidden, qw)),
            "o_bias": optional_bias(n["o"] + ".bias", bf16(spec.hidden)),
            "post_attention_norm": norm(n["post_attention_norm"]),
            "gate_up_weight": kernels.interleave_gate_up(gate, up), "gate_up_bias": gu_b,
            "down_weight": load_into(n["down"] + ".weight", bf16(spec.hidden, spec.intermediate)),
            "down_bias": optional_bias(n["down"] + ".bias", bf16(spec.hidden)),
            "q_norm": norm(n["q_norm"]) if mspec.qk_norm else None,
            "k_norm": norm(n["k_norm"]) if mspec.qk_norm else None,
        })
        del gate, up
    embed = load_into("model.embed_tokens.weight", bf16(spec.vocab, spec.hidden))
    lm_head = None
    if not spec.tie_word_embeddings:
        lm_head = load_into("lm_head.weight", bf16(spec.vocab, spec.hidden))
    elif "lm_head.weight" in where:
        tied_check()
    return DecoderWeights(embed=embed, final_norm=norm("model.norm.weight"), layers=layers,
                          lm_head=lm_head)
