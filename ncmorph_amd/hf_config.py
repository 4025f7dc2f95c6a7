"""Checkpoint configuration and manifest checks for the decoder families the
loader accepts (Llama, Qwen2, Qwen3, Mistral), restated from
packages/hf_config: parse_config (config.zig:99-216) turns a Transformers
config.json into a spec and a list of named problems; templates and check
(manifest.zig:52-290) compare the tensors of the safetensors headers with the
tensors that spec needs, one problem per feature; check_index
(manifest.zig:300-330) compares a sharded index with the shard headers.
Nothing here reads weight data: the loader runs all of it before the first
tensor read and refuses the checkpoint when any problem is found.

A problem is a (feature, message) pair, as config.problem_t.
"""
from __future__ import annotations

import json
from dataclasses import dataclass

# model_type -> (family, architecture), config.zig:66-71.
FAMILIES = {"llama": ("Llama", "LlamaForCausalLM"), "qwen2": ("Qwen2", "Qwen2ForCausalLM"),
            "qwen3": ("Qwen3", "Qwen3ForCausalLM"), "mistral": ("Mistral", "MistralForCausalLM")}
QWEN3_DEFAULT_HEAD_DIM = 128      # Qwen3Config's default, not hidden / heads (config.zig:74)
DEFAULT_ROPE_THETA = 10000.0      # default_theta of every family here (config.zig:78)
MISTRAL_DEFAULT_WINDOW = 4096     # MistralConfig's sliding_window default (config.zig:519)
INV_FREQ = "self_attn.rotary_emb.inv_freq"   # per-layer buffer older exports stored
SUPPORTED_DTYPES = ("BF16", "F16", "F32")


class ConfigError(ValueError):
    """config.json is not JSON or its root is not an object."""


@dataclass(frozen=True)
class Llama3Scaling:
    factor: float
    low_freq_factor: float
    high_freq_factor: float
    original_max_position_embeddings: int


@dataclass(frozen=True)
class ConfigSpec:
    """config.spec_t (config.zig:31-50)."""

    family: str
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    rope_scaling: Llama3Scaling | None
    qkv_bias: bool
    o_bias: bool
    mlp_bias: bool
    qk_norm: bool
    tie_word_embeddings: bool
    sliding_window: int | None

    def decoder_spec(self):
        """The DecoderSpec the device forward takes."""
        from .decoder import DecoderSpec

        s = self.rope_scaling
        return DecoderSpec(hidden=self.hidden_size, intermediate=self.intermediate_size,
                           vocab=self.vocab_size, q_heads=self.num_attention_heads,
                           kv_heads=self.num_key_value_heads, head_dim=self.head_dim,
                           layers=self.num_hidden_layers, rms_eps=self.rms_norm_eps,
                           window=int(self.sliding_window or 0), rope_theta=self.rope_theta,
                           rope_llama3=None if s is None else (
                               s.factor, s.low_freq_factor, s.high_freq_factor,
                               s.original_max_position_embeddings),
                           tie_word_embeddings=self.tie_word_embeddings)


class _Problems(list):
    def add(self, feature: str, message: str):
        self.append((feature, message))


def _is_int(v):
    return isinstance(v, int) and not isinstance(v, bool)


def _uint(p, fields, key):
    """Absent -> None; present and not a non-negative integer -> problem."""
    if key not in fields:
        return None
    v = fields[key]
    if _is_int(v) and v <= 2**63 - 1:
        if v >= 0:
            return v
        p.add(key, "must not be negative")
    else:
        p.add(key, "must be an integer")
    return None


def _positive(p, fields, key):
    if key not in fields:
        p.add(key, "required key is missing")
        return 0
    v = _uint(p, fields, key)
    if v is None:
        return 0
    if v == 0:
        p.add(key, "must be positive")
    return v


def _float(p, fields, key, feature=None):
    feature = feature or key
    if key not in fields:
        p.add(feature, "required key is missing")
        return None
    v = fields[key]
    if isinstance(v, float) or _is_int(v):
        return float(v)
    p.add(feature, "must be a number")
    return None


def _bool(p, fields, key, default=False):
    if key not in fields:
        return default
    v = fields[key]
    if isinstance(v, bool):
        return v
    p.add(key, "must be true or false")
    return default


def _string(p, fields, key, required):
    if key not in fields:
        if required:
            p.add(key, "required key is missing")
        return None
    v = fields[key]
    if isinstance(v, str):
        return v
    p.add(key, "must be a string")
    return None


def _partial_rotary(p, fields, key, feature):
    if key not in fields:
        return
    v = fields[key]
    if isinstance(v, float) or _is_int(v):
        if v != 1:
            p.add(feature, "only full rotary embeddings are supported")
    else:
        p.add(feature, "must be a number")


def _scaling(p, scaling, feature):
    """parse_scaling_map (config.zig:385-405): default or llama3."""
    key = "rope_type" if "rope_type" in scaling else "type"
    if key not in scaling:
        return None
    rt = scaling[key]
    if not isinstance(rt, str):
        p.add(feature, "rope type must be a string")
        return None
    if rt == "default":
        return None
    if rt != "llama3":
        p.add(feature, f"rope type '{rt}' is not supported in this version")
        return None

    def num(key):
        v = _float(p, scaling, key, f"{feature}.{key}")
        return 0.0 if v is None else v

    path = f"{feature}.original_max_position_embeddings"
    ome = scaling.get("original_max_position_embeddings")
    if ome is None and "original_max_position_embeddings" not in scaling:
        p.add(path, "required key is missing")
        ome = 0
    elif not _is_int(ome):
        p.add(path, "must be a non-negative integer")
        ome = 0
    elif ome < 0:
        ome = 0
    return Llama3Scaling(num("factor"), num("low_freq_factor"), num("high_freq_factor"), ome)


def _rope_parameters(p, fields):
    """(rope_theta or None, scaling) of the rope_parameters object, or None
    when absent (config.zig:326-350)."""
    if "rope_parameters" not in fields:
        return None
    params = fields["rope_parameters"]
    if not isinstance(params, dict):
        p.add("rope_parameters", "must be an object")
        return None
    if any(isinstance(v, dict) for v in params.values()):
        p.add("rope_parameters", "nested per-layer RoPE parameters are not supported")
    _partial_rotary(p, params, "partial_rotary_factor", "rope_parameters.partial_rotary_factor")
    theta = _float(p, params, "rope_theta", "rope_parameters.rope_theta") \
        if "rope_theta" in params else None
    return theta, _scaling(p, params, "rope_parameters")


def _sliding_window(p, fields, family):
    """config.zig:502-523."""
    if family in ("Qwen2", "Qwen3"):
        if _bool(p, fields, "use_sliding_window", False):
            p.add("use_sliding_window", "sliding-window attention is not supported in this version")
        return None
    if family == "Llama":
        if fields.get("sliding_window", None) is not None:
            p.add("sliding_window", "sliding-window attention is not supported for llama")
        return None
    if "sliding_window" not in fields:
        return MISTRAL_DEFAULT_WINDOW
    if fields["sliding_window"] is None:
        return None
    return _uint(p, fields, "sliding_window")


def parse_config(text) -> tuple:
    """(ConfigSpec or None, [problems]) of a config.json document (str or
    bytes); the spec is None whenever a problem was found. Invalid JSON or a
    non-object root raises ConfigError."""
    try:
        fields = json.loads(text)
    except (ValueError, UnicodeDecodeError) as e:
        raise ConfigError(f"config.json is not valid JSON: {e}") from None
    if not isinstance(fields, dict):
        raise ConfigError("config.json root is not an object")
    p = _Problems()
    mt = _string(p, fields, "model_type", True)
    if mt is None:
        return None, list(p)
    if mt not in FAMILIES:
        p.add("model_type", f"unsupported model_type '{mt}'")
        return None, list(p)
    family, arch = FAMILIES[mt]
    archs = fields.get("architectures")
    if "architectures" not in fields:
        p.add("architectures", "required key is missing")
    elif not isinstance(archs, list):
        p.add("architectures", "must be a list")
    elif len(archs) != 1:
        p.add("architectures", "must list exactly one architecture")
    elif not isinstance(archs[0], str):
        p.add("architectures", "must contain strings")
    elif archs[0] != arch:
        p.add("architectures", f"'{archs[0]}' does not match model_type '{mt}', which expects "
              f"'{arch}'")

    vocab = _positive(p, fields, "vocab_size")
    hidden = _positive(p, fields, "hidden_size")
    inter = _positive(p, fields, "intermediate_size")
    layers = _positive(p, fields, "num_hidden_layers")
    heads = _positive(p, fields, "num_attention_heads")
    kv = _uint(p, fields, "num_key_value_heads")
    kv = heads if kv is None else kv
    if kv == 0 or heads % kv != 0:
        p.add("num_key_value_heads", "must divide num_attention_heads")
    head_dim = _uint(p, fields, "head_dim")
    if head_dim is None:
        if family == "Qwen3":
            head_dim = QWEN3_DEFAULT_HEAD_DIM
        elif heads > 0 and hidden % heads == 0:
            head_dim = hidden // heads
        else:
            p.add("head_dim", "hidden_size must divide by num_attention_heads when head_dim is "
                  "absent")
            head_dim = 0

    eps = _float(p, fields, "rms_norm_eps") or 0.0
    params = _rope_parameters(p, fields)
    top_theta = _float(p, fields, "rope_theta") if "rope_theta" in fields else None
    if top_theta is not None:
        theta = top_theta
    elif params is not None and params[0] is not None:
        theta = params[0]
    else:
        theta = DEFAULT_ROPE_THETA
    if params is not None and params[0] is not None:
        legacy = DEFAULT_ROPE_THETA if top_theta is None else top_theta
        if (top_theta is not None or "rope_scaling" in fields) and legacy != params[0]:
            p.add("rope_parameters", "rope_theta disagrees with legacy RoPE settings")
    if "rope_scaling" in fields:
        v = fields["rope_scaling"]
        if v is None:
            scaling = None
        elif isinstance(v, dict):
            scaling = _scaling(p, v, "rope_scaling")
        else:
            p.add("rope_scaling", "must be an object or null")
            scaling = None
        if params is not None and scaling != params[1]:
            p.add("rope_parameters", "RoPE settings disagree with rope_scaling")
    else:
        scaling = params[1] if params is not None else None

    act = _string(p, fields, "hidden_act", False) or "silu"
    if act != "silu":
        p.add("hidden_act", f"only silu is supported, not '{act}'")
    if _bool(p, fields, "use_mrope"):
        p.add("use_mrope", "multimodal rotary embeddings are not supported")
    if _bool(p, fields, "rope_interleaved"):
        p.add("rope_interleaved", "only the rotate-half RoPE layout is supported")
    _partial_rotary(p, fields, "partial_rotary_factor", "partial_rotary_factor")
    for key in ("num_local_experts", "num_experts", "num_experts_per_tok"):
        if key in fields and fields[key] is not None and not (_is_int(fields[key])
                                                               and fields[key] == 0):
            p.add(key, "mixture-of-experts models are not supported")
    lt = fields.get("layer_types")
    if lt is not None:
        if not isinstance(lt, list):
            p.add("layer_types", "must be a list")
        elif any(x != "full_attention" for x in lt):
            p.add("layer_types", "only full attention is supported in this version")

    tie = _bool(p, fields, "tie_word_embeddings", False)
    attention_bias = _bool(p, fields, "attention_bias", False) if family in ("Llama", "Qwen3") \
        else False
    mlp_bias = _bool(p, fields, "mlp_bias", False) if family == "Llama" else False
    window = _sliding_window(p, fields, family)
    spec = ConfigSpec(family=family, vocab_size=vocab, hidden_size=hidden,
                      intermediate_size=inter, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv, head_dim=head_dim,
                      rms_norm_eps=eps, rope_theta=theta, rope_scaling=scaling,
                      qkv_bias=attention_bias if family in ("Llama", "Qwen3") else
                      family == "Qwen2",
                      o_bias=attention_bias if family in ("Llama", "Qwen3") else False,
                      mlp_bias=mlp_bias, qk_norm=family == "Qwen3", tie_word_embeddings=tie,
                      sliding_window=window)
    return (spec if not p else None), list(p)


@dataclass(frozen=True)
class Template:
    """One kind of tensor (manifest.template_t): per-layer patterns are the
    suffix after "model.layers.{i}."."""

    pattern: str
    feature: str
    per_layer: bool
    shape: tuple
    optional: bool


def templates(spec: ConfigSpec) -> list:
    """Every tensor kind `spec` needs, optional ones marked (manifest.zig:52-91)."""
    H, I, hd = spec.hidden_size, spec.intermediate_size, spec.head_dim
    qw, kw = spec.num_attention_heads * hd, spec.num_key_value_heads * hd
    rows = [("model.embed_tokens.weight", False, (spec.vocab_size, H), False),
            ("model.norm.weight", False, (H,), False),
            ("lm_head.weight", False, (spec.vocab_size, H), spec.tie_word_embeddings),
            ("input_layernorm.weight", True, (H,), False),
            ("self_attn.q_proj.weight", True, (qw, H), False),
            ("self_attn.k_proj.weight", True, (kw, H), False),
            ("self_attn.v_proj.weight", True, (kw, H), False),
            ("self_attn.o_proj.weight", True, (H, qw), False)]
    if spec.qkv_bias:
        rows += [("self_attn.q_proj.bias", True, (qw,), False),
                 ("self_attn.k_proj.bias", True, (kw,), False),
                 ("self_attn.v_proj.bias", True, (kw,), False)]
    if spec.o_bias:
        rows.append(("self_attn.o_proj.bias", True, (H,), False))
    if spec.qk_norm:
        rows += [("self_attn.q_norm.weight", True, (hd,), False),
                 ("self_attn.k_norm.weight", True, (hd,), False)]
    rows += [("post_attention_layernorm.weight", True, (H,), False),
             ("mlp.gate_proj.weight", True, (I, H), False),
             ("mlp.up_proj.weight", True, (I, H), False),
             ("mlp.down_proj.weight", True, (H, I), False)]
    if spec.mlp_bias:
        rows += [("mlp.gate_proj.bias", True, (I,), False),
                 ("mlp.up_proj.bias", True, (I,), False),
                 ("mlp.down_proj.bias", True, (H,), False)]
    rows.append((INV_FREQ, True, (hd // 2,), True))
    return [Template(pat, f"model.layers.{{i}}.{pat}" if per else pat, per, shape, opt)
            for pat, per, shape, opt in rows]


def _split_layer(name):
    """(layer, layer text, suffix) of "model.layers.<n>.<suffix>", else None."""
    pre = "model.layers."
    if not name.startswith(pre):
        return None
    rest = name[len(pre):]
    dot = rest.find(".")
    if dot < 0:
        return None
    text = rest[:dot]
    # Decimal as std.fmt.parseInt reads it: an optional "+", digits with
    # single "_" separators between them, below 2^64.
    digits = text[1:] if text.startswith("+") else text
    parts = digits.split("_")
    if not all(part and all("0" <= c <= "9" for c in part) for part in parts):
        return None
    n = int("".join(parts))
    if n >= 2**64:
        return None
    return n, text, rest[dot + 1:]


def _shape_text(shape):
    return "[" + ", ".join(str(d) for d in shape) + "]"


def check(spec: ConfigSpec, present) -> tuple:
    """(problems, notes) of the tensors `present` (objects with name, dtype,
    shape, as the headers list them) against `spec` (manifest.zig:178-290).
    Problems are grouped per feature and kind, in order of first occurrence:
    Noncanonical layer index, Unexpected, Duplicate, Shape, Dtype, then
    Missing. Notes: a stored lm_head with tied embeddings, and stored
    rotary inv_freq buffers, which the loader skips."""
    tl = templates(spec)
    seen = [[0] * (spec.num_hidden_layers if t.per_layer else 1) for t in tl]
    groups, notes = {}, []

    def group(kind, feature, sample, detail=""):
        g = groups.get((kind, feature))
        if g is None:
            groups[(kind, feature)] = [1, sample, detail]
        else:
            g[0] += 1

    def find(pattern, per_layer):
        for k, t in enumerate(tl):
            if t.per_layer == per_layer and t.pattern == pattern:
                return k
        return None

    for tensor in present:
        layer = 0
        parsed = _split_layer(tensor.name)
        if parsed is not None:
            n, text, suffix = parsed
            feature = f"model.layers.{{i}}.{suffix}"
            if text != str(n):
                group("Noncanonical", feature, tensor.name)
                continue
            k = find(suffix, True)
            if k is None or n >= spec.num_hidden_layers:
                group("Unexpected", feature, tensor.name)
                continue
            layer = n
        else:
            k = find(tensor.name, False)
            if k is None:
                group("Unexpected", tensor.name, tensor.name)
                continue
            if tensor.name == "lm_head.weight" and spec.tie_word_embeddings:
                notes.append(("lm_head.weight", "present although the embeddings are tied; "
                              "the loader checks that the two are equal"))
        t = tl[k]
        seen[k][layer] += 1
        if seen[k][layer] == 2:
            group("Duplicate", t.feature, tensor.name)
        if tuple(tensor.shape) != t.shape:
            group("Shape", t.feature, tensor.name,
                  f"actual {_shape_text(tensor.shape)}, expected {_shape_text(t.shape)}")
        if tensor.dtype not in SUPPORTED_DTYPES:
            group("Dtype", t.feature, tensor.name, tensor.dtype)

    for t, counts in zip(tl, seen):
        if t.optional:
            continue
        if t.per_layer:
            for layer, c in enumerate(counts):
                if c == 0:
                    group("Missing", t.feature, f"model.layers.{layer}.{t.pattern}")
        elif counts[0] == 0:
            group("Missing", t.feature, t.pattern)
    for t, counts in zip(tl, seen):
        if t.pattern == INV_FREQ and sum(counts):
            notes.append((t.feature, f"{sum(counts)} tensor(s) present but not loaded: the "
                          "frequencies are computed from rope_theta"))

    text = {
        "Missing": "missing from the checkpoint: {n} tensor(s), first {s}",
        "Shape": "shape mismatch ({d}): {n} tensor(s), first {s}",
        "Dtype": "dtype {d} is not supported (expected BF16, F16 or F32): {n} tensor(s), first {s}",
        "Unexpected": "not expected for this configuration: {n} tensor(s), first {s}",
        "Noncanonical": "noncanonical layer index; use the decimal layer number without "
                        "leading zeroes: {s}",
        "Duplicate": "appears more than once, first {s}",
    }
    problems = [(feature, text[kind].format(n=g[0], s=g[1], d=g[2]))
                for (kind, feature), g in groups.items()]
    return problems, notes


def check_index(entries, shards: dict) -> list:
    """Problems between a sharded index and the shard headers
    (manifest.zig:300-330): an indexed shard that is absent (ShardMissing),
    an indexed tensor not in its shard (NotInShard), a shard's tensor not
    indexed under that shard (NotIndexed); one problem per kind and shard,
    with its count and first tensor. entries: [(tensor, shard file)];
    shards: {shard file: tensor names in header order}."""
    groups = {}

    def add(kind, shard, tensor):
        g = groups.setdefault((kind, shard), [0, tensor])
        g[0] += 1

    indexed = set(entries)
    names = {s: set(v) for s, v in shards.items()}
    for tensor, shard in entries:
        if shard not in names:
            add("ShardMissing", shard, tensor)
        elif tensor not in names[shard]:
            add("NotInShard", shard, tensor)
    for shard, tensors in shards.items():
        for tensor in tensors:
            if (tensor, shard) not in indexed:
                add("NotIndexed", shard, tensor)
    text = {"ShardMissing": "shard '{s}' is listed for {n} tensor(s) but was not found, first '{t}'",
            "NotInShard": "{n} tensor(s) are listed under shard '{s}' but are not in it, first '{t}'",
            "NotIndexed": "{n} tensor(s) in shard '{s}' are missing from the index, first '{t}'"}
    return [("model.safetensors.index.json", text[kind].format(s=shard, n=g[0], t=g[1]))
            for (kind, shard), g in groups.items()]
