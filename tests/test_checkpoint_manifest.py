"""Checkpoint configuration and manifest checks (ncmorph_amd.hf_config) and
the loader's manifest-first order, on the CPU.

The 13 real-checkpoint fixtures under tests/golden/checkpoints/ are the
reference's own (packages/hf_config/testdata, copied unchanged by
tests/golden/copy_checkpoint_headers.py): config.json, the exact header bytes
of every shard, the index and the shard sizes of published checkpoints, no
weight data. As packages/hf_config/fixtures_test.zig:233-286 does, every
config parses without a problem into the expected family, every header
parses (the C reader and the oracle's parser agree on every tensor), the
tensors match the manifest with the expected number of notes, and the index
agrees with the headers. The config and manifest cases restate
config.zig:538-727 and manifest_test.zig; the loader cases restate
src/loader.zig:462-489 (a manifest failure is raised before any tensor
data read)."""
import json
import os

import pytest

from ncmorph_amd import hf_config as hc
from ncmorph_amd import safetensors as st

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = os.path.join(HERE, "golden", "checkpoints")

# name -> (family, expected notes), packages/hf_config/fixtures_test.zig:30-211.
EXPECTED = {
    "smollm2-135m": ("Llama", 0), "qwen2.5-0.5b": ("Qwen2", 0), "qwen3-0.6b": ("Qwen3", 1),
    "llama-3.2-1b": ("Llama", 0), "mistral-7b-v0.3": ("Mistral", 0),
    "mistral-7b-v0.1": ("Mistral", 0), "llama-2-7b": ("Llama", 1), "llama-3.0-8b": ("Llama", 0),
    "qwen3-1.7b": ("Qwen3", 1), "qwen3-4b": ("Qwen3", 0), "qwen3-8b": ("Qwen3", 0),
    "qwen3-14b": ("Qwen3", 0), "qwen3-32b": ("Qwen3", 0),
}


def _fixture(name):
    """(config text, index text or None, {shard file: header bytes}, sizes)."""
    d = os.path.join(FIXTURES, name)
    idx = os.path.join(d, "model.safetensors.index.json")
    headers = {f[:-len(".header")]: open(os.path.join(d, f), "rb").read()
               for f in sorted(os.listdir(d)) if f.endswith(".safetensors.header")}
    return (open(os.path.join(d, "config.json")).read(),
            open(idx).read() if os.path.exists(idx) else None, headers,
            json.load(open(os.path.join(d, "sizes.json"))))


def _headers(name, oracle=None):
    """(present tensors in shard order, {shard: tensor names}) of a fixture,
    each header parsed by the C reader (and by the oracle when given)."""
    _, _, headers, sizes = _fixture(name)
    present, shards = [], {}
    for shard, raw in headers.items():
        with st.SafetensorsFile(data=raw, file_size=sizes[shard]) as f:
            tensors = f.tensors()
        if oracle is not None:
            hl, dl, ts = oracle.st_parse_header(raw, sizes[shard])
            names = [n for n, _ in oracle.ST_DTYPES]
            assert [(t.name, t.dtype, t.shape, t.data_begin, t.data_end) for t in tensors] == \
                [(n, names[d], tuple(s), b, e) for n, d, s, b, e in ts]
            assert 8 + hl + dl == sizes[shard]
        present += tensors
        shards[shard] = [t.name for t in tensors]
    return present, shards


def test_all_reference_fixtures_present():
    assert sorted(os.listdir(FIXTURES)) == sorted(EXPECTED)


@pytest.mark.parametrize("name", sorted(EXPECTED))
def test_real_checkpoint_matches_its_manifest(ncm, oracle, name):
    family, n_notes = EXPECTED[name]
    cfg_text, index_text, _, _ = _fixture(name)
    spec, problems = hc.parse_config(cfg_text)
    assert problems == []
    assert spec.family == family
    present, shards = _headers(name, oracle)
    problems, notes = hc.check(spec, present)
    assert problems == [], problems
    assert len(notes) == n_notes, notes
    if index_text is not None:
        entries, total = st.parse_index(index_text)
        assert (entries, total) == oracle.st_parse_index(index_text)
        assert hc.check_index(entries, shards) == []
        assert len(entries) == len(present)
    ds = spec.decoder_spec()
    assert ds.qkv_width == (spec.num_attention_heads + 2 * spec.num_key_value_heads) \
        * spec.head_dim


def test_fixture_tensor_counts(ncm):
    """fixtures_test.zig:273-286, and the tensors the stored headers hold."""
    qwen2, _ = hc.parse_config(_fixture("qwen2.5-0.5b")[0])
    assert sum(1 for t in hc.templates(qwen2) if not t.optional and not t.per_layer) == 2
    present, _ = _headers("qwen2.5-0.5b")
    assert len(present) == 24 * 12 + 2
    smol, _ = hc.parse_config(_fixture("smollm2-135m")[0])
    assert sum(1 for t in hc.templates(smol) if t.per_layer and not t.optional) == 9
    present, _ = _headers("smollm2-135m")
    assert len(present) == 30 * 9 + 2
    present, _ = _headers("llama-3.2-1b")
    embed = next(t for t in present if t.name == "model.embed_tokens.weight")
    assert embed.dtype == "BF16" and embed.shape == (128256, 2048)
    spec, _ = hc.parse_config(_fixture("llama-3.2-1b")[0])
    assert spec.rope_scaling == hc.Llama3Scaling(32.0, 1.0, 4.0, 8192)
    assert spec.tie_word_embeddings and spec.head_dim == 64
    q8, _ = hc.parse_config(_fixture("qwen3-8b")[0])
    assert (q8.hidden_size, q8.num_attention_heads, q8.num_key_value_heads, q8.head_dim,
            q8.qk_norm, q8.qkv_bias) == (4096, 32, 8, 128, True, False)


def test_fixture_mutations_are_one_problem_each(ncm):
    """A real header list with one feature removed from every layer, one
    layer's shape changed, an unsupported dtype, a duplicate, a
    noncanonical layer index and an extra tensor: each is one problem, with
    the feature the reference names."""
    spec, _ = hc.parse_config(_fixture("qwen3-8b")[0])
    present, _ = _headers("qwen3-8b")

    def run(tensors):
        problems, _ = hc.check(spec, tensors)
        return [f for f, _ in problems], [m for _, m in problems]

    feats, msgs = run([t for t in present if not t.name.endswith("self_attn.k_norm.weight")])
    assert feats == ["model.layers.{i}.self_attn.k_norm.weight"]
    assert "36 tensor(s)" in msgs[0]
    bent = [st.TensorInfo(t.name, t.dtype, (1, 1) if t.name ==
                          "model.layers.3.mlp.up_proj.weight" else t.shape, 0, 0) for t in present]
    feats, msgs = run(bent)
    assert feats == ["model.layers.{i}.mlp.up_proj.weight"]
    assert "actual [1, 1], expected [12288, 4096]" in msgs[0]
    feats, msgs = run([st.TensorInfo(t.name, "U8" if t.name.endswith("input_layernorm.weight")
                                     else t.dtype, t.shape, 0, 0) for t in present])
    assert feats == ["model.layers.{i}.input_layernorm.weight"] and "36 tensor(s)" in msgs[0]
    feats, msgs = run(present + [present[5]])
    assert feats == [_feature(present[5].name)] and msgs[0].startswith("appears more")
    odd = [st.TensorInfo("model.layers.07." + present[5].name.split(".", 3)[3],
                         present[5].dtype, present[5].shape, 0, 0)]
    feats, msgs = run(present + odd)
    assert len(feats) == 1 and msgs[0].startswith("noncanonical")
    feats, _ = run(present + [st.TensorInfo("model.layers.36.mlp.up_proj.weight", "BF16",
                                            (12288, 4096), 0, 0)])
    assert feats == ["model.layers.{i}.mlp.up_proj.weight"]


def _feature(name):
    parts = name.split(".", 3)
    if name.startswith("model.layers."):
        return "model.layers.{i}." + parts[3]
    return name


def test_index_disagreements():
    """manifest_test.zig:122-146, and each kind of index problem."""
    entries = [("a", "s1"), ("b", "s2")]
    assert len(hc.check_index(entries, {"s1": ["a"], "s2": ["b", "c"]})) == 1
    probs = hc.check_index([("a", "s1"), ("b", "s3"), ("d", "s3"), ("x", "s2")],
                           {"s1": ["a", "y"], "s2": ["b"]})
    msgs = [m for _, m in probs]
    assert msgs == ["shard 's3' is listed for 2 tensor(s) but was not found, first 'b'",
                    "1 tensor(s) are listed under shard 's2' but are not in it, first 'x'",
                    "1 tensor(s) in shard 's1' are missing from the index, first 'y'",
                    "1 tensor(s) in shard 's2' are missing from the index, first 'b'"]


LLAMA_TINY = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "vocab_size": 8,
              "hidden_size": 4, "intermediate_size": 8, "num_hidden_layers": 1,
              "num_attention_heads": 2, "num_key_value_heads": 1, "rms_norm_eps": 1e-05,
              "rope_theta": 10000.0}


def _cfg(**kw):
    c = dict(LLAMA_TINY)
    for k, v in kw.items():
        if v is None and k.startswith("drop_"):
            c.pop(k[5:], None)
        else:
            c[k] = v
    return json.dumps(c)


def test_config_rules():
    """The cases of config.zig:538-727, with configurations of our own."""
    q25 = json.dumps({"architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2",
                      "vocab_size": 151936, "hidden_size": 896, "intermediate_size": 4864,
                      "num_hidden_layers": 24, "num_attention_heads": 14,
                      "num_key_value_heads": 2, "rms_norm_eps": 1e-06, "rope_theta": 1e6,
                      "hidden_act": "silu", "tie_word_embeddings": True,
                      "use_sliding_window": False, "sliding_window": 32768})
    s, p = hc.parse_config(q25)
    assert p == [] and s.family == "Qwen2" and s.head_dim == 64
    assert s.qkv_bias and not s.o_bias and s.sliding_window is None
    s, p = hc.parse_config(json.dumps(dict(
        LLAMA_TINY, architectures=["Qwen3ForCausalLM"], model_type="qwen3")))
    assert p == [] and s.head_dim == hc.QWEN3_DEFAULT_HEAD_DIM and s.qk_norm
    s, p = hc.parse_config(_cfg(drop_rope_theta=None))
    assert p == [] and s.rope_theta == 10000.0
    mistral = dict(LLAMA_TINY, architectures=["MistralForCausalLM"], model_type="mistral")
    s, _ = hc.parse_config(json.dumps(mistral))
    assert s.sliding_window == 4096
    s, _ = hc.parse_config(json.dumps(dict(mistral, sliding_window=None)))
    assert s.sliding_window is None
    s, _ = hc.parse_config(json.dumps(dict(mistral, sliding_window=1024)))
    assert s.sliding_window == 1024

    def one(text, feature):
        spec, problems = hc.parse_config(text)
        assert spec is None and [f for f, _ in problems] == [feature], problems

    one(_cfg(hidden_act="gelu"), "hidden_act")
    one(_cfg(model_type="qwen2"), "architectures")
    one(_cfg(rope_scaling={"rope_type": "linear", "factor": 2.0}), "rope_scaling")
    one(_cfg(sliding_window=4096), "sliding_window")
    one(_cfg(num_key_value_heads=3), "num_key_value_heads")
    one(_cfg(drop_rms_norm_eps=None), "rms_norm_eps")
    one(_cfg(hidden_size=5, num_attention_heads=2, num_key_value_heads=1), "head_dim")
    one(_cfg(layer_types=["full_attention", "sliding_attention"]), "layer_types")
    one(_cfg(drop_rope_theta=None, rope_parameters={
        "rope_theta": 1e4, "rope_type": "default", "partial_rotary_factor": 0.5}),
        "rope_parameters.partial_rotary_factor")
    one(_cfg(drop_rope_theta=None, rope_parameters={"full_attention": {"rope_theta": 5e5}}),
        "rope_parameters")
    l3 = {"factor": 32.0, "high_freq_factor": 4.0, "low_freq_factor": 1.0,
          "original_max_position_embeddings": 8192, "rope_type": "llama3"}
    legacy, p1 = hc.parse_config(_cfg(rope_theta=5e5, rope_scaling=l3))
    params, p2 = hc.parse_config(_cfg(drop_rope_theta=None,
                                      rope_parameters=dict(l3, rope_theta=5e5)))
    assert p1 == [] and p2 == [] and legacy == params
    assert legacy.rope_scaling == hc.Llama3Scaling(32.0, 1.0, 4.0, 8192)
    one(_cfg(rope_theta=5e5, rope_scaling=l3, rope_parameters=dict(l3, rope_theta=5e5,
                                                                    factor=64.0)),
        "rope_parameters")
    one(_cfg(rope_theta=5e5, rope_parameters={"rope_theta": 1e4}), "rope_parameters")
    s, p = hc.parse_config(json.dumps(dict(
        LLAMA_TINY, architectures=["Qwen2ForCausalLM"], model_type="qwen2", use_mrope=True,
        rope_interleaved=True, num_experts=4)))
    assert s is None and len(p) == 3
    s, p = hc.parse_config(_cfg(model_type="gpt2"))
    assert s is None and p == [("model_type", "unsupported model_type 'gpt2'")]
    s, p = hc.parse_config(_cfg(attention_bias=True, mlp_bias=True, tie_word_embeddings=True))
    assert p == [] and s.qkv_bias and s.o_bias and s.mlp_bias and s.tie_word_embeddings
    with pytest.raises(hc.ConfigError):
        hc.parse_config("[1, 2]")
    with pytest.raises(hc.ConfigError):
        hc.parse_config("{")


def _tiny_spec(family, qk_norm, qkv_bias, tie):
    return hc.ConfigSpec(family=family, vocab_size=16, hidden_size=8, intermediate_size=12,
                         num_hidden_layers=2, num_attention_heads=2, num_key_value_heads=1,
                         head_dim=4, rms_norm_eps=1e-6, rope_theta=1e6, rope_scaling=None,
                         qkv_bias=qkv_bias, o_bias=False, mlp_bias=False, qk_norm=qk_norm,
                         tie_word_embeddings=tie, sliding_window=None)


def _complete(spec, skip=None):
    out = []
    for t in hc.templates(spec):
        if t.optional or t.pattern == skip:
            continue
        names = [f"model.layers.{i}.{t.pattern}" for i in range(spec.num_hidden_layers)] \
            if t.per_layer else [t.pattern]
        out += [st.TensorInfo(n, "BF16", t.shape, 0, 0) for n in names]
    return out


def test_manifest_cases():
    """manifest_test.zig:56-120."""
    spec = _tiny_spec("Qwen2", False, True, True)
    assert hc.check(spec, _complete(spec)) == ([], [])
    spec = _tiny_spec("Qwen3", True, False, True)
    probs, _ = hc.check(spec, _complete(spec, "self_attn.q_norm.weight"))
    assert [f for f, _ in probs] == ["model.layers.{i}.self_attn.q_norm.weight"]
    spec = _tiny_spec("Llama", False, False, True)
    present = _complete(spec)
    present[0] = st.TensorInfo(present[0].name, "BF16", (1, 1), 0, 0)
    probs, _ = hc.check(spec, present)
    assert [f for f, _ in probs] == ["model.embed_tokens.weight"]
    probs, _ = hc.check(spec, _complete(spec) + [
        st.TensorInfo("model.layers.0.mlp.extra.weight", "F32", (1,), 0, 0)])
    assert len(probs) == 1
    spec = _tiny_spec("Qwen3", True, False, True)
    probs, notes = hc.check(spec, _complete(spec) + [
        st.TensorInfo("lm_head.weight", "BF16", (16, 8), 0, 0)])
    assert probs == [] and len(notes) == 1
    spec = _tiny_spec("Llama", False, False, True)
    present = _complete(spec)
    present[0] = st.TensorInfo(present[0].name, "U8", present[0].shape, 0, 0)
    probs, _ = hc.check(spec, present)
    assert len(probs) == 1 and "dtype U8" in probs[0][1]
    spec = _tiny_spec("Llama", False, False, False)
    probs, _ = hc.check(spec, [t for t in _complete(spec) if t.name != "lm_head.weight"])
    assert probs == [("lm_head.weight", "missing from the checkpoint: 1 tensor(s), first "
                      "lm_head.weight")]


def _write_st(path, tensors):
    st.write_file(path, {n: (dt, shape, bytes(raw)) for n, (dt, shape, raw) in tensors.items()})


def _tiny_checkpoint(d, config=LLAMA_TINY, extra=None, drop=()):
    """A complete checkpoint of `config` with zero weights, all BF16."""
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(config, f)
    spec, _ = hc.parse_config(json.dumps(config))
    tensors = {}
    for t in _complete(spec):
        if t.name in drop:
            continue
        n = 1
        for s in t.shape:
            n *= s
        tensors[t.name] = ("BF16", t.shape, bytes(2 * n))
    tensors.update(extra or {})
    _write_st(os.path.join(d, "model.safetensors"), tensors)
    return spec


def test_manifest_failure_before_any_read(ncm, tmp_path):
    """src/loader.zig:462-489: a checkpoint whose only tensor is unexpected is
    refused as InvalidManifest with zero tensor data reads; so is one with
    a missing tensor, an extra one, or an index that disagrees with the
    shards."""
    from ncmorph_amd import decoder

    with open(tmp_path / "config.json", "w") as f:
        json.dump(dict(LLAMA_TINY, vocab_size=4, hidden_size=2, intermediate_size=3,
                       num_attention_heads=1), f)
    _write_st(str(tmp_path / "model.safetensors"), {"unexpected.weight": ("F32", (1,), b"\0" * 4)})
    reads = [0]
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(tmp_path), "cpu", read_count=reads)
    assert e.value.kind == "InvalidManifest" and reads == [0]
    assert ("unexpected.weight", "not expected for this configuration: 1 tensor(s), first "
            "unexpected.weight") in e.value.problems

    for case in ("missing", "extra"):
        d = tmp_path / case
        d.mkdir()
        if case == "missing":
            _tiny_checkpoint(str(d), drop=("model.layers.0.mlp.up_proj.weight",))
        else:
            _tiny_checkpoint(str(d), extra={"model.layers.0.self_attn.q_proj.bias":
                                            ("BF16", (4,), b"\0" * 8)})
        reads = [0]
        with pytest.raises(decoder.CheckpointError) as e:
            decoder.load_checkpoint(str(d), "cpu", read_count=reads)
        assert e.value.kind == "InvalidManifest" and reads == [0] and len(e.value.problems) == 1

    d = tmp_path / "sharded"
    d.mkdir()
    spec = _tiny_checkpoint(str(d))
    os.rename(d / "model.safetensors", d / "model-00001-of-00001.safetensors")
    names = [t.name for t in _complete(spec)]
    wm = {n: "model-00001-of-00001.safetensors" for n in names[1:]}
    with open(d / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)
    reads = [0]
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(d), "cpu", read_count=reads)
    assert e.value.kind == "InvalidManifest" and reads == [0]
    assert e.value.problems == [("model.safetensors.index.json",
                                 f"1 tensor(s) in shard 'model-00001-of-00001.safetensors' are "
                                 f"missing from the index, first '{names[0]}'")]
    with open(d / "model.safetensors.index.json", "w") as f:
        f.write('{"weight_map": {"a": "../x"}}')
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(d), "cpu")
    assert e.value.kind == "InvalidManifest" and "UnsafeShardName" in e.value.problems[0][1]


def test_config_and_pickle_rejections(ncm, tmp_path):
    """src/loader.zig:104-113 and :130-141: an unsupported or unreadable
    config.json is InvalidConfig with its problems; pickle weights without
    safetensors are named as UnsupportedPickleWeights."""
    from ncmorph_amd import decoder

    (tmp_path / "config.json").write_text('{"architectures":["UnsupportedForCausalLM"],'
                                          '"model_type":"unsupported"}')
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(tmp_path), "cpu")
    assert e.value.kind == "InvalidConfig"
    assert e.value.problems == [("model_type", "unsupported model_type 'unsupported'")]
    (tmp_path / "config.json").write_text("{not json")
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(tmp_path), "cpu")
    assert e.value.kind == "InvalidConfig" and e.value.problems[0][0] == "config.json"
    (tmp_path / "config.json").write_text(json.dumps(LLAMA_TINY))
    (tmp_path / "pytorch_model.bin").write_bytes(b"\0" * 16)
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(tmp_path), "cpu")
    assert e.value.kind == "UnsupportedPickleWeights"
    assert e.value.problems[0][0] == "pytorch_model.bin"
