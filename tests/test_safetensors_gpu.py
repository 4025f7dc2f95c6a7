"""Device weight path: safetensors tensors uploaded to HBM as stored (bytes
identical, across the pinned staging chunks) and a Llama-layout checkpoint
(single file and sharded) loaded into the decoder's layout: the forward
gives the same bits as with the same weights handed over directly."""
import json
import os

import numpy as np
import pytest

from ncmorph_amd import safetensors as st
from ncmorph_amd import synth

from .decoder_f64 import random_model

pytestmark = pytest.mark.gpu


def test_upload_bytes_identical(ncm, cuda, tmp_path):
    import torch

    rng = np.random.default_rng(1)
    big = rng.integers(0, 2**16, 150 * 2**20 // 2 + 7, dtype=np.uint16)  # > two 64 MB chunks
    small = rng.standard_normal(33).astype(np.float32)
    p = str(tmp_path / "w.safetensors")
    st.write_file(p, {"big": ("BF16", (big.size,), big.tobytes()),
                      "small": ("F32", (33,), small.tobytes()),
                      "empty": ("BF16", (0, 4), b"")})
    with st.SafetensorsFile(p) as f:
        out = torch.empty(big.size, dtype=torch.int16, device=cuda)
        f.upload("big", out)
        o2 = torch.empty(33, dtype=torch.float32, device=cuda)
        f.upload("small", o2)
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy().view(np.uint16), big)
        assert np.array_equal(o2.cpu().numpy(), small)
        with pytest.raises(st.NcmError):  # wrong byte count
            f.upload("small", torch.empty(32, dtype=torch.float32, device=cuda))
        with pytest.raises(st.NcmError):
            f.upload("missing", o2)
        assert f.find("empty").shape == (0, 4)


def test_upload_staging_reuse(ncm, cuda, tmp_path):
    """One context's pinned staging grows and is reused: uploads of growing,
    shrinking and odd sizes in a row (one and several copy threads, one and
    several chunks) all arrive bytes identical."""
    import torch

    rng = np.random.default_rng(2)
    sizes = [1000, 3 << 20, (5 << 20) + 3, 70 << 20, 17, (130 << 20) + 1]
    arrays = {f"t{i}": rng.integers(0, 256, n, dtype=np.uint8) for i, n in enumerate(sizes)}
    p = str(tmp_path / "w.safetensors")
    st.write_file(p, {k: ("U8", (a.size,), a.tobytes()) for k, a in arrays.items()})
    with st.SafetensorsFile(p) as f:
        for rep in range(2):
            for k, a in arrays.items():
                out = torch.empty(a.size, dtype=torch.uint8, device=cuda)
                f.upload(k, out)
                torch.cuda.synchronize()
                assert np.array_equal(out.cpu().numpy(), a), (rep, k)


def _write_checkpoint(path, embed, layers, fnorm, hq, hkv, hd, shards=1, f32_keys=(),
                      f16_keys=(), lm_head=None):
    tensors = {"model.embed_tokens.weight": embed}
    qw, kw = hq * hd, hkv * hd
    inter = layers[0]["gate_up_weight"].shape[0] // 2
    for i, L in enumerate(layers):
        p = f"model.layers.{i}."
        tensors[p + "input_layernorm.weight"] = L["input_norm"]
        tensors[p + "self_attn.q_proj.weight"] = L["qkv_weight"][:qw]
        tensors[p + "self_attn.k_proj.weight"] = L["qkv_weight"][qw:qw + kw]
        tensors[p + "self_attn.v_proj.weight"] = L["qkv_weight"][qw + kw:]
        if L.get("qkv_bias") is not None:
            tensors[p + "self_attn.q_proj.bias"] = L["qkv_bias"][:qw]
            tensors[p + "self_attn.k_proj.bias"] = L["qkv_bias"][qw:qw + kw]
            tensors[p + "self_attn.v_proj.bias"] = L["qkv_bias"][qw + kw:]
        tensors[p + "self_attn.o_proj.weight"] = L["o_weight"]
        tensors[p + "post_attention_layernorm.weight"] = L["post_attention_norm"]
        tensors[p + "mlp.gate_proj.weight"] = L["gate_up_weight"][:inter]
        tensors[p + "mlp.up_proj.weight"] = L["gate_up_weight"][inter:]
        tensors[p + "mlp.down_proj.weight"] = L["down_weight"]
        if L.get("o_bias") is not None:
            tensors[p + "self_attn.o_proj.bias"] = L["o_bias"]
        if L.get("gate_up_bias") is not None:
            tensors[p + "mlp.gate_proj.bias"] = L["gate_up_bias"][:inter]
            tensors[p + "mlp.up_proj.bias"] = L["gate_up_bias"][inter:]
        if L.get("down_bias") is not None:
            tensors[p + "mlp.down_proj.bias"] = L["down_bias"]
        if L.get("q_norm") is not None:
            tensors[p + "self_attn.q_norm.weight"] = L["q_norm"]
            tensors[p + "self_attn.k_norm.weight"] = L["k_norm"]
    tensors["model.norm.weight"] = fnorm
    if lm_head is not None:
        tensors["lm_head.weight"] = lm_head

    def entry(name, a):
        a = np.ascontiguousarray(a, np.float32)
        if name in f32_keys:
            return ("F32", a.shape, a.tobytes())
        if name in f16_keys:
            h = a.astype(np.float16)
            assert np.array_equal(h.astype(np.float32), a)  # exact in f16
            return ("F16", a.shape, h.tobytes())
        return ("BF16", a.shape, synth.bf16_bits(a).tobytes())

    names = list(tensors)
    if shards == 1:
        st.write_file(os.path.join(path, "model.safetensors"),
                      {n: entry(n, tensors[n]) for n in names}, metadata={"format": "pt"})
        return
    wm = {}
    for s in range(shards):
        part = names[s::shards]
        fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        st.write_file(os.path.join(path, fname), {n: entry(n, tensors[n]) for n in part})
        wm.update({n: fname for n in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {"total_size": 0}, "weight_map": wm}, f)


@pytest.mark.parametrize("shards,biases,f32", [(1, False, False), (3, True, True)])
def test_checkpoint_loads_into_decoder(ncm, oracle, cuda, tmp_path, shards, biases, f32):
    import torch
    from ncmorph_amd import decoder, kernels

    rng = np.random.default_rng(shards)
    hidden, inter, vocab, hq, hkv, hd, nl = 256, 512, 300, 4, 2, 64, 2
    embed, layers, fnorm = random_model(rng, oracle.round_bf16, hidden, inter, vocab, hq, hkv,
                                        hd, nl, biases=biases)
    f32_keys = ("model.layers.0.mlp.down_proj.weight", "model.norm.weight") if f32 else ()
    _write_checkpoint(str(tmp_path), embed, layers, fnorm, hq, hkv, hd, shards, f32_keys)
    spec = decoder.DecoderSpec(hidden=hidden, intermediate=inter, vocab=vocab, q_heads=hq,
                               kv_heads=hkv, head_dim=hd, layers=nl)
    loaded = decoder.load_safetensors(spec, str(tmp_path), cuda)

    def dev16(a):
        return torch.from_numpy(synth.bf16_bits(np.ascontiguousarray(a, np.float32))
                                .view(np.int16).copy()).to(cuda).view(torch.bfloat16)

    direct = []
    for L in layers:
        d = {k: (torch.from_numpy(v).to(cuda) if k.endswith("norm") else
                 (None if v is None else dev16(v))) for k, v in L.items()}
        d["gate_up_weight"] = dev16(kernels.interleave_gate_up(L["gate_up_weight"][:inter],
                                                                L["gate_up_weight"][inter:]))
        if L.get("gate_up_bias") is not None:
            d["gate_up_bias"] = dev16(kernels.interleave_gate_up(L["gate_up_bias"][:inter],
                                                                  L["gate_up_bias"][inter:]))
        direct.append(d)
    w = decoder.DecoderWeights(embed=dev16(embed), final_norm=torch.from_numpy(fnorm).to(cuda),
                               layers=direct)
    cos, sin = decoder.rope_tables(spec, 40)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    ids = rng.integers(0, vocab, (2, 40))
    a = decoder.forward(spec, loaded, ids, cd, sd)
    b = decoder.forward(spec, w, ids, cd, sd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _direct_weights(cuda, embed, layers, fnorm, inter, lm_head=None):
    """The same weights handed to the decoder directly, in its layout."""
    import torch
    from ncmorph_amd import decoder, kernels

    def dev16(a):
        return torch.from_numpy(synth.bf16_bits(np.ascontiguousarray(a, np.float32))
                                .view(np.int16).copy()).to(cuda).view(torch.bfloat16)

    direct = []
    for L in layers:
        d = {k: (torch.from_numpy(v).to(cuda) if k.endswith("norm") else
                 (None if v is None else dev16(v))) for k, v in L.items()}
        d["gate_up_weight"] = dev16(kernels.interleave_gate_up(L["gate_up_weight"][:inter],
                                                                L["gate_up_weight"][inter:]))
        direct.append(d)
    return decoder.DecoderWeights(embed=dev16(embed), final_norm=torch.from_numpy(fnorm).to(cuda),
                                  layers=direct, lm_head=None if lm_head is None else
                                  dev16(lm_head))


def test_qwen3_checkpoint_with_config(ncm, oracle, cuda, tmp_path):
    """load_checkpoint on a Qwen3-layout directory (config.json, QK-norm
    scales, tied embeddings with a stored equal lm_head, F16 norm scales):
    the manifest passes, the weights load (reads counted) and the forward
    gives the bits of the same weights handed over directly. A stored
    lm_head that differs from the tied embeddings in one element is refused
    as TiedHeadMismatch (src/loader.zig:259-267)."""
    import torch
    from ncmorph_amd import decoder

    rng = np.random.default_rng(11)
    hidden, inter, vocab, hq, hkv, hd, nl = 256, 512, 300, 4, 2, 64, 2
    embed, layers, fnorm = random_model(rng, oracle.round_bf16, hidden, inter, vocab, hq, hkv,
                                        hd, nl, qk_norm=True)
    cfg = {"architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3", "vocab_size": vocab,
           "hidden_size": hidden, "intermediate_size": inter, "num_hidden_layers": nl,
           "num_attention_heads": hq, "num_key_value_heads": hkv, "head_dim": hd,
           "rms_norm_eps": 1e-6, "rope_theta": 1000000.0, "tie_word_embeddings": True,
           "attention_bias": False, "use_sliding_window": False}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    f16 = ("model.norm.weight", "model.layers.1.self_attn.q_norm.weight")
    _write_checkpoint(str(tmp_path), embed, layers, fnorm, hq, hkv, hd, shards=2,
                      f16_keys=f16, lm_head=embed)
    reads = [0]
    # F16 tensors would select the f32 mode (as the reference's loader); the
    # bf16 layout is asked for explicitly.
    mc, spec, loaded = decoder.load_checkpoint(str(tmp_path), cuda, read_count=reads,
                                               mode="bf16")
    assert mc.family == "Qwen3" and spec.head_dim == hd and spec.tie_word_embeddings
    assert reads[0] >= nl * 11 + 2
    assert loaded.lm_head is None
    w = _direct_weights(cuda, embed, layers, fnorm, inter)
    cos, sin = decoder.rope_tables(spec, 33)
    cd, sd = torch.from_numpy(cos).to(cuda), torch.from_numpy(sin).to(cuda)
    ids = rng.integers(0, vocab, (1, 33))
    a = decoder.forward(spec, loaded, ids, cd, sd)
    b = decoder.forward(spec, w, ids, cd, sd)
    torch.cuda.synchronize()
    assert torch.equal(a, b)

    bad = embed.copy()
    bad[7, 3] = oracle.round_bf16(np.array([bad[7, 3] + 0.5], np.float32))[0]
    d2 = tmp_path / "mismatch"
    d2.mkdir()
    (d2 / "config.json").write_text(json.dumps(cfg))
    _write_checkpoint(str(d2), embed, layers, fnorm, hq, hkv, hd, lm_head=bad)
    with pytest.raises(decoder.CheckpointError) as e:
        decoder.load_checkpoint(str(d2), cuda)
    assert e.value.kind == "TiedHeadMismatch"


def test_f32_checkpoint_loads_in_f32_mode(ncm, oracle, cuda, tmp_path):
    """A checkpoint holding F32 tensors loads in the reference's f32 mode
    (bf16_compute only when every tensor is BF16, src/loader.zig:191-199):
    load_checkpoint picks it, and the f32 forward of the loaded weights gives
    the bits of the same weights handed over directly; mode="bf16" forces
    the bf16 layout."""
    import torch
    from ncmorph_amd import decoder

    rng = np.random.default_rng(13)
    hidden, inter, vocab, hq, hkv, hd, nl = 128, 256, 200, 4, 2, 32, 2
    embed, layers, fnorm = random_model(rng, lambda a: np.asarray(a, np.float32), hidden, inter,
                                        vocab, hq, hkv, hd, nl, biases=True)
    cfg = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "vocab_size": vocab,
           "hidden_size": hidden, "intermediate_size": inter, "num_hidden_layers": nl,
           "num_attention_heads": hq, "num_key_value_heads": hkv, "rms_norm_eps": 1e-5,
           "rope_theta": 10000.0, "attention_bias": True, "mlp_bias": True,
           "tie_word_embeddings": False}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    everything = ["model.embed_tokens.weight", "model.norm.weight", "lm_head.weight"]
    for i in range(nl):
        p = f"model.layers.{i}."
        everything += [p + s for s in (
            "input_layernorm.weight", "post_attention_layernorm.weight",
            "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
            "self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias",
            "self_attn.o_proj.weight", "self_attn.o_proj.bias", "mlp.gate_proj.weight",
            "mlp.up_proj.weight", "mlp.down_proj.weight", "mlp.gate_proj.bias",
            "mlp.up_proj.bias", "mlp.down_proj.bias")]
    head = (rng.standard_normal((vocab, hidden)) * 0.05).astype(np.float32)
    _write_checkpoint(str(tmp_path), embed, layers, fnorm, hq, hkv, hd, f32_keys=everything,
                      lm_head=head)
    cfg_spec, spec, w = decoder.load_checkpoint(str(tmp_path), cuda)
    assert w.mode == "f32" and w.layers[0]["qkv_weight"].dtype == torch.float32
    from .test_decoder_f32_gpu import _f32_weights

    direct = _f32_weights(decoder, cuda, embed, layers, fnorm, lm_head=head)
    cos, sin = oracle.rope_tables(oracle.rope_default_frequencies(hd, 10000.0), 29)
    cd = torch.from_numpy(cos).to(cuda)
    sd = torch.from_numpy(sin).to(cuda)
    ids = rng.integers(0, vocab, (2, 29))
    a = decoder.run(spec, w, ids, cd, sd)
    b = decoder.forward_f32(spec, direct, ids, cd, sd)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    _, _, w16 = decoder.load_checkpoint(str(tmp_path), cuda, mode="bf16")
    assert w16.mode == "bf16" and w16.layers[0]["qkv_weight"].dtype == torch.bfloat16
