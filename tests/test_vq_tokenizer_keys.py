"""The tokenizer's state_dict table and checkpoint checks (CPU).

Golden values: research/converter/wmt14_tokenizer_keys.md section 3 (the 96
rows, their order and shapes) and section 6 (144,002,816 parameter scalars,
17,391,616 buffer scalars).
"""
import dataclasses
import math

import numpy as np
import pytest

from ncmorph_amd import vq_tokenizer as vt
from ncmorph_amd.safetensors import write_file

WMT = vt.WMT14


def test_wmt14_has_96_entries_in_state_dict_order():
    e = vt.state_dict_entries(WMT)
    assert len(e) == 96
    names = [n for n, _, _ in e]
    assert len(set(names)) == 96
    # rows of section 3 (1-based there)
    assert e[0] == ("encoder.wte.weight", (151680, 384), "float32")
    assert e[1] == ("encoder.wpe.weight", (64, 384), "float32")
    assert e[2][0] == "vq.ema_cluster_size_0" and e[4] == ("vq.codebook_hit_0", (4096,), "int64")
    assert e[35] == ("vq.embeddings.0.weight", (4096, 384), "float32")
    assert e[46] == ("vq.quant_resi.0.weight", (384, 384, 3), "float32")
    assert e[67] == ("vq.quant_resi.10.bias", (384,), "float32")
    assert [n for n, _, _ in e[68:80]] == [
        "vq.learned_down_l1.0.weight", "vq.learned_down_l1.0.bias",
        "vq.learned_down_l1.2.weight", "vq.learned_down_l1.2.bias",
        "vq.learned_down_l1.4.weight", "vq.learned_down_l1.4.bias",
        "vq.learned_up_l1.0.weight", "vq.learned_up_l1.0.bias",
        "vq.learned_up_l1.2.weight", "vq.learned_up_l1.2.bias",
        "vq.learned_up_l1.4.weight", "vq.learned_up_l1.4.bias"]
    assert e[68][1] == (384, 384, 4)
    assert e[80] == ("decoder.ln_f.weight", (384,), "float32")
    assert e[87] == ("decoder.middle_block.attn.q_norm.weight", (64,), "float32")
    assert e[95] == ("decoder.output_layer.weight", (151680, 384), "float32")


def test_wmt14_scalar_totals():
    e = vt.state_dict_entries(WMT)
    buffers = [x for x in e if x[0].startswith(("vq.ema_", "vq.codebook_hit_"))]
    params = [x for x in e if x not in buffers]
    count = lambda xs: sum(math.prod(s) for _, s, _ in xs)  # noqa: E731
    assert len(params) == 63 and len(buffers) == 33
    assert count(params) == 144_002_816
    assert count(buffers) == 17_391_616


def test_owt_layout_has_no_cascade_norm_gaps():
    cfg = vt.TokenizerConfig(in_vocab=50304, context_length=1024,
                             levels=tuple((k + 1) ** 2 for k in range(32)),
                             vocab_sizes=(8192,) * 32, cascade_norm=False,
                             cascade_norm_final=False)
    assert cfg.cascade_strides() == [4] * 5
    names = [n for n, _, _ in vt.state_dict_entries(cfg)]
    assert [n for n in names if "learned_down_l1" in n and n.endswith("weight")] == [
        f"vq.learned_down_l1.{i}.weight" for i in range(5)]
    assert sum("quant_resi" in n for n in names) == 64


def test_config_validation():
    with pytest.raises(ValueError):
        dataclasses.replace(WMT, levels=(1, 4, 4, 64), vocab_sizes=(8,) * 4).validate()
    with pytest.raises(ValueError):
        dataclasses.replace(WMT, context_length=32).validate()
    with pytest.raises(ValueError):
        dataclasses.replace(WMT, levels=(1, 48), vocab_sizes=(8, 8), context_length=48).validate()
    dataclasses.replace(WMT, levels=(1, 4, 16), vocab_sizes=(8,) * 3).validate()


def _present(cfg):
    return {n: ("I64" if d == "int64" else "F32", s) for n, s, d in vt.state_dict_entries(cfg)}


def test_check_entries_finds_every_kind_of_problem():
    p = _present(WMT)
    assert vt.check_entries(WMT, p) == []
    q = dict(p)
    del q["vq.embeddings.3.weight"]
    q["vq.embeddings.11.weight"] = ("F32", (4096, 384))
    q["vq.quant_resi.2.weight"] = ("F32", (384, 384, 5))
    q["decoder.ln_f.weight"] = ("I32", (384,))
    probs = vt.check_entries(WMT, q)
    assert "missing vq.embeddings.3.weight" in probs
    assert "unexpected vq.embeddings.11.weight" in probs
    assert any(x.startswith("shape vq.quant_resi.2.weight") for x in probs)
    assert any(x.startswith("dtype decoder.ln_f.weight") for x in probs)
    # bf16 / f16 storage is accepted for float entries
    q = dict(p)
    q["vq.embeddings.0.weight"] = ("BF16", (4096, 384))
    assert vt.check_entries(WMT, q) == []


def test_load_rejects_before_reading(tmp_path):
    cfg = dataclasses.replace(WMT, in_vocab=10, levels=(1, 4, 16), vocab_sizes=(8, 8, 8),
                              context_length=16, embed_dim=32, groups=4, n_head=2)
    tensors = {}
    for n, s, d in vt.state_dict_entries(cfg):
        dt = np.int64 if d == "int64" else np.float32
        tensors[n] = ("I64" if d == "int64" else "F32", s, np.zeros(s, dt).tobytes())
    tensors.pop("vq.quant_resi.1.bias")
    path = tmp_path / "tokenizer.safetensors"
    write_file(str(path), tensors)
    with pytest.raises(vt.TokenizerError) as ei:
        vt.load(str(path), cfg, device="cpu")
    assert ei.value.problems == ["missing vq.quant_resi.1.bias"]
