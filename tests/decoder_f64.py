"""An f64 Llama-style decoder forward in numpy (the published architecture:
RMSNorm, rotate-half RoPE, grouped causal softmax attention, SwiGLU MLP,
residual adds, tied or separate LM head), used as the independent check of
the oracle's bf16 composition."""
import math

import numpy as np


def forward_f64(ids, embed, layers, final_norm, lm_head, cos, sin, hq, hkv, hd, eps, window=0,
                skip=None):
    """skip: None, "rope", "residual" or "qk_norm" (a planted mistake, to
    show that a test's bound tells the composition apart from a wrong one).
    A layer with q_norm / k_norm [head_dim] scales RMS-normalizes every
    query and key head before the rotation (Qwen3)."""
    x = embed[np.asarray(ids)].astype(np.float64)
    t = len(ids)
    qi, ki = np.meshgrid(np.arange(t), np.arange(t), indexing="ij")
    mask = (ki <= qi) & ((window == 0) | (qi - window < ki))

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v, axis=1, keepdims=True) + eps) * w

    def rope(v, heads):
        out = v.copy()
        for h in range(heads):
            s = v[:, h * hd:(h + 1) * hd]
            rot = np.concatenate([-s[:, hd // 2:], s[:, :hd // 2]], axis=1)
            out[:, h * hd:(h + 1) * hd] = s * cos + rot * sin
        return out

    def head_rms(v, heads, w):
        out = v.copy()
        for h in range(heads):
            out[:, h * hd:(h + 1) * hd] = rms(v[:, h * hd:(h + 1) * hd], w)
        return out

    def bias(b):
        return 0.0 if b is None else b.astype(np.float64)

    for layer in layers:
        n = rms(x, layer["input_norm"])
        qkv = n @ layer["qkv_weight"].T.astype(np.float64) + bias(layer.get("qkv_bias"))
        q = qkv[:, :hq * hd]
        k = qkv[:, hq * hd:(hq + hkv) * hd]
        v = qkv[:, (hq + hkv) * hd:]
        if layer.get("q_norm") is not None and skip != "qk_norm":
            q, k = head_rms(q, hq, layer["q_norm"]), head_rms(k, hkv, layer["k_norm"])
        if skip != "rope":
            q, k = rope(q, hq), rope(k, hkv)
        ctx = np.zeros((t, hq * hd))
        for h in range(hq):
            kv = h // (hq // hkv)
            s = q[:, h * hd:(h + 1) * hd] @ k[:, kv * hd:(kv + 1) * hd].T / math.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            e = np.exp(s - s.max(axis=1, keepdims=True))
            ctx[:, h * hd:(h + 1) * hd] = (e / e.sum(axis=1, keepdims=True)) @ v[:, kv * hd:(kv + 1) * hd]
        att = ctx @ layer["o_weight"].T.astype(np.float64) + bias(layer.get("o_bias"))
        x = att if skip == "residual" else x + att
        n = rms(x, layer["post_attention_norm"])
        inter = layer["gate_up_weight"].shape[0] // 2
        gu = n @ layer["gate_up_weight"].T.astype(np.float64) + bias(layer.get("gate_up_bias"))
        g, u = gu[:, :inter], gu[:, inter:]
        a = g / (1 + np.exp(-g)) * u
        x = x + a @ layer["down_weight"].T.astype(np.float64) + bias(layer.get("down_bias"))
    n = rms(x, final_norm)
    head = embed if lm_head is None else lm_head
    return n @ head.T.astype(np.float64)


def random_model(rng, round_bf16, hidden, inter, vocab, hq, hkv, hd, layers, std=0.05,
                 biases=False, qk_norm=False):
    """bf16-valued float32 weights: projections ~N(0, std), embeddings
    ~N(0, 5 std), norm scales ~1 + N(0, 0.1); with qk_norm, per-head query
    and key norm scales ~1.2 + N(0, 0.2)."""
    def w(*shape, s=std):
        return round_bf16((rng.standard_normal(shape) * s).astype(np.float32))

    def norm():
        return round_bf16((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float32))

    ls = []
    for _ in range(layers):
        ls.append(dict(
            input_norm=norm(),
            qkv_weight=w((hq + 2 * hkv) * hd, hidden),
            qkv_bias=w((hq + 2 * hkv) * hd, s=0.05) if biases else None,
            o_weight=w(hidden, hq * hd),
            o_bias=w(hidden, s=0.05) if biases else None,
            post_attention_norm=norm(),
            gate_up_weight=w(2 * inter, hidden),
            gate_up_bias=w(2 * inter, s=0.05) if biases else None,
            down_weight=w(hidden, inter),
            down_bias=w(hidden, s=0.05) if biases else None,
        ))
        if qk_norm:
            for name in ("q_norm", "k_norm"):
                ls[-1][name] = round_bf16((1.2 + 0.2 * rng.standard_normal(hd)).astype(np.float32))
    return w(vocab, hidden, s=5 * std), ls, norm()
