"""An f64 forward of the NCM level-parallel body in numpy, written from the
published architecture (RMSNorm with optional bias, rotate-half RoPE at the
given positions, grouped softmax attention under a boolean mask, optional
per-head QK RMSNorm before RoPE, SwiGLU MLP, residual adds) and the
reference's input stage (prefix table rows, learned level-0 queries, a
3-tap Conv1d with a residual per level, input projection + bias, level
embeddings). It is the independent check of the oracle's NCM composition."""
import math

import numpy as np


def random_ncm(rng, round_bf16, hidden, vq, inter, hq, hkv, hd, layers, levels, prefix,
               prefix_vocab, std=0.05, biases=False, qk_norm=False, convs=False,
               query_level0=True):
    """bf16-valued float32 weights in the reference's weights_t layout
    (src/ncm_model.zig:37-72)."""
    def w(*shape, s=std):
        return round_bf16((rng.standard_normal(shape) * s).astype(np.float32))

    def norm(n=hidden):
        return round_bf16((1 + 0.1 * rng.standard_normal(n)).astype(np.float32))

    def maybe(*shape):
        return w(*shape, s=0.05) if biases else None

    ls = []
    fused = (hq + 2 * hkv) * hd
    for _ in range(layers):
        ls.append(dict(
            fused_qkv_weight=w(fused, hidden), fused_qkv_bias=maybe(fused),
            output_weight=w(hidden, hq * hd), output_bias=maybe(hidden),
            query_norm_weight=norm(hd) if qk_norm else None,
            key_norm_weight=norm(hd) if qk_norm else None,
            ln_1_weight=norm(), ln_1_bias=maybe(hidden),
            gate_weight=w(inter, hidden), gate_bias=maybe(inter),
            up_weight=w(inter, hidden), up_bias=maybe(inter),
            down_weight=w(hidden, inter), down_bias=maybe(hidden),
            ln_2_weight=norm(), ln_2_bias=maybe(hidden),
        ))
    weights = dict(
        prefix_token_embedding=w(prefix_vocab, vq, s=1.0),
        prefix_vocab_size=prefix_vocab,
        input_projection=w(hidden, vq, s=1.0 / math.sqrt(vq)),
        input_projection_bias=w(hidden, s=0.05),
        level_embedding=w(len(levels), hidden, s=0.5),
        l0_queries=w(levels[0], vq, s=1.0) if query_level0 else None,
        final_norm_weight=norm(),
        final_norm_bias=maybe(hidden),
        layers=ls,
        post_upsample_convs=[dict(weight=w(vq, vq, 3, s=0.2 / math.sqrt(3 * vq)),
                                  bias=w(vq, s=0.05)) for _ in levels] if convs else [],
    )
    return weights


def ncm_forward_f64(cfg, weights, prefix_ids, target_inputs, mask, skip=None):
    """mask: bool [S, S] (True = key allowed). skip: None or a planted
    mistake ("positions": positions do not restart per level; "level":
    no level embeddings; "l0": level-0 inputs not replaced by the queries)."""
    H, vq = cfg["hidden_size"], cfg["vq_width"]
    hq, hkv, hd = cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"]
    eps = cfg["rms_norm_epsilon"]
    levels = list(cfg["level_lengths"])
    P = cfg["prefix_length"]
    S = P + sum(levels)
    f = lambda a: None if a is None else np.asarray(a, np.float64)
    x = np.zeros((S, vq))
    x[:P] = f(weights["prefix_token_embedding"]).reshape(-1, vq)[list(prefix_ids)]
    x[P:] = f(target_inputs).reshape(-1, vq)
    if cfg.get("query_level0", False) and skip != "l0":
        x[P:P + levels[0]] = f(weights["l0_queries"]).reshape(levels[0], vq)
    off = P
    for n, conv in zip(levels, weights.get("post_upsample_convs") or []):
        chunk = x[off:off + n]
        wc, bc = f(conv["weight"]).reshape(vq, vq, 3), f(conv["bias"])
        padded = np.concatenate([np.zeros((1, vq)), chunk, np.zeros((1, vq))])
        val = bc[None, :] + sum(padded[k:k + n] @ wc[:, :, k].T for k in range(3))
        x[off:off + n] = chunk + val
        off += n
    h = x @ f(weights["input_projection"]).T + f(weights["input_projection_bias"])
    if cfg.get("use_level_encoding", True) and skip != "level":
        emb = f(weights["level_embedding"]).reshape(len(levels), H)
        off = P
        for l, n in enumerate(levels):
            h[off:off + n] += emb[l]
            off += n
    if skip == "positions":
        pos = np.arange(S)
    else:
        pos = np.concatenate([np.arange(P)] + [np.arange(n) for n in levels])
    inv = np.asarray(cfg["inv_freq"], np.float64)
    ang = pos[:, None] * inv[None, :]
    cos = np.concatenate([np.cos(ang)] * 2, axis=1)
    sin = np.concatenate([np.sin(ang)] * 2, axis=1)

    def rms(v, w, b=None):
        y = v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps) * f(w)
        return y if b is None else y + f(b)

    def rope(v, heads):
        out = v.copy()
        for hh in range(heads):
            s = v[:, hh * hd:(hh + 1) * hd]
            rot = np.concatenate([-s[:, hd // 2:], s[:, :hd // 2]], axis=1)
            out[:, hh * hd:(hh + 1) * hd] = s * cos + rot * sin
        return out

    def proj(v, w, b):
        y = v @ f(w).T
        return y if b is None else y + f(b)

    qw, kvw = hq * hd, hkv * hd
    for L in weights["layers"]:
        n = rms(h, L["ln_1_weight"], L.get("ln_1_bias"))
        wq, bq = f(L["fused_qkv_weight"]), f(L.get("fused_qkv_bias"))
        qkv = n @ wq.T + (0.0 if bq is None else bq)
        q, k, v = qkv[:, :qw], qkv[:, qw:qw + kvw], qkv[:, qw + kvw:]
        if L.get("query_norm_weight") is not None:
            q = rms(q.reshape(S, hq, hd), L["query_norm_weight"]).reshape(S, qw)
            k = rms(k.reshape(S, hkv, hd), L["key_norm_weight"]).reshape(S, kvw)
        q, k = rope(q, hq), rope(k, hkv)
        ctx = np.zeros((S, qw))
        for hh in range(hq):
            g = hh // (hq // hkv)
            s = q[:, hh * hd:(hh + 1) * hd] @ k[:, g * hd:(g + 1) * hd].T / math.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            mx = np.max(s, axis=1, keepdims=True)
            e = np.where(mask, np.exp(s - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
            den = e.sum(axis=1, keepdims=True)
            p = np.divide(e, den, out=np.zeros_like(e), where=den > 0)
            ctx[:, hh * hd:(hh + 1) * hd] = p @ v[:, g * hd:(g + 1) * hd]
        h = h + proj(ctx, L["output_weight"], L.get("output_bias"))
        n = rms(h, L["ln_2_weight"], L.get("ln_2_bias"))
        g = proj(n, L["gate_weight"], L.get("gate_bias"))
        u = proj(n, L["up_weight"], L.get("up_bias"))
        h = h + proj(g / (1 + np.exp(-g)) * u, L["down_weight"], L.get("down_bias"))
    return rms(h, weights["final_norm_weight"], weights.get("final_norm_bias"))
