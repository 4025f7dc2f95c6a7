"""numpy (float64) restatement of the upstream VQ-VAE tokenizer's inference
forward. TEST INFRASTRUCTURE ONLY: imported by the test suite, the smoke check
and the benchmark's CPU-baseline leg; the product path never imports it.

The upstream model is PyTorch code that is not part of the reference tree;
the reference documents it in research/reference/vq_forward_semantics.md (the
forward pass and its PyTorch semantics) and research/converter/
wmt14_tokenizer_keys.md (the released WMT14 tokenizer's configuration and its
96 state_dict entries). Eval mode throughout: every dropout is the identity,
there is no nested-dropout cutoff (vq_forward_semantics.md:105) and no EMA
write (:153).

Pinning (tests/test_oracle_vq_tokenizer.py):
  group_norm        torch.nn.functional.group_norm, affine=False
  area_pool         torch.nn.functional.interpolate(mode="area")
  linear_up         torch.nn.functional.interpolate(mode="linear"), default
                    align_corners
  down_stage        torch.nn.functional.conv1d (kernel = stride = s)
  up_stage          torch.nn.functional.conv_transpose1d (kernel = stride = s)
  phi               torch.nn.functional.conv1d (kernel 3, padding 1), blend
  cascade           the closed form of the identity initialisation
                    (vq_forward_semantics.md:132-135: mean pooling and repeat)
  quantize          brute-force nearest code per level (f64), the telescoping
                    identity zhat + r_K = z, and reconstruct(codes) == zhat
  decoder pieces    torch layer_norm, rms_norm, scaled_dot_product_attention,
                    gelu (exact) and linear
The composition itself (the order of the stages) follows the cited lines and
is checked only through the invariants above: parity with the upstream
PyTorch module is unpinned, since that code is not available.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


@dataclass
class TokenizerConfig:
    """Shapes and switches of one tokenizer (wmt14_tokenizer_keys.md section 2)."""
    embed_dim: int = 384                 # D (wmt14.yaml:52)
    in_vocab: int = 151680               # C (wmt14.yaml:53)
    context_length: int = 64             # T, encoder wpe rows (wmt14.yaml:54)
    levels: tuple = (1, 4, 8, 14, 20, 26, 32, 40, 48, 56, 64)   # wmt14.yaml:96-106
    vocab_sizes: tuple = (4096,) * 11    # wmt14.yaml:60-71
    groups: int = 8                      # pre-quant GroupNorm(8, D, affine=False)
    group_eps: float = 1e-5              # PyTorch GroupNorm default
    learned_level0: bool = True          # learned_l1_sampling (wmt14.yaml:78)
    cascade_base: int = 4                # learned_l1_cascade_base (wmt14.yaml:80)
    cascade_norm: bool = True            # learned_l1_cascade_norm (wmt14.yaml:81)
    cascade_norm_final: bool = True      # learned_l1_cascade_norm_final (wmt14.yaml:82)
    resi_ratio: float = 0.5              # quant_resi.ratio (wmt14.yaml:86)
    quant_resi: bool = True              # quant_resi.enabled (wmt14.yaml:85)
    n_head: int = 6                      # decoder heads = n_layers (wmt14.yaml:51)
    ln_eps: float = 1e-6                 # models/vae.py:6-13
    qk_eps: float = 1e-6                 # models/vae.py:16-26

    @property
    def seq_len(self) -> int:
        return self.levels[-1]

    @property
    def n_levels(self) -> int:
        return len(self.levels)

    def cascade_strides(self) -> list:
        return cascade_strides(self.seq_len // self.levels[0], self.cascade_base)


WMT14 = TokenizerConfig()
# The OWT tokenizer of vq_forward_semantics.md section 1: L = 1024, 32 levels
# of (k + 1)^2 positions, 8192 codes, no cascade norms, ratio 0.5.
OWT = TokenizerConfig(in_vocab=50304, context_length=1024,
                      levels=tuple((k + 1) ** 2 for k in range(32)),
                      vocab_sizes=(8192,) * 32, cascade_norm=False, cascade_norm_final=False)


def cascade_strides(total: int, base: int) -> list:
    """_plan_cascade_strides (models/quant.py:165-178, vq_forward_semantics.md:131):
    repeated division of the total stride by the base. Only exact powers of
    the base are restated (1024 -> [4]*5, 64 -> [4]*3); other totals raise."""
    if total < 1 or base < 2:
        raise ValueError("cascade stride plan needs total >= 1 and base >= 2")
    out = []
    rem = total
    while rem > 1:
        if rem % base:
            raise ValueError(f"total stride {total} is not a power of {base}")
        out.append(base)
        rem //= base
    return out


# ---------------------------------------------------------------- primitives
# Activations are [B, L, C] (position-major, channel-contiguous), the layout
# the device path uses; the PyTorch modules see the transposed [B, C, L].

def group_norm(x, groups, eps):
    """GroupNorm(groups, C, affine=False) over [B, L, C]: per sample and group,
    biased statistics over (C / groups channels) x L positions
    (vq_forward_semantics.md:46, wmt14_tokenizer_keys.md section 4)."""
    x = np.asarray(x, np.float64)
    b, l, c = x.shape
    g = x.reshape(b, l, groups, c // groups).transpose(0, 2, 1, 3).reshape(b, groups, -1)
    mean = g.mean(axis=2, keepdims=True)
    var = ((g - mean) ** 2).mean(axis=2, keepdims=True)
    y = (g - mean) / np.sqrt(var + eps)
    return y.reshape(b, groups, l, c // groups).transpose(0, 2, 1, 3).reshape(b, l, c)


def area_bounds(length, n):
    """Window [start, end) of output position j of adaptive average pooling
    (F.interpolate mode "area", vq_forward_semantics.md:80)."""
    return [((j * length) // n, -((-(j + 1) * length) // n)) for j in range(n)]


def area_pool(x, n):
    """F.interpolate(mode="area") along positions: [B, L, C] -> [B, n, C]."""
    x = np.asarray(x, np.float64)
    return np.stack([x[:, s:e].mean(axis=1) for s, e in area_bounds(x.shape[1], n)], axis=1)


def linear_weights(n, length):
    """Source indices and weights of F.interpolate(mode="linear",
    align_corners=False) from n to `length` positions
    (vq_forward_semantics.md:82): src = max((t + 0.5) * n / length - 0.5, 0)."""
    out = []
    scale = n / length
    for t in range(length):
        src = max(scale * (t + 0.5) - 0.5, 0.0)
        i0 = int(src)
        i1 = i0 + (1 if i0 < n - 1 else 0)
        lam = src - i0
        out.append((i0, i1, 1.0 - lam, lam))
    return out


def linear_up(x, length):
    """F.interpolate(mode="linear") along positions: [B, n, C] -> [B, length, C]."""
    x = np.asarray(x, np.float64)
    rows = [w0 * x[:, i0] + w1 * x[:, i1] for i0, i1, w0, w1 in linear_weights(x.shape[1], length)]
    return np.stack(rows, axis=1)


def down_stage(x, weight, bias, s):
    """Conv1d(C, C, kernel s, stride s, bias) over [B, L, C] (models/quant.py:145-152):
    y[j, o] = bias[o] + sum_k sum_c W[o, c, k] x[s j + k, c]. weight (out, in, s)."""
    x = np.asarray(x, np.float64)
    b, l, c = x.shape
    w = np.asarray(weight, np.float64)                    # [o, c, k]
    wk = w.transpose(0, 2, 1).reshape(w.shape[0], s * c)  # [o, (k, c)]
    return x.reshape(b, l // s, s * c) @ wk.T + np.asarray(bias, np.float64)


def up_stage(x, weight, bias, s):
    """ConvTranspose1d(C, C, kernel s, stride s, bias) over [B, n, C]
    (models/quant.py:155-162): y[s j + k, o] = bias[o] + sum_c W[c, o, k] x[j, c].
    weight (in, out, s)."""
    x = np.asarray(x, np.float64)
    b, n, c = x.shape
    w = np.asarray(weight, np.float64)                    # [c, o, k]
    o = w.shape[1]
    y = x @ w.transpose(0, 2, 1).reshape(c, s * o)        # [B, n, (k, o)]
    return (y.reshape(b, n, s, o) + np.asarray(bias, np.float64)).reshape(b, n * s, o)


def conv3(h, weight, bias):
    """Conv1d(C, C, kernel 3, stride 1, padding 1) over [B, L, C]
    (models/quant.py:11-20): y[t, o] = bias[o] + sum_k sum_c W[o, c, k] h[t + k - 1, c]."""
    h = np.asarray(h, np.float64)
    b, l, c = h.shape
    hp = np.zeros((b, l + 2, c))
    hp[:, 1:-1] = h
    w = np.asarray(weight, np.float64)
    return np.asarray(bias, np.float64) + sum(hp[:, k:k + l] @ w[:, :, k].T for k in range(3))


def phi(h, weight, bias, ratio):
    """Phi (models/quant.py:36-38, vq_forward_semantics.md:121): (1 - r) h + r Conv(h)."""
    h = np.asarray(h, np.float64)
    return (1.0 - ratio) * h + ratio * conv3(h, weight, bias)


# ------------------------------------------------------------------- encoder

def encode_front(cfg, ids, wte, wpe):
    """Encoder + pre-quant norm in eval mode (vq_forward_semantics.md:38-49):
    z = GroupNorm(wte[ids] + wpe[0..L-1])."""
    ids = np.asarray(ids)
    x = np.asarray(wte, np.float64)[ids] + np.asarray(wpe, np.float64)[: ids.shape[1]]
    return group_norm(x, cfg.groups, cfg.group_eps)


@dataclass
class QuantizerWeights:
    """Per-level codebooks and Phi convs plus the level-0 cascade (PyTorch layouts)."""
    codebooks: list                      # [V_i, D]
    resi_weight: list = field(default_factory=list)   # [D, D, 3] (out, in, k)
    resi_bias: list = field(default_factory=list)     # [D]
    down_weight: list = field(default_factory=list)   # [D, D, s] (out, in, k)
    down_bias: list = field(default_factory=list)
    up_weight: list = field(default_factory=list)     # [D, D, s] (in, out, k)
    up_bias: list = field(default_factory=list)


def cascade_down(cfg, w, r):
    """learned_down_l1 (models/quant.py:185-194, keys doc section 4): conv
    stages, GroupNorm after each inner stage (cascade_norm) and after the
    last (cascade_norm_final)."""
    x = np.asarray(r, np.float64)
    strides = cfg.cascade_strides()
    for i, s in enumerate(strides):
        x = down_stage(x, w.down_weight[i], w.down_bias[i], s)
        last = i == len(strides) - 1
        if (cfg.cascade_norm and not last) or (cfg.cascade_norm_final and last):
            x = group_norm(x, cfg.groups, cfg.group_eps)
    return x


def cascade_up(cfg, w, q):
    """learned_up_l1 (models/quant.py:197-204): transposed-conv stages with a
    GroupNorm between stages (cascade_norm), none after the last."""
    x = np.asarray(q, np.float64)
    strides = cfg.cascade_strides()
    for i, s in enumerate(strides):
        x = up_stage(x, w.up_weight[i], w.up_bias[i], s)
        if cfg.cascade_norm and i < len(strides) - 1:
            x = group_norm(x, cfg.groups, cfg.group_eps)
    return x


def _down(cfg, w, level, r):
    """_down_for_quant (models/quant.py:395-402, :472-476)."""
    if level == 0 and cfg.learned_level0:
        return cascade_down(cfg, w, r)
    if cfg.levels[level] == r.shape[1]:
        return np.asarray(r, np.float64)
    return area_pool(r, cfg.levels[level])


def _up(cfg, w, level, q):
    """_up_to_full (models/quant.py:404-411, :507-510)."""
    if level == 0 and cfg.learned_level0:
        return cascade_up(cfg, w, q)
    if cfg.levels[level] == cfg.seq_len:
        return np.asarray(q, np.float64)
    return linear_up(q, cfg.seq_len)


def _resi(cfg, w, level, h):
    """_apply_quant_resi (models/quant.py:380-386): Phi of module `level`."""
    if not cfg.quant_resi:
        return h
    return phi(h, w.resi_weight[level], w.resi_bias[level], cfg.resi_ratio)


def quantize(cfg, w, z, forced=None):
    """The multiscale residual loop (models/quant.py:448-549,
    vq_forward_semantics.md:59-76) in eval mode.

    forced: optional [B, sum(levels)] codes to use instead of the argmin (so a
    device result can be replayed level by level). Returns codes [B, sum],
    zhat [B, L, D], r (the residual after the last level) and, per level, the
    f64 distance of the used code and of the best code (`d_used`, `d_best`,
    [B, n_l] each)."""
    z = np.asarray(z, np.float64)
    b, length, d = z.shape
    r = z.copy()
    zhat = np.zeros_like(z)
    codes, d_used, d_best = [], [], []
    off = 0
    for level, n in enumerate(cfg.levels):
        u = _down(cfg, w, level, r)                                   # [B, n, D]
        e = np.asarray(w.codebooks[level], np.float64)
        dist = ((u * u).sum(-1)[..., None] + (e * e).sum(-1)
                - 2.0 * (u @ e.T))                                    # quant.py:388-393
        best = dist.argmin(-1)                                        # lowest index on ties
        idx = best if forced is None else np.asarray(forced)[:, off:off + n].astype(np.int64)
        d_used.append(np.take_along_axis(dist, idx[..., None], -1)[..., 0])
        d_best.append(dist.min(-1))
        codes.append(idx)
        q = e[idx]                                                    # [B, n, D]
        big_q = _resi(cfg, w, level, _up(cfg, w, level, q))          # [B, L, D]
        zhat = zhat + big_q
        r = r - big_q
        off += n
    return {"codes": np.concatenate(codes, axis=1).astype(np.int32), "zhat": zhat, "r": r,
            "d_used": d_used, "d_best": d_best}


def reconstruct(cfg, w, codes):
    """zhat = sum_l Phi_l(U_l(e_l[codes_l])) (the decoder input of
    vq_forward_semantics.md:76 in eval mode)."""
    codes = np.asarray(codes)
    zhat = None
    off = 0
    for level, n in enumerate(cfg.levels):
        e = np.asarray(w.codebooks[level], np.float64)
        big_q = _resi(cfg, w, level, _up(cfg, w, level, e[codes[:, off:off + n]]))
        zhat = big_q if zhat is None else zhat + big_q
        off += n
    return zhat


# ------------------------------------------------------------------- decoder

def layer_norm(x, weight, bias, eps):
    """LayerNorm (models/vae.py:6-13): (x - mean) / sqrt(var + eps) * w (+ b)."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps) * np.asarray(weight, np.float64)
    return y if bias is None else y + np.asarray(bias, np.float64)


def rms_norm(x, weight, eps):
    """RMSNorm (models/vae.py:16-26): x / sqrt(mean(x^2) + eps) * w."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(weight, np.float64)


def gelu(x):
    """Exact GELU (nn.GELU default, models/vae.py:77): x Phi(x) via erf."""
    from math import erf
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.vectorize(erf)(x / math.sqrt(2.0)))


def linear(x, weight, bias=None):
    y = np.asarray(x, np.float64) @ np.asarray(weight, np.float64).T
    return y if bias is None else y + np.asarray(bias, np.float64)


def decoder_forward(cfg, dw, zhat):
    """The VQ-VAE decoder (models/vae.py:198-258, vq_forward_semantics.md:84-94)
    in eval mode: one pre-LN block with bidirectional multi-head attention
    (QK RMSNorm) and a GELU MLP, then ln_f (no bias) and the output layer.
    dw: dict of the decoder's state_dict entries without the "decoder." prefix."""
    x = np.asarray(zhat, np.float64)
    b, t, d = x.shape
    hn = cfg.n_head
    hd = d // hn
    p = "middle_block."
    h = layer_norm(x, dw[p + "ln_1.weight"], dw[p + "ln_1.bias"], cfg.ln_eps)
    qkv = linear(h, dw[p + "attn.c_attn.weight"], dw[p + "attn.c_attn.bias"])
    q, k, v = (qkv[..., i * d:(i + 1) * d].reshape(b, t, hn, hd).transpose(0, 2, 1, 3)
               for i in range(3))
    q = rms_norm(q, dw[p + "attn.q_norm.weight"], cfg.qk_eps)
    k = rms_norm(k, dw[p + "attn.k_norm.weight"], cfg.qk_eps)
    s = q @ k.transpose(0, 1, 3, 2) / math.sqrt(hd)
    s = s - s.max(-1, keepdims=True)
    pr = np.exp(s)
    pr = pr / pr.sum(-1, keepdims=True)
    a = (pr @ v).transpose(0, 2, 1, 3).reshape(b, t, d)
    x = x + linear(a, dw[p + "attn.c_proj.weight"], dw[p + "attn.c_proj.bias"])
    h = layer_norm(x, dw[p + "ln_2.weight"], dw[p + "ln_2.bias"], cfg.ln_eps)
    h = gelu(linear(h, dw[p + "mlp.c_fc.weight"], dw[p + "mlp.c_fc.bias"]))
    x = x + linear(h, dw[p + "mlp.c_proj.weight"], dw[p + "mlp.c_proj.bias"])
    x = layer_norm(x, dw["ln_f.weight"], None, cfg.ln_eps)
    return linear(x, dw["output_layer.weight"])


# ------------------------------------------------------------ synthetic model

def random_weights(cfg, seed=0, vocab_cap=None):
    """Random-initialised weights of the configuration's shapes (float32):
    N(0, 1) codebooks (models/quant.py:299), Conv and Linear weights at
    PyTorch's default uniform(+-1/sqrt(fan_in)) scale. `vocab_cap` bounds the
    token table and output-layer rows (small test models)."""
    rng = np.random.default_rng(seed)
    d = cfg.embed_dim
    c = cfg.in_vocab if vocab_cap is None else min(cfg.in_vocab, vocab_cap)

    def uni(shape, fan_in):
        bound = 1.0 / math.sqrt(fan_in)
        return rng.uniform(-bound, bound, size=shape).astype(np.float32)

    strides = cfg.cascade_strides() if cfg.learned_level0 else []
    qw = QuantizerWeights(
        codebooks=[rng.standard_normal((v, d)).astype(np.float32) for v in cfg.vocab_sizes],
        resi_weight=[uni((d, d, 3), 3 * d) for _ in cfg.levels],
        resi_bias=[uni((d,), 3 * d) for _ in cfg.levels],
        down_weight=[uni((d, d, s), s * d) for s in strides],
        down_bias=[uni((d,), s * d) for s in strides],
        up_weight=[uni((d, d, s), s * d) for s in strides],
        up_bias=[uni((d,), s * d) for s in strides],
    )
    enc = {"wte": rng.standard_normal((c, d)).astype(np.float32),
           "wpe": rng.standard_normal((cfg.context_length, d)).astype(np.float32)}
    hd = d // cfg.n_head
    p = "middle_block."
    dec = {
        "ln_f.weight": (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        p + "ln_1.weight": (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        p + "ln_1.bias": (0.1 * rng.standard_normal(d)).astype(np.float32),
        p + "attn.c_attn.weight": uni((3 * d, d), d),
        p + "attn.c_attn.bias": uni((3 * d,), d),
        p + "attn.c_proj.weight": uni((d, d), d),
        p + "attn.c_proj.bias": uni((d,), d),
        p + "attn.q_norm.weight": (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
        p + "attn.k_norm.weight": (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32),
        p + "ln_2.weight": (1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        p + "ln_2.bias": (0.1 * rng.standard_normal(d)).astype(np.float32),
        p + "mlp.c_fc.weight": uni((4 * d, d), d),
        p + "mlp.c_fc.bias": uni((4 * d,), d),
        p + "mlp.c_proj.weight": uni((d, 4 * d), 4 * d),
        p + "mlp.c_proj.bias": uni((d,), 4 * d),
        "output_layer.weight": uni((c, d), d),
    }
    return enc, qw, dec
