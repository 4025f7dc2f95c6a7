"""The upstream VQ-VAE tokenizer (inference) on device tensors.

The tokenizer of research/reference/vq_forward_semantics.md: an encoder
(token and position tables, pre-quant GroupNorm), the multiscale residual
quantizer with area down-sampling, linear up-sampling, the per-level Phi
blend conv and the learned level-0 conv cascade, and a one-block decoder.
The released WMT14 tokenizer's configuration and state_dict entries are
research/converter/wmt14_tokenizer_keys.md sections 2-3. The reference plans
this path as a Zig port (ROADMAP.md:259-261, packages/vq) and has no code for
it; these wrappers follow the conventions of its kernels module (flat device
buffers, explicit sizes, caller-visible outputs) and the C ABI of
include/ncmorph_amd.h (ncm_vq_tok_*).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from . import _check as _ck
from ._lib import NCM_E_ARG, NCM_E_SHAPE, NcmError, check, lib
from .context import default_context

MAX_LEVELS = 64
MAX_STAGES = 8


@dataclass
class TokenizerConfig:
    """The tokenizer.vqvae block of a config (wmt14_tokenizer_keys.md
    section 2); field names match the test oracle's configuration."""
    embed_dim: int = 384
    in_vocab: int = 151680
    context_length: int = 64
    levels: tuple = (1, 4, 8, 14, 20, 26, 32, 40, 48, 56, 64)
    vocab_sizes: tuple = (4096,) * 11
    groups: int = 8
    group_eps: float = 1e-5
    learned_level0: bool = True
    cascade_base: int = 4
    cascade_norm: bool = True
    cascade_norm_final: bool = True
    resi_ratio: float = 0.5
    quant_resi: bool = True
    n_head: int = 6
    ln_eps: float = 1e-6
    qk_eps: float = 1e-6

    @property
    def seq_len(self) -> int:
        return self.levels[-1]

    @property
    def n_levels(self) -> int:
        return len(self.levels)

    @property
    def codes_per_sequence(self) -> int:
        return int(sum(self.levels))

    def cascade_strides(self) -> list:
        """_plan_cascade_strides (models/quant.py:165-178): the total level-0
        stride L / levels[0] divided by the base until 1; totals that are not
        a power of the base are rejected (their plan is not documented)."""
        if not self.learned_level0:
            return []
        total = self.seq_len // self.levels[0]
        out, rem = [], total
        while rem > 1:
            if rem % self.cascade_base:
                raise ValueError(f"level-0 stride {total} is not a power of {self.cascade_base}")
            out.append(self.cascade_base)
            rem //= self.cascade_base
        return out

    def validate(self) -> None:
        k = self.n_levels
        if not 1 <= k <= MAX_LEVELS or len(self.vocab_sizes) != k:
            raise ValueError("levels and vocab_sizes must have the same length, 1 .. 64")
        if any(b <= a for a, b in zip(self.levels, self.levels[1:])) or self.levels[0] < 1:
            raise ValueError("levels must be positive and increasing")
        if self.context_length < self.seq_len:
            raise ValueError("context_length is shorter than the last level")
        if self.embed_dim % (4 * self.groups) or self.embed_dim % self.n_head:
            raise ValueError("embed_dim must be a multiple of 4 * groups and of n_head")
        if self.learned_level0 and self.seq_len % self.levels[0]:
            raise ValueError("the level-0 stride must divide the sequence length")
        if len(self.cascade_strides()) > MAX_STAGES:
            raise ValueError("more than 8 cascade stages")


WMT14 = TokenizerConfig()


def state_dict_entries(cfg: TokenizerConfig) -> list:
    """(name, shape, torch dtype name) of every state_dict entry of the
    module in state_dict order (wmt14_tokenizer_keys.md section 3: 96 for
    WMT14). Cascade GroupNorms have no entries, so the down convs sit at
    indices 0, 2, 4, ... when cascade norms are on (section 4)."""
    d, c = cfg.embed_dim, cfg.in_vocab
    out = [("encoder.wte.weight", (c, d), "float32"),
           ("encoder.wpe.weight", (cfg.context_length, d), "float32")]
    for i, v in enumerate(cfg.vocab_sizes):
        out += [(f"vq.ema_cluster_size_{i}", (v,), "float32"),
                (f"vq.ema_w_{i}", (v, d), "float32"),
                (f"vq.codebook_hit_{i}", (v,), "int64")]
    out += [(f"vq.embeddings.{i}.weight", (v, d), "float32")
            for i, v in enumerate(cfg.vocab_sizes)]
    if cfg.quant_resi:
        for i in range(cfg.n_levels):
            out += [(f"vq.quant_resi.{i}.weight", (d, d, 3), "float32"),
                    (f"vq.quant_resi.{i}.bias", (d,), "float32")]
    for kind in ("down", "up"):
        for j, s in enumerate(cfg.cascade_strides()):
            idx = _cascade_index(cfg, kind, j)
            out += [(f"vq.learned_{kind}_l1.{idx}.weight", (d, d, s), "float32"),
                    (f"vq.learned_{kind}_l1.{idx}.bias", (d,), "float32")]
    p = "decoder.middle_block."
    hd = d // cfg.n_head
    out += [("decoder.ln_f.weight", (d,), "float32"),
            (p + "ln_1.weight", (d,), "float32"), (p + "ln_1.bias", (d,), "float32"),
            (p + "attn.c_attn.weight", (3 * d, d), "float32"),
            (p + "attn.c_attn.bias", (3 * d,), "float32"),
            (p + "attn.c_proj.weight", (d, d), "float32"), (p + "attn.c_proj.bias", (d,), "float32"),
            (p + "attn.q_norm.weight", (hd,), "float32"),
            (p + "attn.k_norm.weight", (hd,), "float32"),
            (p + "ln_2.weight", (d,), "float32"), (p + "ln_2.bias", (d,), "float32"),
            (p + "mlp.c_fc.weight", (4 * d, d), "float32"),
            (p + "mlp.c_fc.bias", (4 * d,), "float32"),
            (p + "mlp.c_proj.weight", (d, 4 * d), "float32"),
            (p + "mlp.c_proj.bias", (d,), "float32"),
            ("decoder.output_layer.weight", (c, d), "float32")]
    return out


def _cascade_index(cfg, kind, j):
    """Module index of conv stage j inside learned_{down,up}_l1: every inner
    stage is followed by a GroupNorm when cascade_norm is on (keys doc
    section 4: down convs 0, 2, 4 and norms 1, 3, 5; up convs 0, 2, 4)."""
    return 2 * j if cfg.cascade_norm else j


class _Tok(C.Structure):
    _fields_ = [
        ("embed_dim", C.c_int64), ("in_vocab", C.c_int64), ("context_length", C.c_int64),
        ("n_levels", C.c_int32), ("groups", C.c_int32),
        ("level_len", C.c_int64 * MAX_LEVELS), ("level_vocab", C.c_int64 * MAX_LEVELS),
        ("group_eps", C.c_float), ("resi_ratio", C.c_float),
        ("learned_level0", C.c_int32), ("n_stages", C.c_int32),
        ("stage_stride", C.c_int64 * MAX_STAGES),
        ("cascade_norm", C.c_int32), ("cascade_norm_final", C.c_int32),
        ("wte", C.c_void_p), ("wpe", C.c_void_p),
        ("codebook", C.c_void_p * MAX_LEVELS),
        ("resi_weight", C.c_void_p * MAX_LEVELS), ("resi_bias", C.c_void_p * MAX_LEVELS),
        ("down_weight", C.c_void_p * MAX_STAGES), ("down_bias", C.c_void_p * MAX_STAGES),
        ("up_weight", C.c_void_p * MAX_STAGES), ("up_bias", C.c_void_p * MAX_STAGES),
    ]


class _Dec(C.Structure):
    _fields_ = [("n_head", C.c_int32), ("ln_eps", C.c_float), ("qk_eps", C.c_float)] + [
        (f, C.c_void_p) for f in (
            "ln1_weight", "ln1_bias", "attn_weight", "attn_bias", "proj_weight", "proj_bias",
            "q_norm", "k_norm", "ln2_weight", "ln2_bias", "fc_weight", "fc_bias",
            "fc_proj_weight", "fc_proj_bias", "lnf_weight", "out_weight")]


# _Dec field -> (state_dict name, shape factory of (D, hd, C))
_DEC_NAMES = {
    "ln1_weight": ("decoder.middle_block.ln_1.weight", lambda d, h, c: (d,)),
    "ln1_bias": ("decoder.middle_block.ln_1.bias", lambda d, h, c: (d,)),
    "attn_weight": ("decoder.middle_block.attn.c_attn.weight", lambda d, h, c: (3 * d, d)),
    "attn_bias": ("decoder.middle_block.attn.c_attn.bias", lambda d, h, c: (3 * d,)),
    "proj_weight": ("decoder.middle_block.attn.c_proj.weight", lambda d, h, c: (d, d)),
    "proj_bias": ("decoder.middle_block.attn.c_proj.bias", lambda d, h, c: (d,)),
    "q_norm": ("decoder.middle_block.attn.q_norm.weight", lambda d, h, c: (h,)),
    "k_norm": ("decoder.middle_block.attn.k_norm.weight", lambda d, h, c: (h,)),
    "ln2_weight": ("decoder.middle_block.ln_2.weight", lambda d, h, c: (d,)),
    "ln2_bias": ("decoder.middle_block.ln_2.bias", lambda d, h, c: (d,)),
    "fc_weight": ("decoder.middle_block.mlp.c_fc.weight", lambda d, h, c: (4 * d, d)),
    "fc_bias": ("decoder.middle_block.mlp.c_fc.bias", lambda d, h, c: (4 * d,)),
    "fc_proj_weight": ("decoder.middle_block.mlp.c_proj.weight", lambda d, h, c: (d, 4 * d)),
    "fc_proj_bias": ("decoder.middle_block.mlp.c_proj.bias", lambda d, h, c: (d,)),
    "lnf_weight": ("decoder.ln_f.weight", lambda d, h, c: (d,)),
    "out_weight": ("decoder.output_layer.weight", lambda d, h, c: (c, d)),
}


class TokenizerError(ValueError):
    """A checkpoint whose names, shapes or dtypes do not match the config."""

    def __init__(self, problems: list):
        self.problems = problems
        super().__init__("tokenizer checkpoint rejected: " + "; ".join(problems[:8]) +
                         (f" (+{len(problems) - 8} more)" if len(problems) > 8 else ""))


class Tokenizer:
    """Device weights of one tokenizer plus the C descriptor over them.

    `state` maps state_dict names to float32 device tensors (extra entries,
    such as the EMA buffers, may be absent: inference does not read them)."""

    def __init__(self, cfg: TokenizerConfig, state: dict, ctx=None):
        import torch

        cfg.validate()
        self.cfg = cfg
        self.state = state
        d = cfg.embed_dim
        dev = state["vq.embeddings.0.weight"].device
        self.device = dev
        self.ctx = ctx or default_context(dev.index or 0)
        W = "vq_tok"

        def get(name, shape):
            t = state.get(name)
            if t is None:
                raise NcmError(NCM_E_ARG, W, f"missing weight {name}")
            a = _ck.Args(W)
            a.dev(t, name, _ck.F32, shape)
            a.done()
            return t

        def pack(name, shape, k, transposed):
            src = get(name, shape)
            dst = torch.empty((d * d * k,), dtype=torch.float32, device=dev)
            self.ctx.bind_stream()
            check(lib().ncm_vq_tok_pack_conv_dev(self.ctx.handle, C.c_void_p(src.data_ptr()),
                                                 C.c_void_p(dst.data_ptr()), d, k,
                                                 1 if transposed else 0), W)
            return dst

        t = _Tok()
        t.embed_dim, t.in_vocab, t.context_length = d, cfg.in_vocab, cfg.context_length
        t.n_levels, t.groups = cfg.n_levels, cfg.groups
        t.group_eps, t.resi_ratio = cfg.group_eps, cfg.resi_ratio
        self._keep = []
        for i, (n, v) in enumerate(zip(cfg.levels, cfg.vocab_sizes)):
            t.level_len[i], t.level_vocab[i] = n, v
            t.codebook[i] = get(f"vq.embeddings.{i}.weight", (v, d)).data_ptr()
            if cfg.quant_resi:
                w = pack(f"vq.quant_resi.{i}.weight", (d, d, 3), 3, False)
                b = get(f"vq.quant_resi.{i}.bias", (d,))
                self._keep.append(w)
                t.resi_weight[i], t.resi_bias[i] = w.data_ptr(), b.data_ptr()
        strides = cfg.cascade_strides()
        t.learned_level0 = 1 if cfg.learned_level0 else 0
        t.n_stages = len(strides)
        t.cascade_norm = 1 if cfg.cascade_norm else 0
        t.cascade_norm_final = 1 if cfg.cascade_norm_final else 0
        for j, s in enumerate(strides):
            t.stage_stride[j] = s
            for kind, transposed in (("down", False), ("up", True)):
                base = f"vq.learned_{kind}_l1.{_cascade_index(cfg, kind, j)}"
                w = pack(base + ".weight", (d, d, s), s, transposed)
                b = get(base + ".bias", (d,))
                self._keep.append(w)
                getattr(t, kind + "_weight")[j] = w.data_ptr()
                getattr(t, kind + "_bias")[j] = b.data_ptr()
        if "encoder.wte.weight" in state:
            t.wte = get("encoder.wte.weight", (cfg.in_vocab, d)).data_ptr()
            t.wpe = get("encoder.wpe.weight", (cfg.context_length, d)).data_ptr()
        self.desc = t
        self.dec = None
        if "decoder.output_layer.weight" in state:
            dd = _Dec()
            dd.n_head, dd.ln_eps, dd.qk_eps = cfg.n_head, cfg.ln_eps, cfg.qk_eps
            for f, (name, shape) in _DEC_NAMES.items():
                if name in state:
                    setattr(dd, f, get(name, shape(d, d // cfg.n_head, cfg.in_vocab)).data_ptr())
            self.dec = dd

    # ---------------------------------------------------------------- calls
    def _outputs(self, B, zhat, W):
        import torch

        cfg = self.cfg
        codes = torch.empty((B, cfg.codes_per_sequence), dtype=torch.int32, device=self.device)
        if zhat is True:
            zhat = torch.empty((B, cfg.seq_len, cfg.embed_dim), dtype=torch.float32,
                               device=self.device)
        a = _ck.Args(W)
        a.dev(codes, "codes", _ck.I32, codes.shape)
        pz = a.dev(zhat, "zhat", _ck.F32, (B, cfg.seq_len, cfg.embed_dim), optional=True)
        a.done()
        return codes, zhat, pz

    def encode(self, token_ids, want_zhat=True, want_latent=False):
        """token_ids: int [B, L] (host or device; copied to the host and
        validated there). Returns dict(codes int32 [B, sum levels], zhat,
        latent)."""
        import numpy as np
        import torch

        W = "vq_tok_encode"
        cfg = self.cfg
        ids = np.ascontiguousarray(
            token_ids.detach().cpu().numpy() if hasattr(token_ids, "detach") else token_ids,
            dtype=np.int64)
        if ids.ndim != 2 or ids.shape[1] != cfg.seq_len:
            raise NcmError(NCM_E_SHAPE, W, f"token_ids must be [B, {cfg.seq_len}]")
        B = ids.shape[0]
        codes, zhat, pz = self._outputs(B, True if want_zhat else None, W)
        latent = (torch.empty((B, cfg.seq_len, cfg.embed_dim), dtype=torch.float32,
                              device=self.device) if want_latent else None)
        self.ctx.bind_stream()
        check(lib().ncm_vq_tok_encode_dev(self.ctx.handle, C.byref(self.desc),
                                          C.c_void_p(ids.ctypes.data), B,
                                          C.c_void_p(codes.data_ptr()), pz,
                                          C.c_void_p(latent.data_ptr()) if want_latent else None),
              W)
        return {"codes": codes, "zhat": zhat, "latent": latent}

    def quantize(self, latent, want_zhat=True):
        """latent: float32 device [B, L, D] (the pre-quant z)."""
        W = "vq_tok_quantize"
        cfg = self.cfg
        B, L, D = _ck.dims(latent, "latent", W, 3)
        a = _ck.Args(W)
        pl = a.dev(latent, "latent", _ck.F32, (B, cfg.seq_len, cfg.embed_dim))
        a.done()
        codes, zhat, pz = self._outputs(B, True if want_zhat else None, W)
        self.ctx.bind_stream()
        check(lib().ncm_vq_tok_quantize_dev(self.ctx.handle, C.byref(self.desc), pl, B,
                                            C.c_void_p(codes.data_ptr()), pz), W)
        return {"codes": codes, "zhat": zhat}

    def reconstruct(self, codes, zhat=None):
        """zhat = sum_l Phi_l(Up_l(e_l[codes_l])): codes int32 [B, sum levels].
        A code outside [0, V_l) of its level raises NcmError (NCM_E_ARG), as
        upstream's embedding lookup does; the check reads the codes on the
        device and synchronizes the stream (the C entry point itself only
        clamps, to stay in bounds)."""
        import torch

        W = "vq_tok_reconstruct"
        cfg = self.cfg
        B, n = _ck.dims(codes, "codes", W, 2)
        if zhat is None:
            zhat = torch.empty((B, cfg.seq_len, cfg.embed_dim), dtype=torch.float32,
                               device=self.device)
        a = _ck.Args(W)
        pc = a.dev(codes, "codes", _ck.I32, (B, cfg.codes_per_sequence))
        pz = a.dev(zhat, "zhat", _ck.F32, (B, cfg.seq_len, cfg.embed_dim))
        a.done()
        limit = self._code_limits()
        if bool(((codes < 0) | (codes >= limit[None, :])).any()):
            raise NcmError(NCM_E_ARG, W, "a code is outside [0, V) of its level")
        self.ctx.bind_stream()
        check(lib().ncm_vq_tok_reconstruct_dev(self.ctx.handle, C.byref(self.desc), pc, B, pz), W)
        return zhat


    def _code_limits(self):
        """int32 [codes_per_sequence]: V_l of each code position's level."""
        import numpy as np
        import torch

        if getattr(self, "_limits", None) is None:
            v = np.concatenate([np.full(n, vs, np.int32)
                                for n, vs in zip(self.cfg.levels, self.cfg.vocab_sizes)])
            self._limits = torch.from_numpy(v).to(self.device)
        return self._limits

    def decode(self, zhat, logits=None):
        """logits float32 [B, L, C] of the decoder block, ln_f and the output
        layer on zhat float32 [B, L, D]."""
        import torch

        W = "vq_tok_decode"
        cfg = self.cfg
        if self.dec is None:
            raise NcmError(NCM_E_ARG, W, "the tokenizer was built without decoder weights")
        B, _, _ = _ck.dims(zhat, "zhat", W, 3)
        if logits is None:
            logits = torch.empty((B, cfg.seq_len, cfg.in_vocab), dtype=torch.float32,
                                 device=self.device)
        a = _ck.Args(W)
        pz = a.dev(zhat, "zhat", _ck.F32, (B, cfg.seq_len, cfg.embed_dim))
        pl = a.dev(logits, "logits", _ck.F32, (B, cfg.seq_len, cfg.in_vocab))
        a.done()
        self.ctx.bind_stream()
        check(lib().ncm_vq_tok_decode_dev(self.ctx.handle, C.byref(self.desc), C.byref(self.dec),
                                          pz, B, pl), W)
        return logits


# ------------------------------------------------------------------ loading

def check_entries(cfg: TokenizerConfig, present: dict) -> list:
    """Problems of a checkpoint's {name: (dtype name, shape)} against the
    config's state_dict: missing and unexpected names, shapes, dtypes (the
    strict load of tokenization/vqvae_tokenizer.py:18; float entries may be
    F32, BF16 or F16, codebook_hit any integer type)."""
    want = {n: (s, d) for n, s, d in state_dict_entries(cfg)}
    problems = []
    for n in want:
        if n not in present:
            problems.append(f"missing {n}")
    for n, (dt, shape) in present.items():
        if n not in want:
            problems.append(f"unexpected {n}")
            continue
        ws, wd = want[n]
        if tuple(shape) != tuple(ws):
            problems.append(f"shape {n}: {tuple(shape)}, expected {tuple(ws)}")
        ok = ("I64", "I32") if wd == "int64" else ("F32", "BF16", "F16")
        if dt not in ok:
            problems.append(f"dtype {n}: {dt}")
    return problems


def load(path: str, cfg: TokenizerConfig = WMT14, device=None, ctx=None) -> Tokenizer:
    """Reads tokenizer.safetensors (the converter's output, ROADMAP.md:255):
    every name and shape is checked against the config before any tensor is
    read; float tensors reach the device as stored and are widened there to
    float32; the EMA buffers and hit counters are checked but not loaded."""
    import torch

    from .safetensors import SafetensorsFile

    device = torch.device(device or "cuda:0")
    with SafetensorsFile(path) as f:
        infos = {t.name: t for t in f.tensors()}
        problems = check_entries(cfg, {n: (t.dtype, t.shape) for n, t in infos.items()})
        if problems:
            raise TokenizerError(problems)
        state = {}
        tdt = {"F32": torch.float32, "BF16": torch.bfloat16, "F16": torch.float16}
        for n, t in infos.items():
            if n.startswith(("vq.ema_", "vq.codebook_hit_")):
                continue
            raw = torch.empty(tuple(t.shape), dtype=tdt[t.dtype], device=device)
            f.upload(n, raw, ctx)
            state[n] = raw if t.dtype == "F32" else raw.float()
    return Tokenizer(cfg, state, ctx)


def random_state(cfg: TokenizerConfig, device, seed: int = 0, decoder: bool = True) -> dict:
    """Random-initialised float32 device weights of every inference entry:
    N(0, 1) token, position and codebook tables (models/quant.py:299),
    uniform(+-1/sqrt(fan_in)) conv and linear weights and biases (PyTorch's
    default scale), LayerNorm / RMSNorm weights near 1."""
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    st = {}
    for name, shape, dt in state_dict_entries(cfg):
        if dt != "float32" or name.startswith("vq.ema_"):
            continue
        if name.startswith("decoder.") and not decoder:
            continue
        if name.endswith(("wte.weight", "wpe.weight")) or "embeddings" in name:
            t = torch.randn(shape, device=device, generator=g)
        elif "norm" in name or "ln_" in name:
            t = (1.0 + 0.1 * torch.randn(shape, device=device, generator=g)
                 if name.endswith("weight") else 0.1 * torch.randn(shape, device=device, generator=g))
        else:
            if "quant_resi" in name or "learned_" in name:
                fan_in = cfg.embed_dim * (3 if "quant_resi" in name else cfg.cascade_base)
            elif name.endswith(".bias"):
                fan_in = cfg.embed_dim * (4 if "mlp.c_proj" in name else 1)
            else:
                fan_in = shape[-1]
            bound = fan_in ** -0.5
            t = (torch.rand(shape, device=device, generator=g) * 2.0 - 1.0) * bound
        st[name] = t.contiguous()
    return st


def flops_per_sequence(cfg: TokenizerConfig) -> dict:
    """Algorithmic multiply-add flops (2 per MAC) of one sequence's encode:
    the nearest-code searches, the Phi convs and the level-0 cascade."""
    d, L = cfg.embed_dim, cfg.seq_len
    search = sum(2 * n * v * d for n, v in zip(cfg.levels, cfg.vocab_sizes))
    phi = 2 * L * d * 3 * d * cfg.n_levels if cfg.quant_resi else 0
    casc = 0
    length = L
    for s in cfg.cascade_strides():
        length //= s
        casc += 2 * length * s * d * d      # down stage
    casc *= 2                               # the up stages mirror them
    return {"search": search, "phi": phi, "cascade": casc, "total": search + phi + casc}
