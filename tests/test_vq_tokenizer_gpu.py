"""The VQ-VAE tokenizer on the GPU against the float64 oracle
(oracle/vq_tokenizer.py), through the C ABI (ncm_vq_tok_*).

Codes: the device searches |e|^2 - 2 u.e in float32 on the MFMA, so a code
may differ from the exact argmin only where two distances agree to float32
rounding. The oracle replays the device's codes level by level and every
used code must be within DIST_TOL of the exact minimum (relative to |u|^2 +
|e|^2, the scale of the distance), and all but a handful must be the exact
argmin. Reconstruction: within RECON_TOL of the oracle's replay (float32
sums of up to 3 D products per Phi output against float64).
"""
import dataclasses

import numpy as np
import pytest

from oracle import vq_tokenizer as vo

pytestmark = pytest.mark.gpu

DIST_TOL = 2e-5      # |d_used - d_best| <= DIST_TOL * (|u|^2 + |e_best|^2)
RECON_TOL = 2e-4     # |zhat - oracle| <= RECON_TOL * (1 + |oracle|) elementwise


def _torch():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _cascade_index(cfg, j):
    return 2 * j if cfg.cascade_norm else j


def _state(cfg, enc, qw, dec, torch, dev):
    st = {"encoder.wte.weight": enc["wte"], "encoder.wpe.weight": enc["wpe"]}
    for i, e in enumerate(qw.codebooks):
        st[f"vq.embeddings.{i}.weight"] = e
    if cfg.quant_resi:
        for i in range(cfg.n_levels):
            st[f"vq.quant_resi.{i}.weight"] = qw.resi_weight[i]
            st[f"vq.quant_resi.{i}.bias"] = qw.resi_bias[i]
    if cfg.learned_level0:
        for j in range(len(cfg.cascade_strides())):
            k = _cascade_index(cfg, j)
            st[f"vq.learned_down_l1.{k}.weight"] = qw.down_weight[j]
            st[f"vq.learned_down_l1.{k}.bias"] = qw.down_bias[j]
            st[f"vq.learned_up_l1.{k}.weight"] = qw.up_weight[j]
            st[f"vq.learned_up_l1.{k}.bias"] = qw.up_bias[j]
    for k, v in dec.items():
        st["decoder." + k] = v
    return {k: torch.from_numpy(np.ascontiguousarray(v, np.float32)).to(dev) for k, v in st.items()}


def _model(ocfg, seed, cb_scale=0.3, vocab_cap=None):
    torch = _torch()
    from ncmorph_amd import vq_tokenizer as vt

    enc, qw, dec = vo.random_weights(ocfg, seed=seed, vocab_cap=vocab_cap)
    qw.codebooks = [(c * cb_scale).astype(np.float32) for c in qw.codebooks]
    pcfg = vt.TokenizerConfig(**dataclasses.asdict(ocfg))
    if vocab_cap is not None:
        pcfg.in_vocab = enc["wte"].shape[0]
        ocfg = dataclasses.replace(ocfg, in_vocab=enc["wte"].shape[0])
    tok = vt.Tokenizer(pcfg, _state(ocfg, enc, qw, dec, torch, "cuda:0"))
    return ocfg, enc, qw, dec, tok


def _check_codes(ocfg, qw, z, codes, zhat=None, min_exact=0.995):
    """Replay the device codes in the oracle; returns the oracle result."""
    ref = vo.quantize(ocfg, qw, z, forced=codes)
    exact = total = 0
    r = np.asarray(z, np.float64).copy()
    for level in range(ocfg.n_levels):
        du, db = ref["d_used"][level], ref["d_best"][level]
        u = vo._down(ocfg, qw, level, r)
        e = np.asarray(qw.codebooks[level], np.float64)
        scale = (u * u).sum(-1) + (e * e).sum(-1).max()
        assert (du - db <= DIST_TOL * scale).all(), (level, float((du - db).max()))
        exact += int((du == db).sum())
        total += du.size
        off = sum(ocfg.levels[:level])
        idx = codes[:, off:off + ocfg.levels[level]]
        r = r - vo._resi(ocfg, qw, level, vo._up(ocfg, qw, level, e[idx]))
    assert exact >= min_exact * total, (exact, total)
    if zhat is not None:
        err = np.abs(zhat - ref["zhat"]) / (1.0 + np.abs(ref["zhat"]))
        assert err.max() <= RECON_TOL, float(err.max())
    return ref


SMALL_WMT = vo.TokenizerConfig(in_vocab=1000, vocab_sizes=(512,) * 11)


@pytest.mark.parametrize("ocfg,batch", [
    (SMALL_WMT, 3),
    # the OWT arrangement (no cascade norms), a shorter sequence: 4 stages
    (vo.TokenizerConfig(embed_dim=64, in_vocab=300, context_length=256,
                        levels=(1, 4, 9, 16, 25, 49, 100, 256), vocab_sizes=(64, 128, 96, 64,
                                                                               200, 128, 64, 256),
                        cascade_norm=False, cascade_norm_final=False, n_head=2), 2),
    # level 0 pooled like the others, no Phi, D not a multiple of the tile
    (vo.TokenizerConfig(embed_dim=96, in_vocab=50, context_length=24, levels=(1, 3, 7, 16),
                        vocab_sizes=(40, 300, 33, 129), groups=4, learned_level0=False,
                        quant_resi=False, n_head=3), 5),
    # norms between stages but none after the last, an odd code count
    (vo.TokenizerConfig(embed_dim=32, in_vocab=64, context_length=16, levels=(1, 2, 5, 16),
                        vocab_sizes=(17, 31, 65, 129), groups=2, cascade_norm=True,
                        cascade_norm_final=False, n_head=2), 4),
])
def test_encode_matches_oracle(ocfg, batch):
    torch = _torch()
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=batch)
    rng = np.random.default_rng(batch)
    ids = rng.integers(0, ocfg.in_vocab, size=(batch, ocfg.seq_len))
    print(f"vq_tok encode B={batch} L={ocfg.seq_len} D={ocfg.embed_dim}", flush=True)
    out = tok.encode(ids, want_zhat=True, want_latent=True)
    torch.cuda.synchronize()
    z_ref = vo.encode_front(ocfg, ids, enc["wte"], enc["wpe"])
    z = out["latent"].cpu().numpy()
    np.testing.assert_allclose(z, z_ref, rtol=1e-4, atol=1e-4)
    codes = out["codes"].cpu().numpy()
    assert codes.shape == (batch, sum(ocfg.levels))
    _check_codes(ocfg, qw, z_ref, codes, out["zhat"].cpu().numpy())
    # quantize from the device latent and reconstruct from the codes run the
    # same kernels in the same order: identical bits
    q = tok.quantize(out["latent"])
    assert torch.equal(q["codes"], out["codes"])
    assert torch.equal(q["zhat"], out["zhat"])
    rec = tok.reconstruct(out["codes"])
    assert torch.equal(rec, out["zhat"])


def test_planted_codes_single_level():
    torch = _torch()
    ocfg = vo.TokenizerConfig(embed_dim=64, in_vocab=10, context_length=32, levels=(32,),
                              vocab_sizes=(300,), learned_level0=False, quant_resi=False,
                              n_head=2)
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=1, cb_scale=1.0)
    rng = np.random.default_rng(3)
    want = rng.integers(0, 300, size=(6, 32))
    z = torch.from_numpy(qw.codebooks[0][want]).cuda()
    out = tok.quantize(z)
    assert np.array_equal(out["codes"].cpu().numpy(), want)
    assert torch.equal(out["zhat"], z)


def test_ties_take_the_lowest_index():
    torch = _torch()
    ocfg = vo.TokenizerConfig(embed_dim=32, in_vocab=10, context_length=8, levels=(8,),
                              vocab_sizes=(200,), groups=2, learned_level0=False,
                              quant_resi=False, n_head=2)
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=2, cb_scale=1.0)
    # duplicate rows: codes 7 and 150 equal, 20 and 199 equal
    cb = tok.state["vq.embeddings.0.weight"]
    cb[150] = cb[7]
    cb[199] = cb[20]
    z = torch.stack([cb[7], cb[20]] * 4).reshape(1, 8, 32).contiguous()
    out = tok.quantize(z)
    assert out["codes"].cpu().numpy().tolist() == [[7, 20] * 4]


def test_reconstruct_rejects_out_of_range_codes():
    """A caller code outside [0, V) of its level is refused (NCM_E_ARG), as
    upstream's embedding lookup raises; codes at both ends of the range are
    accepted."""
    torch = _torch()
    from ncmorph_amd._lib import NCM_E_ARG, NcmError

    ocfg, enc, qw, dec, tok = _model(SMALL_WMT, seed=4)
    codes = torch.randint(0, 512, (2, sum(SMALL_WMT.levels)), dtype=torch.int32, device="cuda")
    edge = codes.clone()
    edge[:, 0] = 0
    edge[:, 7] = 511
    tok.reconstruct(edge)
    for pos, val in ((0, -5), (7, 512), (7, 10 ** 6)):
        bad = codes.clone()
        bad[1, pos] = val
        with pytest.raises(NcmError) as e:
            tok.reconstruct(bad)
        assert e.value.status == NCM_E_ARG


def test_encode_rejects_out_of_range_ids():
    _torch()
    from ncmorph_amd._lib import NcmError

    ocfg, enc, qw, dec, tok = _model(SMALL_WMT, seed=5)
    ids = np.zeros((1, 64), dtype=np.int64)
    ids[0, 5] = SMALL_WMT.in_vocab
    with pytest.raises(NcmError):
        tok.encode(ids)


def test_wmt14_full_size_properties():
    """The released tokenizer's shapes (D 384, 11 levels of 4096 codes,
    151680 token rows) on 64 sequences: an oracle replay of 4 of them,
    determinism, and the reconstruction identity."""
    torch = _torch()
    ocfg = vo.WMT14
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=11)
    rng = np.random.default_rng(11)
    ids = rng.integers(0, ocfg.in_vocab, size=(64, 64))
    print("vq_tok WMT14 B=64", flush=True)
    a = tok.encode(ids, want_latent=True)
    b = tok.encode(ids)
    torch.cuda.synchronize()
    assert torch.equal(a["codes"], b["codes"]) and torch.equal(a["zhat"], b["zhat"])
    codes = a["codes"].cpu().numpy()
    off = 0
    for n, v in zip(ocfg.levels, ocfg.vocab_sizes):
        blk = codes[:, off:off + n]
        assert blk.min() >= 0 and blk.max() < v
        off += n
    assert len(np.unique(codes[:, -64:])) > 500
    z = a["latent"][:4].cpu().numpy().astype(np.float64)
    _check_codes(ocfg, qw, z, codes[:4], a["zhat"][:4].cpu().numpy())
    assert torch.equal(tok.reconstruct(a["codes"]), a["zhat"])


@pytest.mark.parametrize("ocfg,batch", [
    (SMALL_WMT, 2),
    (vo.TokenizerConfig(embed_dim=96, in_vocab=52, context_length=24, levels=(1, 3, 7, 16),
                        vocab_sizes=(40, 300, 33, 129), groups=4, learned_level0=False,
                        n_head=3), 3),
])
def test_decoder_matches_oracle(ocfg, batch):
    torch = _torch()
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=21)
    rng = np.random.default_rng(21)
    zhat = rng.standard_normal((batch, ocfg.seq_len, ocfg.embed_dim)).astype(np.float32)
    print(f"vq_tok decode B={batch} D={ocfg.embed_dim}", flush=True)
    logits = tok.decode(torch.from_numpy(zhat).cuda()).cpu().numpy()
    want = vo.decoder_forward(ocfg, dec, zhat)
    np.testing.assert_allclose(logits, want, rtol=1e-4, atol=1e-4)


def test_codes_to_logits_full_wmt14_vocab():
    """Codes -> reconstruction -> logits over the full 151680-token output
    layer for two sequences, against the oracle on the device's zhat."""
    torch = _torch()
    ocfg, enc, qw, dec, tok = _model(vo.WMT14, seed=12)
    rng = np.random.default_rng(12)
    ids = rng.integers(0, ocfg.in_vocab, size=(2, 64))
    out = tok.encode(ids)
    zhat = tok.reconstruct(out["codes"])
    logits = tok.decode(zhat)
    torch.cuda.synchronize()
    want = vo.decoder_forward(ocfg, dec, zhat.cpu().numpy())
    np.testing.assert_allclose(logits.cpu().numpy(), want, rtol=1e-4, atol=1e-4)


def test_load_round_trip(tmp_path):
    """A checkpoint with every state_dict entry (float tensors stored F32,
    codebooks BF16, hit counters I64) loads and encodes exactly as the
    tokenizer built from the same values."""
    torch = _torch()
    from ncmorph_amd import vq_tokenizer as vt
    from ncmorph_amd.safetensors import write_file

    ocfg = vo.TokenizerConfig(embed_dim=64, in_vocab=40, context_length=32,
                              levels=(2, 8, 16, 32), vocab_sizes=(16, 64, 32, 128), n_head=2)
    _, enc, qw, dec, tok = _model(ocfg, seed=8)
    pcfg = tok.cfg
    tensors = {}
    for name, shape, dt in vt.state_dict_entries(pcfg):
        if dt == "int64":
            tensors[name] = ("I64", shape, np.zeros(shape, np.int64).tobytes())
        elif name.startswith("vq.ema_"):
            tensors[name] = ("F32", shape, np.zeros(shape, np.float32).tobytes())
        elif name.startswith("vq.embeddings."):
            bits = tok.state[name].cpu().numpy().view(np.uint32)
            # round to bf16 (values chosen to be bf16 already: truncate then
            # compare against the same truncation on the device tokenizer)
            b16 = (bits >> 16).astype(np.uint16)
            tok.state[name].copy_(torch.from_numpy((b16.astype(np.uint32) << 16).view(np.float32)))
            tensors[name] = ("BF16", shape, b16.tobytes())
        else:
            tensors[name] = ("F32", shape, tok.state[name].cpu().numpy().tobytes())
    path = tmp_path / "tokenizer.safetensors"
    write_file(str(path), tensors)
    loaded = vt.load(str(path), pcfg, device="cuda:0")
    ids = np.random.default_rng(0).integers(0, 40, size=(3, 32))
    a = tok.encode(ids)
    b = loaded.encode(ids)
    assert torch.equal(a["codes"], b["codes"]) and torch.equal(a["zhat"], b["zhat"])
    assert torch.equal(tok.decode(a["zhat"]), loaded.decode(b["zhat"]))


def test_owt_full_size_replay():
    """The OWT tokenizer of vq_forward_semantics.md section 1 at its full
    shapes (1024 positions, 32 levels of (k + 1)^2 positions, 8192 codes, a
    five-stage cascade without norms) on one sequence: the oracle replay of
    every level and the reconstruction identity."""
    torch = _torch()
    ocfg = dataclasses.replace(vo.OWT, in_vocab=512)
    ocfg, enc, qw, dec, tok = _model(ocfg, seed=13)
    rng = np.random.default_rng(13)
    ids = rng.integers(0, ocfg.in_vocab, size=(1, 1024))
    print("vq_tok OWT B=1", flush=True)
    out = tok.encode(ids, want_latent=True)
    torch.cuda.synchronize()
    z = out["latent"].cpu().numpy().astype(np.float64)
    _check_codes(ocfg, qw, z, out["codes"].cpu().numpy(), out["zhat"].cpu().numpy())
    assert torch.equal(tok.reconstruct(out["codes"]), out["zhat"])
