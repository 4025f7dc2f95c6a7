"""GPU parity of the NCM codebook-tied head (ncm_tied_head_logits) against
the oracle's f64 statement of it (PROJECT.md:222; no reference code exists,
so the formula is pinned by tests/test_oracle_tied_head.py).

Bound: every logit within scale * ((d + 4) 2^-24 sum|2 z_i E_ki| + d 2^-24 E_sq
+ 2^-22 |2S - E_sq|) + 2^-21 (|logit| + |bias|) of the f64 value (fp32
accumulation of d exact products, E_sq's own fp32 sum, the subtraction, the
scale's rounding, the scaling and the bias add), scale = exp(log_inv_T) / mean
E_sq.
The argmax of every row with a clear top-2 gap is the RVQ encode's code (the
exact nearest code) computed by the same library."""
import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu


def _bf16_dev(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


@pytest.mark.parametrize("rows,d,v,log_inv_t,bias,check_rows", [
    (512, 4096, 8192, 0.0, False, 64),      # one level of the 8B step (128 x 128 tiles)
    (2048, 512, 8192, 0.7, True, 256),      # 256 x 256 tiles
    (300, 200, 1000, -0.3, True, 300),      # ragged tiles, d not a multiple of 64
    (1, 8, 1, 0.0, False, 1),               # one code
])
def test_tied_head_against_oracle(ncm, oracle, cuda, rows, d, v, log_inv_t, bias, check_rows):
    import torch
    from ncmorph_amd import kernels, vq

    rng = np.random.default_rng(rows + d + v)
    zb = synth.bf16_bits(rng.standard_normal((rows, d)).astype(np.float32))
    eb = synth.bf16_bits((rng.standard_normal((v, d)) / np.sqrt(d)).astype(np.float32))
    bf = rng.standard_normal(v).astype(np.float32) if bias else None
    zd, ed = _bf16_dev(zb, cuda), _bf16_dev(eb, cuda)
    csq = vq.prepare(ed.view(1, v, d))[0]
    bd = torch.from_numpy(bf).to(cuda) if bias else None
    got = kernels.tied_head_logits(zd, ed, csq, log_inv_t, bias=bd)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    sel = np.sort(rng.choice(rows, size=check_rows, replace=False))
    z = synth.bf16_to_f32(zb)[sel]
    E = synth.bf16_to_f32(eb)
    ref, mag = oracle.tied_head_logits_f64(z, E, log_inv_t, bf)
    esq = np.sum(E.astype(np.float64) ** 2, axis=1)
    scale = np.exp(log_inv_t) / esq.mean()
    t = np.abs(ref - (bf if bias else 0)) / scale
    babs = np.abs(bf.astype(np.float64)) if bias else 0.0
    bound = (scale * ((d + 4) * 2.0**-24 * mag + d * 2.0**-24 * esq[None, :] + 2.0**-22 * t)
             + 2.0**-21 * (np.abs(ref) + babs) + 1e-30)
    err = np.abs(got[sel].astype(np.float64) - ref)
    assert np.all(err <= bound), float(np.max(err / bound))
    if v > 1 and not bias:
        # argmax = the exact nearest code (single-level RVQ encode of z).
        r = vq.encode(zd.float().view(1, rows, d), ed.view(1, v, d), (1,), csq=csq.view(1, v),
                      want_gap=True)
        codes = r["codes"].cpu().numpy()[0]
        gap = r["gap"].cpu().numpy()[0]
        clear = gap > 1e-4
        assert np.array_equal(np.argmax(got, axis=1)[clear], codes[clear])


def test_tied_head_rejects_bad_arguments(ncm, cuda):
    import torch
    from ncmorph_amd import kernels
    from ncmorph_amd._lib import NcmError

    z = torch.zeros((4, 12), dtype=torch.bfloat16, device=cuda)   # d % 8 != 0
    e = torch.zeros((6, 12), dtype=torch.bfloat16, device=cuda)
    c = torch.ones(6, device=cuda)
    with pytest.raises(NcmError):
        kernels.tied_head_logits(z, e, c)


def test_tied_head_levels_one_launch(ncm, oracle, cuda):
    """Several levels in one launch (ragged row counts, an empty level, a
    scale and a bias per level): each level block against the oracle with the
    level's own codebook, norms, bias and scale."""
    import torch
    from ncmorph_amd import kernels, vq

    rng = np.random.default_rng(123)
    d, v = 256, 1000
    level_rows = [40, 0, 300, 129]
    lit = [0.0, 1.0, -0.5, 0.25]
    L = len(level_rows)
    zb = synth.bf16_bits(rng.standard_normal((sum(level_rows), d)).astype(np.float32))
    eb = synth.bf16_bits((rng.standard_normal((L, v, d)) / np.sqrt(d)).astype(np.float32))
    bf = rng.standard_normal((L, v)).astype(np.float32)
    zd, ed = _bf16_dev(zb, cuda), _bf16_dev(eb, cuda)
    csq = vq.prepare(ed)
    got = kernels.tied_head_logits_levels(zd, ed, csq, level_rows, lit,
                                          bias=torch.from_numpy(bf).to(cuda))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    off = 0
    for l, n in enumerate(level_rows):
        if n:
            z = synth.bf16_to_f32(zb[off:off + n])
            E = synth.bf16_to_f32(eb[l])
            ref, mag = oracle.tied_head_logits_f64(z, E, lit[l], bf[l])
            esq = np.sum(E.astype(np.float64) ** 2, axis=1)
            scale = np.exp(lit[l]) / esq.mean()
            t = np.abs(ref - bf[l]) / scale
            bound = (scale * ((d + 4) * 2.0**-24 * mag + d * 2.0**-24 * esq[None, :]
                              + 2.0**-22 * t) + 2.0**-21 * (np.abs(ref) + np.abs(bf[l])) + 1e-30)
            err = np.abs(got[off:off + n].astype(np.float64) - ref)
            assert np.all(err <= bound), (l, float(np.max(err / bound)))
        off += n


def test_tied_head_levels_split_launch(ncm, oracle, cuda):
    """The NCM layout's growing levels (32 ... 1024 rows, 8192 codes): the
    levels below 256 rows run as a launch of 128 x 128 tiles of their own
    (their 256 x 256 tiles would add a round), the rest on 256 x 256 tiles;
    sampled rows of every level against the oracle's bound, and the argmax of
    rows with a clear top-2 gap against the exact nearest code."""
    import torch
    from ncmorph_amd import kernels, vq

    rng = np.random.default_rng(321)
    d, v = 512, 8192
    level_rows = [32, 64, 128, 256, 512, 1024]
    lit = [0.1 * l for l in range(len(level_rows))]
    L = len(level_rows)
    zb = synth.bf16_bits(rng.standard_normal((sum(level_rows), d)).astype(np.float32))
    eb = synth.bf16_bits((rng.standard_normal((L, v, d)) / np.sqrt(d)).astype(np.float32))
    zd, ed = _bf16_dev(zb, cuda), _bf16_dev(eb, cuda)
    csq = vq.prepare(ed)
    got = kernels.tied_head_logits_levels(zd, ed, csq, level_rows, lit)
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    off = 0
    for l, n in enumerate(level_rows):
        sel = off + np.sort(rng.choice(n, size=min(n, 24), replace=False))
        z = synth.bf16_to_f32(zb[sel])
        E = synth.bf16_to_f32(eb[l])
        ref, mag = oracle.tied_head_logits_f64(z, E, lit[l], None)
        esq = np.sum(E.astype(np.float64) ** 2, axis=1)
        scale = np.exp(lit[l]) / esq.mean()
        t = np.abs(ref) / scale
        bound = (scale * ((d + 4) * 2.0**-24 * mag + d * 2.0**-24 * esq[None, :] + 2.0**-22 * t)
                 + 2.0**-21 * np.abs(ref) + 1e-30)
        err = np.abs(got[sel].astype(np.float64) - ref)
        assert np.all(err <= bound), (l, float(np.max(err / bound)))
        r = vq.encode(zd[off:off + n].float().view(1, n, d), ed[l].view(1, v, d), (1,),
                      csq=csq[l].view(1, v), want_gap=True)
        codes = r["codes"].cpu().numpy()[0]
        clear = r["gap"].cpu().numpy()[0] > 1e-4
        assert np.array_equal(np.argmax(got[off:off + n], axis=1)[clear], codes[clear]), l
        off += n


def test_tied_head_levels_full_8b_layout(ncm, oracle, cuda):
    """The NCM step's whole head launch: 8 levels of 32 ... 4096 rows (8160),
    z and codebooks of width 4096, 8192 codes per level, a scale and a bias
    per level. 16 sampled rows of every level against the oracle's f64 head
    within the bound above, and the argmax of every row of the level with a
    clear top-2 gap against the exact nearest code."""
    import torch
    from ncmorph_amd import kernels, vq

    rng = np.random.default_rng(8192)
    d, v = 4096, 8192
    level_rows = [32, 64, 128, 256, 512, 1024, 2048, 4096]
    lit = [0.05 * l - 0.1 for l in range(len(level_rows))]
    L = len(level_rows)
    zb = synth.bf16_bits(rng.standard_normal((sum(level_rows), d), dtype=np.float32))
    eb = synth.bf16_bits((rng.standard_normal((L, v, d), dtype=np.float32) /
                          np.float32(np.sqrt(d))))
    bf = (rng.standard_normal((L, v), dtype=np.float32) * np.float32(0.1))
    zd, ed = _bf16_dev(zb, cuda), _bf16_dev(eb, cuda)
    csq = vq.prepare(ed)
    got = kernels.tied_head_logits_levels(zd, ed, csq, level_rows, lit,
                                          bias=torch.from_numpy(bf).to(cuda))
    torch.cuda.synchronize()
    off = 0
    for l, n in enumerate(level_rows):
        print(f"level {l}: {n} rows", flush=True)
        sel = off + np.sort(rng.choice(n, size=min(n, 16), replace=False))
        z = synth.bf16_to_f32(zb[sel])
        E = synth.bf16_to_f32(eb[l])
        ref, mag = oracle.tied_head_logits_f64(z, E, lit[l], bf[l])
        esq = np.sum(E.astype(np.float64) ** 2, axis=1)
        scale = np.exp(lit[l]) / esq.mean()
        t = np.abs(ref - bf[l]) / scale
        bound = (scale * ((d + 4) * 2.0**-24 * mag + d * 2.0**-24 * esq[None, :] + 2.0**-22 * t)
                 + 2.0**-21 * (np.abs(ref) + np.abs(bf[l])) + 1e-30)
        gl = got[off:off + n]
        err = np.abs(gl[torch.from_numpy(sel - off).to(cuda)].cpu().numpy().astype(np.float64)
                     - ref)
        assert np.all(err <= bound), (l, float(np.max(err / bound)))
        # Without the bias the argmax is the exact nearest code; with it, the
        # argmax of (logit - bias) is.
        r = vq.encode(zd[off:off + n].float().view(1, n, d), ed[l].view(1, v, d), (1,),
                      csq=csq[l].view(1, v), want_gap=True)
        codes = r["codes"].cpu().numpy()[0]
        clear = r["gap"].cpu().numpy()[0] > 1e-4
        unb = (gl - torch.from_numpy(bf[l]).to(cuda)[None, :]).argmax(dim=1).cpu().numpy()
        assert np.array_equal(unb[clear], codes[clear]), l
        off += n
