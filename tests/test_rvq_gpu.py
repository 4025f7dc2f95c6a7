"""GPU parity of the multiscale RVQ encode / decode against the oracle.

Bar: codes bit-identical to the oracle (its fp32 order is reproduced
exactly, so no near-tie exemption is needed; near-ties are still counted and
reported), reconstruction bit-identical, csq bit-identical. At the full
configuration (16 x 2048 x 2048, 8 levels, 4096 codes) the oracle re-derives
sampled rows of every level from the GPU's earlier-level codes (teacher
forcing) and must choose the same code.
"""
import os

import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rvq_small.npz")


def _dev(a, cuda, bf16=False):
    import torch

    if bf16:
        return torch.from_numpy(a.view(np.int16).copy()).to(cuda).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(cuda)


def _encode(x, cb, strides, cuda, force=None, count=True):
    import torch
    from ncmorph_amd import vq

    xd = _dev(x, cuda)
    cbd = _dev(cb, cuda, bf16=True)
    fd = None if force is None else _dev(force.astype(np.int32), cuda)
    r = vq.encode(xd, cbd, strides, force_codes=fd, count_flagged=count)
    torch.cuda.synchronize()
    return {k: (v.cpu().numpy() if hasattr(v, "cpu") else v) for k, v in r.items()}


def test_csq_bit_exact(ncm, oracle, cuda):
    import torch
    from ncmorph_amd import vq

    rng = np.random.default_rng(0)
    for L, V, d in [(2, 37, 64), (1, 512, 256), (3, 100, 320), (1, 64, 2048)]:
        cb = synth.bf16_bits((rng.standard_normal((L, V, d)) / np.sqrt(d)).astype(np.float32))
        got = vq.prepare(_dev(cb, cuda, bf16=True))
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy(), oracle.rvq_csq(cb)), (L, V, d)


def test_small_config_golden(ncm, oracle, cuda):
    c = synth.RVQ_SMALL
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    g = np.load(GOLDEN)
    r = _encode(x, cb, c["strides"], cuda)
    assert np.array_equal(r["codes"].reshape(4, 128), g["codes"])
    ref = oracle.rvq_encode(x, cb, c["strides"])
    assert np.array_equal(r["recon"], ref["recon"])
    finite = np.isfinite(ref["gap"]) & (ref["gap"] < 1e-4)
    assert np.allclose(r["gap"][finite], ref["gap"][finite], rtol=1e-3, atol=1e-9)
    # GPU gap is +inf only where the oracle's gap is not a near-tie.
    assert np.all(ref["gap"][~np.isfinite(r["gap"])] >= 1e-5)


@pytest.mark.parametrize("case", [
    dict(b=2, t=256, d=256, v=512, strides=(128, 64, 32, 16, 8, 4, 2, 1), seed=21),
    dict(b=3, t=64, d=320, v=300, strides=(16, 16, 4, 1), seed=22),
    dict(b=1, t=32, d=64, v=7, strides=(8, 2, 1), seed=23),
    dict(b=2, t=128, d=2048, v=1000, strides=(32, 8, 1), seed=24),
    # 1024 rows on 128 x 128 tiles, then 2048 rows on 256 x 128 tiles
    dict(b=1, t=2048, d=64, v=4096, strides=(2, 1), seed=25),
    # 8192 rows at the finest level, few codes (four code ranges per tile row)
    dict(b=2, t=4096, d=64, v=512, strides=(16, 4, 1), seed=26),
    # 5000 codes: more code tiles than ranges, so workgroups loop over two
    # tiles (the last one ragged), on 128 x 128 tiles (1024 rows) and on
    # 256 x 128 tiles (4096 rows)
    dict(b=1, t=4096, d=64, v=5000, strides=(4, 1), seed=27),
    # 256 x 256 tiles (8192 rows) with two code tiles per workgroup
    # (32x32x16 MFMAs, per-row state kept across the tiles)
    dict(b=2, t=4096, d=64, v=5000, strides=(1,), seed=28),
    # 256 x 256 tiles with one code tile per workgroup (16x16x32 MFMAs), the
    # last code tile ragged (4000 = 15 * 256 + 160)
    dict(b=2, t=4096, d=64, v=4000, strides=(2, 1), seed=29),
    # 256 x 256 tiles, one code tile per workgroup, three rounds of the CUs
    # (768 tiles)
    dict(b=3, t=4096, d=128, v=4096, strides=(4, 1), seed=30),
    # 756 tiles (not a multiple of the 8 XCDs, so the tile order is not
    # remapped), ragged last row tile, 12 code tiles with the last one ragged
    dict(b=1, t=16000, d=64, v=3000, strides=(1,), seed=36),
    # the widest rows (16 register chunks): 4096 rows keep D in registers,
    # then 8192 rows load it again for each use
    dict(b=1, t=8192, d=4096, v=300, strides=(2, 1), seed=37),
    # 16 chunks, the last ones partly or wholly past the row (2112 = 8.25 x 256)
    dict(b=1, t=8192, d=2112, v=64, strides=(1,), seed=38),
    # a single code per level: every code is 0
    dict(b=2, t=64, d=128, v=1, strides=(4, 1), seed=39),
    # the most levels (32)
    dict(b=1, t=64, d=64, v=16, strides=(32, 16, 8, 4, 2) + (1,) * 27, seed=40),
])
def test_multiscale_matches_oracle(ncm, oracle, cuda, case):
    L = len(case["strides"])
    x, cb = synth.rvq_inputs(case["seed"], case["b"], case["t"], case["d"], L, case["v"])
    r = _encode(x, cb, case["strides"], cuda)
    ref = oracle.rvq_encode(x, cb, case["strides"], threads=8)
    assert np.array_equal(r["codes"], ref["codes"]), np.sum(r["codes"] != ref["codes"])
    assert np.array_equal(r["recon"], ref["recon"])
    print("flagged rows:", r["n_flagged"])


@pytest.mark.parametrize("case", [
    dict(b=2, t=256, d=256, v=512, strides=(128, 64, 32, 16, 8, 4, 2, 1), seed=21),
    dict(b=2, t=4096, d=64, v=4000, strides=(2, 1), seed=29),
    dict(b=3, t=4096, d=128, v=4096, strides=(4, 1), seed=30),
])
def test_encode_without_gaps_matches_oracle(ncm, oracle, cuda, case):
    """An encode that reports no gaps has no near-tie margin in its candidate
    window (only the rigorous error bound): codes and reconstruction are the
    oracle's and the gap-reporting encode's, bit for bit."""
    import torch
    from ncmorph_amd import vq

    L = len(case["strides"])
    x, cb = synth.rvq_inputs(case["seed"], case["b"], case["t"], case["d"], L, case["v"])
    xd, cbd = _dev(x, cuda), _dev(cb, cuda, bf16=True)
    with_gap = vq.encode(xd, cbd, case["strides"], want_gap=True)
    no_gap = vq.encode(xd, cbd, case["strides"], want_gap=False)
    torch.cuda.synchronize()
    ref = oracle.rvq_encode(x, cb, case["strides"], threads=8)
    assert "gap" not in no_gap or no_gap["gap"] is None
    assert np.array_equal(no_gap["codes"].cpu().numpy(), ref["codes"])
    assert np.array_equal(no_gap["recon"].cpu().numpy(), ref["recon"])
    assert torch.equal(no_gap["codes"], with_gap["codes"])
    assert torch.equal(no_gap["recon"].view(torch.int32), with_gap["recon"].view(torch.int32))


def test_duplicate_codewords_without_gaps(ncm, oracle, cuda):
    """Exact ties (identical codewords) with no near-tie margin: still the
    lowest index."""
    import torch
    from ncmorph_amd import vq

    d, V = 256, 300
    x, cb = synth.rvq_inputs(31, 1, 64, d, 2, V)
    for l in range(2):
        for k in range(5, V, 7):
            cb[l, k] = cb[l, 3]
    x[0, :8] = synth.bf16_to_f32(cb[0, 3])
    r = vq.encode(_dev(x, cuda), _dev(cb, cuda, bf16=True), (4, 1), want_gap=False)
    torch.cuda.synchronize()
    ref = oracle.rvq_encode(x, cb, (4, 1))
    assert np.array_equal(r["codes"].cpu().numpy(), ref["codes"])


def test_duplicate_codewords_take_lowest_index(ncm, oracle, cuda):
    # Identical codewords tie exactly; the flagged path (every code of an
    # incomplete group rescored) must still return the lowest index, as the
    # oracle does.
    rng = np.random.default_rng(31)
    d, V = 256, 300
    x, cb = synth.rvq_inputs(31, 1, 64, d, 2, V)
    for l in range(2):
        for k in range(5, V, 7):
            cb[l, k] = cb[l, 3]
    x[0, :8] = synth.bf16_to_f32(cb[0, 3])
    r = _encode(x, cb, (4, 1), cuda)
    ref = oracle.rvq_encode(x, cb, (4, 1))
    assert np.array_equal(r["codes"], ref["codes"])
    assert r["n_flagged"] >= 1


def test_all_equal_codebook_rescores_every_code(ncm, oracle, cuda):
    d, V = 128, 600
    x, cb = synth.rvq_inputs(32, 1, 16, d, 1, V)
    cb[0, :] = cb[0, 0]
    r = _encode(x, cb, (1,), cuda)
    assert np.all(r["codes"] == 0)
    assert r["n_flagged"] == 16


def test_teacher_forcing(ncm, oracle, cuda):
    strides = (16, 4, 1)
    x, cb = synth.rvq_inputs(33, 2, 64, 256, 3, 256)
    ref = oracle.rvq_encode(x, cb, strides)
    forced = ref["codes"].copy()
    rng = np.random.default_rng(33)
    flip = rng.random(forced.shape) < 0.3
    forced[flip] = rng.integers(0, 256, size=int(flip.sum()))
    want = oracle.rvq_encode(x, cb, strides, forced=forced)
    r = _encode(x, cb, strides, cuda, force=forced)
    assert np.array_equal(r["codes"], want["codes"])
    assert np.array_equal(r["recon"], want["recon"])


def test_level_counts(ncm, oracle, cuda):
    """ncm_rvq_encode_counts: the same codes, reconstruction and gaps as the
    plain encode; per level, the rows with an exact rescore include every
    row whose gap is finite (two or more exact distances) and never exceed
    the level's rows; an all-equal codebook makes every row rescored."""
    import torch
    from ncmorph_amd import vq

    strides = (8, 2, 1)
    x, cb = synth.rvq_inputs(11, 2, 64, 256, 3, 96)
    xd, cbd = _dev(x, cuda), _dev(cb, cuda, bf16=True)
    plain = vq.encode(xd, cbd, strides, count_flagged=True)
    cnt = vq.encode(xd, cbd, strides, level_counts=True)
    torch.cuda.synchronize()
    for k in ("codes", "recon", "gap"):
        assert torch.equal(plain[k], cnt[k]), k
    assert cnt["n_flagged"] == plain["n_flagged"] == sum(cnt["flagged"])
    gap = cnt["gap"].cpu().numpy()
    off = 0
    for l, s in enumerate(strides):
        n = 2 * (64 // s)
        finite = int(np.isfinite(gap[:, off:off + 64 // s]).sum())
        assert finite <= cnt["scored"][l] <= n, (l, finite, cnt["scored"][l])
        off += 64 // s
    same = np.repeat(cb[:, :1], cb.shape[1], axis=1)
    eq = vq.encode(xd, _dev(same, cuda, bf16=True), strides, level_counts=True)
    torch.cuda.synchronize()
    assert eq["scored"] == [2 * (64 // s) for s in strides]
    assert np.array_equal(eq["codes"].cpu().numpy(), oracle.rvq_encode(x, same, strides)["codes"])


def test_decode_matches_oracle(ncm, oracle, cuda):
    import torch
    from ncmorph_amd import vq

    strides = (8, 2, 1)
    x, cb = synth.rvq_inputs(34, 2, 32, 256, 3, 64)
    rng = np.random.default_rng(34)
    codes = rng.integers(0, 64, size=(2, 4 + 16 + 32)).astype(np.int32)
    got = vq.decode(_dev(codes, cuda), _dev(cb, cuda, bf16=True), strides, 32)
    torch.cuda.synchronize()
    assert np.array_equal(got.cpu().numpy(), oracle.rvq_decode(codes, cb, strides, 32))


def test_large_config_properties(ncm, oracle, cuda):
    """16 x 2048 x 2048, 8 levels, 4096 codes: codes in range, decode equals
    the encode's reconstruction, sampled rows of every level agree with the
    oracle's exhaustive search given the GPU's earlier codes, and sequence 0
    (every level, 4080 codes, and its reconstruction) equals the oracle's
    own encode bit for bit."""
    import torch
    from ncmorph_amd import vq

    c = synth.RVQ_LARGE
    x, cb = synth.rvq_inputs(c["seed"], c["b"], c["t"], c["d"], c["levels"], c["v"])
    xd = _dev(x, cuda)
    cbd = _dev(cb, cuda, bf16=True)
    r = vq.encode(xd, cbd, c["strides"], count_flagged=True)
    rec = vq.decode(r["codes"], cbd, c["strides"], c["t"])
    torch.cuda.synchronize()
    codes = r["codes"].cpu().numpy()
    gap = r["gap"].cpu().numpy()
    assert codes.shape == (16, 4080)
    assert codes.min() >= 0 and codes.max() < c["v"]
    assert torch.equal(rec, r["recon"])
    print("flagged rows:", r["n_flagged"])
    csq = oracle.rvq_csq(cb)
    rng = np.random.default_rng(35)
    off = 0
    for l, s in enumerate(c["strides"]):
        n = 16 * (c["t"] // s)
        rows = np.unique(rng.integers(0, n, size=24)).astype(np.int64)
        got, ogap = oracle.rvq_level_rows(x, cb, c["strides"], csq, codes, l, rows)
        per_b = c["t"] // s
        gpu = codes[rows // per_b, off + rows % per_b]
        assert np.array_equal(got, gpu), (l, np.sum(got != gpu))
        # Near-ties (relative top-2 gap < 1e-5) are reported: the GPU's gap
        # classifies every sampled row as the oracle's full search does, and
        # equals it where it is small.
        g = gap[rows // per_b, off + rows % per_b]
        assert np.array_equal(g < 1e-5, ogap < 1e-5), (l, g, ogap)
        small = ogap < 1e-4
        assert np.allclose(g[small], ogap[small], rtol=1e-3, atol=1e-9), (l, g[small], ogap[small])
        assert np.all(ogap[~np.isfinite(g)] >= 1e-5)
        off += per_b
    print("near-ties (gap < 1e-5):", int((gap < 1e-5).sum()), "of", gap.size)
    # One whole sequence against the oracle's own exhaustive encode (no
    # teacher forcing): all 4080 codes and the 2048 x 2048 reconstruction
    # bit for bit.
    import os

    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    ref = oracle.rvq_encode(np.ascontiguousarray(x[:1]), cb, c["strides"], csq=csq,
                            want_gap=False, threads=threads)
    assert np.array_equal(ref["codes"][0], codes[0]), int(np.sum(ref["codes"][0] != codes[0]))
    assert np.array_equal(ref["recon"][0].view(np.uint32),
                          r["recon"][0].cpu().numpy().view(np.uint32))


def test_rows_wider_than_the_row_kernels_are_refused(ncm, cuda):
    """The row kernels hold a row of up to 4096 elements in registers: a
    wider encode is NCM_E_SHAPE, not a partial row."""
    import torch
    from ncmorph_amd import vq
    from ncmorph_amd._lib import NCM_E_SHAPE, NcmError

    x = torch.zeros((1, 4, 4160), dtype=torch.float32, device=cuda)
    cb = torch.zeros((1, 8, 4160), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(NcmError) as e:
        vq.encode(x, cb, (1,))
    assert e.value.status == NCM_E_SHAPE
