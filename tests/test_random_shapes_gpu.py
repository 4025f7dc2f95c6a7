"""Seeded random shapes through the device paths, each against its bar: the
bf16 linear against the f64 product within the fp32-accumulation bound
(every tile configuration the automatic choice can take, ragged M, N and K),
the RVQ encode bit-identical to the oracle (random strides, widths that are
multiples of 64, codebook sizes), and the causal attention against the
oracle within its stated bound. Sizes stay where the oracle finishes in
seconds."""
import numpy as np
import pytest

from ncmorph_amd import synth

pytestmark = pytest.mark.gpu


def _bf16_dev(bits, cuda):
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(cuda).view(torch.bfloat16)


def _linear_cases(n):
    rng = np.random.default_rng(2026)
    out = []
    for _ in range(n):
        m = int(rng.integers(1, 3000))
        nn = int(rng.integers(1, 6000))
        k = 8 * int(rng.integers(1, 300))
        out.append((m, nn, k, bool(rng.random() < 0.5)))
    return out


@pytest.mark.parametrize("m,n,k,bias", _linear_cases(16))
def test_random_linear(ncm, cuda, m, n, k, bias):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(m * 7 + n * 3 + k)
    xb = synth.bf16_bits(rng.standard_normal((m, k)).astype(np.float32))
    wb = synth.bf16_bits((rng.standard_normal((n, k)) * 0.05).astype(np.float32))
    bb = synth.bf16_bits(rng.standard_normal(n).astype(np.float32)) if bias else None
    y = kernels.linear_bf16(_bf16_dev(xb, cuda), _bf16_dev(wb, cuda),
                            bias=None if bb is None else _bf16_dev(bb, cuda))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    rows = np.unique(rng.integers(0, m, size=min(m, 64)))
    x64 = synth.bf16_to_f32(xb[rows]).astype(np.float64)
    w64 = synth.bf16_to_f32(wb).astype(np.float64)
    ref = x64 @ w64.T
    asum = np.abs(x64) @ np.abs(w64).T
    if bias:
        b64 = synth.bf16_to_f32(bb).astype(np.float64)
        ref = ref + b64
        asum = asum + np.abs(b64)
    assert np.all(np.abs(y[rows] - ref) <= (k + 2) * 2.0**-24 * asum + 1e-30), (m, n, k)


def _rvq_cases(n):
    rng = np.random.default_rng(77)
    out = []
    for i in range(n):
        levels = int(rng.integers(1, 5))
        strides = sorted((int(2 ** rng.integers(0, 5)) for _ in range(levels)), reverse=True)
        t = strides[0] * int(rng.integers(1, 9))
        out.append(dict(b=int(rng.integers(1, 4)), t=t, d=64 * int(rng.integers(1, 7)),
                        v=int(rng.integers(1, 1500)), strides=tuple(strides), seed=100 + i))
    return out


@pytest.mark.parametrize("case", _rvq_cases(8))
def test_random_rvq(ncm, oracle, cuda, case):
    import torch
    from ncmorph_amd import vq

    L = len(case["strides"])
    x, cb = synth.rvq_inputs(case["seed"], case["b"], case["t"], case["d"], L, case["v"])
    xd = torch.from_numpy(x).to(cuda)
    cbd = _bf16_dev(cb, cuda)
    r = vq.encode(xd, cbd, case["strides"])
    torch.cuda.synchronize()
    ref = oracle.rvq_encode(x, cb, case["strides"], threads=8)
    assert np.array_equal(r["codes"].cpu().numpy(), ref["codes"])
    assert np.array_equal(r["recon"].cpu().numpy(), ref["recon"])


def _attention_cases(n):
    rng = np.random.default_rng(31)
    out = []
    for _ in range(n):
        hkv = int(rng.integers(1, 4))
        out.append((int(rng.integers(1, 3)), int(rng.integers(1, 400)),
                    hkv * int(rng.integers(1, 4)), hkv, int(rng.choice([64, 128])),
                    int(rng.choice([0, 0, 50]))))
    return out


@pytest.mark.parametrize("batch,seq,hq,hkv,hd,window", _attention_cases(6))
def test_random_attention(ncm, oracle, cuda, batch, seq, hq, hkv, hd, window):
    import torch
    from ncmorph_amd import kernels

    rng = np.random.default_rng(seq * 11 + hd + window)
    rb = oracle.round_bf16
    q = rb(rng.standard_normal((batch * seq, hq * hd)).astype(np.float32) * 1.5)
    k = rb(rng.standard_normal((batch * seq, hkv * hd)).astype(np.float32) * 1.5)
    v = rb(rng.standard_normal((batch * seq, hkv * hd)).astype(np.float32))
    out = kernels.attention_bf16(_bf16_dev(synth.bf16_bits(q), cuda),
                                 _bf16_dev(synth.bf16_bits(k), cuda),
                                 _bf16_dev(synth.bf16_bits(v), cuda),
                                 batch, seq, hq, hkv, hd, window=window)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    mask = oracle.causal_mask(seq, window)
    vmax = float(np.max(np.abs(v)))
    for b in range(batch):
        rows = slice(b * seq, (b + 1) * seq)
        ref = oracle.attention_core(q[rows], k[rows], v[rows], mask, hq, hkv, hd)
        bound = 2.0**-7 * np.abs(ref) + 2.0**-7 * vmax
        assert np.all(np.abs(got[rows] - ref) <= bound)
