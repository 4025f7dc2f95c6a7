"""One context used from two streams: every entry point shares the
context's device workspace, so switching streams (ncm_set_stream) orders the
new stream after the work queued on the previous one. An RVQ encode on one
stream followed at once, without a host synchronisation, by attention on
another stream (whose transposed-V scratch lands in the same workspace)
gives the results of the same calls run one after the other."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_two_streams_share_the_workspace(ncm, cuda):
    import torch
    from ncmorph_amd import kernels, synth, vq
    from ncmorph_amd.context import default_context

    b, t, d, v = 4, 512, 512, 1024
    strides = (8, 4, 2, 1)
    x, cb = synth.rvq_inputs(5, b, t, d, len(strides), v)
    xd = torch.from_numpy(x).to(cuda)
    cbd = torch.from_numpy(cb.view(np.int16)).to(cuda).view(torch.bfloat16)
    csq = vq.prepare(cbd)
    T, hq, hkv, hd = 2048, 8, 2, 128
    g = torch.Generator(device=cuda).manual_seed(4)
    qkv = torch.randn(T, (hq + 2 * hkv) * hd, device=cuda, generator=g).to(torch.bfloat16)
    q, k, vv = qkv[:, :hq * hd], qkv[:, hq * hd:(hq + hkv) * hd], qkv[:, (hq + hkv) * hd:]

    def run_both(sa, sb, sync_between):
        with torch.cuda.stream(sa):
            r = vq.encode(xd, cbd, strides, csq=csq)
        if sync_between:
            torch.cuda.synchronize()
        with torch.cuda.stream(sb):
            a = kernels.attention_bf16(q, k, vv, 1, T, hq, hkv, hd, out_mode="bf16")
        torch.cuda.synchronize()
        return r["codes"].cpu(), r["recon"].cpu(), a.cpu()

    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    ref = run_both(s1, s1, True)
    for _ in range(3):
        got = run_both(s1, s2, False)
        for a, b_ in zip(ref, got):
            assert torch.equal(a.view(torch.int32) if a.dtype == torch.float32 else a, 
                               b_.view(torch.int32) if b_.dtype == torch.float32 else b_)
    assert default_context(0)._bound == s2.cuda_stream


def test_shape_products_that_would_wrap_are_refused(ncm, cuda):
    """Shape checks bound each factor before multiplying, so sizes whose
    products wrap int64 are refused (NCM_E_SHAPE) before any device work."""
    import ctypes as C

    import torch
    from ncmorph_amd._lib import NCM_E_SHAPE, lib
    from ncmorph_amd.context import default_context

    h = default_context().handle
    buf = torch.zeros(64, dtype=torch.float32, device=cuda)
    p = C.c_void_p(buf.data_ptr())
    strides = (C.c_int32 * 1)(1)
    # b * t = 2^62 * 4 wraps to 0.
    assert lib().ncm_rvq_encode(h, p, 1 << 62, 4, 64, 1, strides, p, p, 1, p, p, None, None,
                                None) == NCM_E_SHAPE
    # rows * heads * head_dim / 2 = 2^62 * 2 * 1 wraps to 0.
    assert lib().ncm_rope_rotate_dev(h, p, 1 << 62, 4, 2, 2, 1, p, p) == NCM_E_SHAPE
    torch.cuda.synchronize()
