"""The device wrappers check every tensor argument (dtype, exact shape,
device, layout), caller-supplied outputs included, and raise NcmError before
any library call: the C ABI receives bare pointers and cannot see allocation
sizes. These run on the CPU: dtype and shape are checked before the device,
and a tensor that passes them but lives on the CPU is refused as well."""
import pytest
import torch

from ncmorph_amd import kernels, vq
from ncmorph_amd._lib import NCM_E_ARG, NCM_E_NULL, NCM_E_SHAPE, NcmError

bf, f32, i32 = torch.bfloat16, torch.float32, torch.int32


def _raises(status, fn, *a, **kw):
    with pytest.raises(NcmError) as e:
        fn(*a, **kw)
    assert e.value.status == status, str(e.value)
    return str(e.value)


def z(*shape, dtype=bf):
    return torch.zeros(shape, dtype=dtype)


def test_linear_checks():
    x, w = z(8, 16), z(4, 16)
    _raises(NCM_E_SHAPE, kernels.linear_bf16, x, z(4, 8))             # k mismatch
    _raises(NCM_E_ARG, kernels.linear_bf16, z(8, 16, dtype=f32), w)   # fp32 x
    _raises(NCM_E_SHAPE, kernels.linear_bf16, x, w, bias=z(5))
    # a bf16 output buffer for the fp32 mode, and a short fp32 one
    _raises(NCM_E_ARG, kernels.linear_bf16, x, w, out=z(8, 4))
    _raises(NCM_E_SHAPE, kernels.linear_bf16, x, w, out=z(8, 3, dtype=f32))
    _raises(NCM_E_ARG, kernels.linear_bf16, x, w, out_mode="bf16", out=z(8, 4, dtype=f32))
    _raises(NCM_E_ARG, kernels.linear_bf16, x, w, out_mode="f16")
    msg = _raises(NCM_E_ARG, kernels.linear_bf16, x, w, out=z(8, 4, dtype=f32))
    assert "GPU" in msg                                               # all fine but on the CPU
    _raises(NCM_E_SHAPE, kernels.linear_bf16_residual, x, w, z(8, 5, dtype=f32))
    _raises(NCM_E_ARG, kernels.linear_bf16_residual, x, w, z(8, 4))
    _raises(NCM_E_SHAPE, kernels.linear_bf16_swiglu, x, z(96, 16))    # rows not % 64
    _raises(NCM_E_SHAPE, kernels.linear_bf16_swiglu, x, z(128, 16), out=z(8, 128))
    _raises(NCM_E_SHAPE, kernels.linear_bf16_rope64, x, z(64, 16), 64, 4, z(4, 32, dtype=f32),
            z(4, 64, dtype=f32))
    _raises(NCM_E_ARG, kernels.linear_f32, x, z(4, 16, dtype=f32))


def test_elementwise_checks():
    _raises(NCM_E_SHAPE, kernels.rms_norm_rows, z(3, 8, dtype=f32), z(7, dtype=f32), 1e-5)
    # the f32 mode writes float32: a bf16 out is refused
    _raises(NCM_E_ARG, kernels.rms_norm_rows, z(3, 8, dtype=f32), z(8, dtype=f32), 1e-5,
            out_mode="f32", out=z(3, 8))
    _raises(NCM_E_SHAPE, kernels.rms_norm_rows, z(3, 8, dtype=f32), z(8, dtype=f32), 1e-5,
            out=z(3, 8, dtype=f32)[:2])
    # up shorter than gate; a bf16 out for the float mode
    _raises(NCM_E_SHAPE, kernels.silu_mul, z(10, dtype=f32), z(9, dtype=f32))
    _raises(NCM_E_ARG, kernels.silu_mul, z(10, dtype=f32), z(10, dtype=f32), out=z(10))
    _raises(NCM_E_NULL, kernels.silu_mul, None)
    _raises(NCM_E_ARG, kernels.bf16_widen, z(4, dtype=f32))
    _raises(NCM_E_ARG, kernels.bf16_from_f32, z(4))


def test_attention_and_rope_checks():
    q, kv = z(8, 64), z(8, 32)
    _raises(NCM_E_SHAPE, kernels.rope_rotate, q, 2, 32, 8, z(8, 16, dtype=f32),
            z(8, 32, dtype=f32))
    _raises(NCM_E_SHAPE, kernels.rope_rotate, q, 4, 32, 8, z(8, 32, dtype=f32),
            z(8, 32, dtype=f32))                                      # 4 heads of 32 > 64 cols
    _raises(NCM_E_SHAPE, kernels.attention_bf16, q, kv, kv, 2, 4, 4, 2, 32)  # kv heads too wide
    _raises(NCM_E_SHAPE, kernels.attention_bf16, q, kv, kv, 1, 4, 2, 1, 32)  # 4 rows, not 8
    _raises(NCM_E_SHAPE, kernels.attention_bf16, q, kv, kv, 2, 4, 2, 1, 32,
            out=z(8, 32, dtype=f32))
    lo, hi = z(8, dtype=i32), z(8, dtype=i32)
    _raises(NCM_E_SHAPE, kernels.attention_bf16_seg, q, kv, kv, 1, 8, 2, 1, 32, 2, lo, z(7,
            dtype=i32))
    _raises(NCM_E_ARG, kernels.attention_bf16_seg, q, kv, kv, 1, 8, 2, 1, 32, 2, lo,
            z(8, dtype=f32))


def test_tied_head_checks():
    zz, cb = z(6, 64), z(10, 64)
    _raises(NCM_E_SHAPE, kernels.tied_head_logits, zz, cb, z(9, dtype=f32))
    _raises(NCM_E_SHAPE, kernels.tied_head_logits, zz, cb, z(10, dtype=f32),
            bias=z(11, dtype=f32))
    _raises(NCM_E_SHAPE, kernels.tied_head_logits_levels, z(6, 64), z(2, 10, 64),
            z(2, 10, dtype=f32), [2, 3])                              # rows sum 5, z has 6
    _raises(NCM_E_SHAPE, kernels.tied_head_logits_levels, z(5, 64), z(2, 10, 64),
            z(2, 10, dtype=f32), [2])


def test_rvq_checks():
    x, cb = z(2, 16, 64, dtype=f32), z(2, 8, 64)
    strides = (4, 1)
    _raises(NCM_E_SHAPE, vq.encode, x, z(2, 8, 32), strides)          # width mismatch
    _raises(NCM_E_SHAPE, vq.encode, x, cb, (4,))                      # one stride, two levels
    _raises(NCM_E_SHAPE, vq.encode, x, cb, (3, 1))                    # 3 does not divide 16
    _raises(NCM_E_ARG, vq.encode, z(2, 16, 64), cb, strides)          # bf16 x
    _raises(NCM_E_SHAPE, vq.encode, x, cb, strides, csq=z(2, 7, dtype=f32))
    _raises(NCM_E_SHAPE, vq.encode, x, cb, strides, csq=z(2, 8, dtype=f32),
            force_codes=z(2, 19, dtype=i32))                          # 4 + 16 = 20 codes
    _raises(NCM_E_ARG, vq.encode, x, cb, strides, csq=z(2, 8, dtype=f32),
            out={"codes": z(2, 20, dtype=f32)})
    _raises(NCM_E_SHAPE, vq.encode, x, cb, strides, csq=z(2, 8, dtype=f32),
            out={"recon": z(2, 16, 63, dtype=f32)})
    _raises(NCM_E_SHAPE, vq.decode, z(2, 19, dtype=i32), cb, strides, 16)
    _raises(NCM_E_ARG, vq.prepare, z(2, 8, 64, dtype=f32))


@pytest.mark.gpu
def test_device_tensors_checked_before_launch(cuda, ncm):
    x = torch.zeros(64, 128, dtype=bf, device=cuda)
    w = torch.zeros(32, 128, dtype=bf, device=cuda)
    _raises(NCM_E_SHAPE, kernels.linear_bf16, x, w,
            out=torch.zeros(64, 31, dtype=f32, device=cuda))
    _raises(NCM_E_ARG, kernels.linear_bf16, x, w.cpu())             # one operand on the host
    _raises(NCM_E_ARG, kernels.linear_bf16, x, w, out_mode="bf16",
            out=torch.zeros(64, 32, dtype=f32, device=cuda))
    g = torch.zeros(100, device=cuda)
    _raises(NCM_E_SHAPE, kernels.silu_mul, g, torch.zeros(99, device=cuda))
    xr = torch.zeros(2, 16, 64, device=cuda)
    cb = torch.zeros(2, 8, 64, dtype=bf, device=cuda)
    _raises(NCM_E_SHAPE, vq.encode, xr, cb, (4, 1),
            out={"codes": torch.zeros(2, 19, dtype=i32, device=cuda)})
    # a correct call still runs
    y = kernels.linear_bf16(x, w)
    torch.cuda.synchronize()
    assert y.shape == (64, 32) and float(y.abs().max()) == 0.0
