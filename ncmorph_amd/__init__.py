"""ncmorph_amd: MI355X (gfx950) hot path of ncmorph.

Python mirror of the reference's Zig operator surface over the C ABI in
include/ncmorph_amd.h:
  - ncmorph_amd.kernels: matmul_bf16, matmul_bf16_bias, round_bf16
    (packages/kernels/root.zig:10-12, :96-104), host slices in and out;
    plus linear_bf16 on device tensors (the benchmarked path).
  - ncmorph_amd.vq: multiscale residual VQ encode / decode on device tensors.
"""
from ._lib import NcmError, lib  # noqa: F401
from .context import Context, default_context  # noqa: F401
