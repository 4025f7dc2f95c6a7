"""Argument checks of the device-tensor wrappers.

The C ABI receives bare device pointers and cannot see how large each
allocation is, so a tensor of the wrong dtype or shape would be read or
written out of bounds on the GPU. Every wrapper therefore checks each tensor
argument (caller-supplied outputs included) here, before any library call,
and raises NcmError on a mismatch: dtype first, then shape, then device and
layout, so that the checks also run without a GPU.
"""
from __future__ import annotations

import ctypes as C

from ._lib import NCM_E_ARG, NCM_E_NULL, NCM_E_SHAPE, NcmError

# bf16 operands travel as 16-bit patterns: torch.bfloat16, or an int16 /
# uint16 view of the same bytes.
BF16 = ("bfloat16", "int16", "uint16")
F32 = ("float32",)
I32 = ("int32",)
U64 = ("int64", "uint64")


def _dtype(t) -> str:
    return str(t.dtype).replace("torch.", "")


def _common(t, name, where, dtypes):
    if not hasattr(t, "data_ptr") or not hasattr(t, "is_cuda"):
        raise NcmError(NCM_E_ARG, where, f"{name} must be a torch tensor")
    if _dtype(t) not in dtypes:
        raise NcmError(NCM_E_ARG, where,
                       f"{name} has dtype {_dtype(t)}, expected {' or '.join(dtypes)}")


def _placed(t, name, where, device):
    if not t.is_cuda:
        raise NcmError(NCM_E_ARG, where, f"{name} must be a GPU tensor")
    if device is not None and t.device != device:
        raise NcmError(NCM_E_ARG, where, f"{name} is on {t.device}, expected {device}")


class Args:
    """The tensor arguments of one call: dev() and rows() check dtype, shape
    and layout as they are named; done() then checks that every one of them
    is a GPU tensor on the first one's device."""

    def __init__(self, where: str):
        self.where = where
        self.seen = []

    def dev(self, t, name, dtypes, shape=None, optional=False):
        """Pointer of a contiguous tensor of one of `dtypes` and exactly
        `shape` (None: any shape); None for an optional None."""
        W = self.where
        if t is None:
            if optional:
                return None
            raise NcmError(NCM_E_NULL, W, f"{name} is required")
        _common(t, name, W, dtypes)
        if shape is not None and tuple(t.shape) != tuple(int(s) for s in shape):
            raise NcmError(NCM_E_SHAPE, W,
                           f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
        if not t.is_contiguous():
            raise NcmError(NCM_E_ARG, W, f"{name} must be contiguous")
        self.seen.append((t, name))
        return C.c_void_p(t.data_ptr())

    def rows(self, t, name, dtypes, n_rows, min_cols):
        """(pointer, row stride) of a 2-D tensor with contiguous rows (a
        column slice of a wider buffer is allowed): exactly n_rows rows of
        at least min_cols elements."""
        W = self.where
        if t is None:
            raise NcmError(NCM_E_NULL, W, f"{name} is required")
        _common(t, name, W, dtypes)
        if t.dim() != 2 or t.shape[0] != n_rows or t.shape[1] < min_cols:
            raise NcmError(NCM_E_SHAPE, W,
                           f"{name} has shape {tuple(t.shape)}, expected ({n_rows}, >= {min_cols})")
        if t.stride(1) != 1 or (n_rows > 1 and t.stride(0) < min_cols):
            raise NcmError(NCM_E_ARG, W, f"{name} must have contiguous, non-overlapping rows")
        self.seen.append((t, name))
        return C.c_void_p(t.data_ptr()), t.stride(0)

    def done(self):
        device = self.seen[0][0].device if self.seen else None
        for t, name in self.seen:
            _placed(t, name, self.where, device)


def dims(t, name, where, ndim):
    """The shape of a tensor that must have `ndim` dimensions."""
    if t is None:
        raise NcmError(NCM_E_NULL, where, f"{name} is required")
    if not hasattr(t, "shape") or len(t.shape) != ndim:
        raise NcmError(NCM_E_SHAPE, where, f"{name} must have {ndim} dimensions")
    return tuple(int(s) for s in t.shape)
