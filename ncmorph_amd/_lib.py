"""ctypes binding of the C ABI in include/ncmorph_amd.h.

The shared library is built in-tree by ncmorph_amd/build.py. There is no
fallback: if the library is missing or cannot be loaded, every entry point
raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libncmorph_amd.so")

NCM_OK = 0
NCM_E_NULL = -1
NCM_E_SHAPE = -2
NCM_E_LENGTH = -3
NCM_E_HIP = -4
NCM_E_NOMEM = -5
NCM_E_DEVICE = -6
NCM_E_ARG = -7
NCM_E_FORMAT = -8
NCM_E_SCRATCH = -9
NCM_RVQ_SCRATCH_BYTES = 64 << 20

NCM_OUT_F32 = 0
NCM_OUT_BF16_F32 = 1
NCM_OUT_BF16 = 2

# (name, restype, argtypes) of every exported entry point, in header order.
vp, i32, i64, sz = C.c_void_p, C.c_int, C.c_int64, C.c_size_t
SIGNATURES = [
    ("ncm_status_string", C.c_char_p, [i32]),
    ("ncm_last_error", C.c_char_p, []),
    ("ncm_init", i32, [i32, C.POINTER(vp)]),
    ("ncm_destroy", i32, [vp]),
    ("ncm_set_stream", i32, [vp, vp]),
    ("ncm_get_stream", vp, [vp]),
    ("ncm_synchronize", i32, [vp]),
    ("ncm_matmul_f32", i32, [vp, sz, vp, sz, vp, sz, sz, sz, sz]),
    ("ncm_matmul_bf16", i32, [vp, sz, vp, sz, vp, sz, sz, sz, sz]),
    ("ncm_matmul_bf16_bias", i32, [vp, sz, vp, sz, vp, sz, vp, sz, sz, sz, sz]),
    ("ncm_matmul_bf16_exact", i32, [vp, sz, vp, sz, vp, sz, sz, sz, sz]),
    ("ncm_matmul_bf16_bias_exact", i32, [vp, sz, vp, sz, vp, sz, vp, sz, sz, sz, sz]),
    ("ncm_round_bf16", i32, [vp, vp, sz]),
    ("ncm_rms_norm_bf16", i32, [vp, sz, vp, sz, vp, sz, C.c_float]),
    ("ncm_silu_bf16", i32, [vp, sz, vp, sz]),
    ("ncm_linear_bf16", i32, [vp, vp, vp, vp, vp, i64, i64, i64, i32]),
    ("ncm_linear_bf16_exact", i32, [vp, vp, vp, vp, vp, i64, i64, i64, i32]),
    ("ncm_linear_bf16_residual", i32, [vp, vp, vp, vp, vp, vp, i64, i64, i64, i32]),
    ("ncm_linear_bf16_swiglu", i32, [vp, vp, vp, vp, vp, i64, i64, i64]),
    ("ncm_linear_bf16_rope64", i32, [vp, vp, vp, vp, vp, i64, i64, i64, i64, i64, vp, vp]),
    ("ncm_linear_f32", i32, [vp, vp, vp, vp, i64, i64, i64]),
    ("ncm_bf16_from_f32_dev", i32, [vp, vp, vp, i64, i32]),
    ("ncm_bf16_widen_dev", i32, [vp, vp, vp, i64]),
    ("ncm_rms_norm_rows_dev", i32, [vp, vp, vp, vp, i64, i64, C.c_float, i32]),
    ("ncm_silu_mul_dev", i32, [vp, vp, vp, vp, i64, i32]),
    ("ncm_rope_rotate_dev", i32, [vp, vp, i64, i64, i32, i32, i64, vp, vp]),
    ("ncm_attention_bf16_dev", i32, [vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, i64, i64, i64,
                                     i64, i32]),
    ("ncm_attention_bf16_seg_dev", i32, [vp, vp, vp, vp, vp, i64, i64, i32, i32, i32, i64, i64,
                                         i64, i64, vp, vp, vp, i32]),
    ("ncm_block_diagonal_segments", i32, [i64, vp, i64, vp, i64, i64, vp, vp, vp]),
    ("ncm_tied_head_logits", i32, [vp, vp, vp, vp, vp, C.c_float, vp, i64, i64, i64]),
    ("ncm_tied_head_logits_levels", i32, [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, vp]),
    ("ncm_decoder_forward_dev", i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp, vp]),
    ("ncm_decoder_forward_f32_dev", i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i64, i64, vp, vp]),
    ("ncm_ncm_forward_dev", i32, [vp, vp, vp, vp, vp, vp, i64, vp, vp, vp, vp, vp]),
    ("ncm_ncm_forward_f32_dev", i32, [vp, vp, vp, vp, vp, vp, i64, vp, vp, vp, vp, vp]),
    ("ncm_rvq_prepare", i32, [vp, vp, i64, i64, i64, vp]),
    ("ncm_rvq_encode", i32, [vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, vp, vp, vp, vp, vp]),
    ("ncm_rvq_encode_counts", i32, [vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, vp, vp, vp, vp,
                                    vp, vp]),
    ("ncm_rvq_encode_noalloc", i32, [vp, vp, i64, i64, i64, i64, vp, vp, vp, i64, vp, vp, vp,
                                     vp]),
    ("ncm_rvq_decode", i32, [vp, vp, i64, i64, i64, i64, vp, vp, i64, vp]),
    ("ncm_vq_tok_pack_conv_dev", i32, [vp, vp, vp, i64, i64, i32]),
    ("ncm_vq_tok_encode_dev", i32, [vp, vp, vp, i64, vp, vp, vp]),
    ("ncm_vq_tok_quantize_dev", i32, [vp, vp, vp, i64, vp, vp]),
    ("ncm_vq_tok_reconstruct_dev", i32, [vp, vp, vp, i64, vp]),
    ("ncm_vq_tok_decode_dev", i32, [vp, vp, vp, vp, i64, vp]),
    ("ncm_st_parse", i32, [vp, sz, C.c_uint64, C.POINTER(vp)]),
    ("ncm_st_open", i32, [C.c_char_p, C.POINTER(vp)]),
    ("ncm_st_close", i32, [vp]),
    ("ncm_st_summary", i32, [vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                             C.POINTER(C.c_int64)]),
    ("ncm_st_tensor", i32, [vp, i64, vp]),
    ("ncm_st_find", i32, [vp, C.c_char_p, vp]),
    ("ncm_st_dtype_name", C.c_char_p, [i32]),
    ("ncm_st_dtype_bits", i32, [i32]),
    ("ncm_st_upload", i32, [vp, vp, C.c_char_p, vp, sz]),
    ("ncm_st_parse_index", i32, [C.c_char_p, sz, C.POINTER(vp)]),
    ("ncm_st_index_close", i32, [vp]),
    ("ncm_st_index_count", i64, [vp]),
    ("ncm_st_index_entry", i32, [vp, i64, C.POINTER(C.c_char_p), C.POINTER(C.c_char_p)]),
    ("ncm_st_index_total_size", i32, [vp, C.POINTER(C.c_uint64)]),
]

_lib = None

# Status texts for errors raised before the library is loaded.
_STATUS_TEXT = {NCM_E_NULL: "null pointer argument", NCM_E_SHAPE: "invalid or unsupported shape",
                NCM_E_ARG: "argument out of range"}


class NcmError(RuntimeError):
    """A nonzero status from the C ABI."""

    def __init__(self, status: int, where: str, detail: str | None = None):
        """detail: the reason, for an error raised by a wrapper's own
        argument checks (the library's last-error text otherwise)."""
        self.status = status
        text = _STATUS_TEXT.get(status, "unknown status")
        lib_detail = ""
        if _lib is not None:
            text = _lib.ncm_status_string(status).decode()
            if detail is None:
                lib_detail = _lib.ncm_last_error().decode()
        msg = f"{where}: {text} ({status})"
        self.detail = lib_detail if status == NCM_E_FORMAT else (detail or "")
        if detail:
            msg += f": {detail}"
        elif lib_detail and status in (NCM_E_HIP, NCM_E_NOMEM, NCM_E_DEVICE, NCM_E_FORMAT,
                                       NCM_E_SCRATCH):
            msg += f" [{lib_detail}]"
        super().__init__(msg)


def lib():
    """Load the HIP library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"ncmorph_amd HIP library missing at {LIB_PATH}; "
                "build it with `python -m ncmorph_amd.build`")
        # One HIP runtime per process: when torch is present its bundled
        # libamdhip64 must be loaded first so that this library binds to the
        # same runtime (same SONAME) instead of loading a second copy.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = C.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, where: str) -> None:
    if status != NCM_OK:
        raise NcmError(status, where)
