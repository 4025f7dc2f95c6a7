"""Safetensors weights on the device (packages/safetensors/root.zig and the
loader's weight path, src/loader.zig:95-202, 339-342): the header and
sharded-index reader of the C ABI (ncm_st_*) and the direct upload of
stored bytes, so bf16 weights reach HBM as they are stored instead of being
widened to f32 on the host.

Malformed input raises NcmError whose `detail` is the reference's error
name ("InvalidOffsets", "SizeMismatch", ...).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

from ._lib import NcmError, check, lib

MAX_DIMS = 8


class _Info(C.Structure):
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_int32), ("ndim", C.c_int32),
                ("shape", C.c_uint64 * MAX_DIMS), ("data_begin", C.c_uint64),
                ("data_end", C.c_uint64)]


@dataclass
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    data_begin: int
    data_end: int

    @property
    def nbytes(self) -> int:
        return self.data_end - self.data_begin


def _info(raw: _Info) -> TensorInfo:
    return TensorInfo(raw.name.decode(), lib().ncm_st_dtype_name(raw.dtype).decode(),
                      tuple(int(raw.shape[k]) for k in range(min(raw.ndim, MAX_DIMS))),
                      int(raw.data_begin), int(raw.data_end))


class SafetensorsFile:
    """A parsed header: from a path (mapped, uploadable) or from bytes in
    memory (parse_header, root.zig:148-193)."""

    def __init__(self, path: str | None = None, data: bytes | None = None,
                 file_size: int | None = None):
        h = C.c_void_p()
        if path is not None:
            check(lib().ncm_st_open(str(path).encode(), C.byref(h)), "safetensors open")
        else:
            buf = bytes(data)
            size = len(buf) if file_size is None else file_size
            check(lib().ncm_st_parse(buf, len(buf), size, C.byref(h)), "safetensors parse")
        self._h = h

    def close(self):
        if self._h:
            lib().ncm_st_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def summary(self):
        hl, dl, n = C.c_uint64(), C.c_uint64(), C.c_int64()
        check(lib().ncm_st_summary(self._h, C.byref(hl), C.byref(dl), C.byref(n)), "summary")
        return int(hl.value), int(dl.value), int(n.value)

    def tensors(self) -> list:
        """Tensors in data-offset order."""
        out = []
        for i in range(self.summary()[2]):
            raw = _Info()
            check(lib().ncm_st_tensor(self._h, i, C.byref(raw)), "safetensors tensor")
            out.append(_info(raw))
        return out

    def find(self, name: str) -> TensorInfo:
        raw = _Info()
        check(lib().ncm_st_find(self._h, name.encode(), C.byref(raw)), f"tensor {name}")
        return _info(raw)

    def upload(self, name: str, out, ctx=None):
        """Copies tensor `name`'s stored bytes into the device tensor `out`
        (contiguous, same byte size) on torch's current stream."""
        from .context import default_context

        if not out.is_cuda or not out.is_contiguous():
            raise ValueError("out must be a contiguous GPU tensor")
        ctx = ctx or default_context(out.device.index or 0)
        ctx.bind_stream()
        check(lib().ncm_st_upload(ctx.handle, self._h, name.encode(), C.c_void_p(out.data_ptr()),
                                  out.numel() * out.element_size()), f"upload {name}")
        return out


def parse_index(text: str):
    """(weight_map [(tensor, shard)], total_size or None) of a sharded index
    (parse_index, root.zig:197-228)."""
    raw = text.encode()
    h = C.c_void_p()
    check(lib().ncm_st_parse_index(raw, len(raw), C.byref(h)), "safetensors index")
    try:
        entries = []
        t, s = C.c_char_p(), C.c_char_p()
        for i in range(lib().ncm_st_index_count(h)):
            check(lib().ncm_st_index_entry(h, i, C.byref(t), C.byref(s)), "index entry")
            entries.append((t.value.decode(), s.value.decode()))
        total = C.c_uint64()
        rc = lib().ncm_st_index_total_size(h, C.byref(total))
        return entries, (int(total.value) if rc == 0 else None)
    finally:
        lib().ncm_st_index_close(h)


def write_file(path: str, tensors: dict, metadata: dict | None = None) -> None:
    """Writes a safetensors file from {name: (dtype_name, shape, raw bytes)}
    (for tests and synthetic checkpoints), tensors in the given order."""
    import json

    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    off = 0
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
    js = json.dumps(header, separators=(",", ":")).encode()
    js += b" " * ((8 - len(js) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(js).to_bytes(8, "little"))
        f.write(js)
        for _, (_, _, raw) in tensors.items():
            f.write(raw)


__all__ = ["SafetensorsFile", "TensorInfo", "parse_index", "write_file", "NcmError"]
