"""Device context: one gfx950 device, one stream, cached workspace."""
from __future__ import annotations

import ctypes as C
import threading

from ._lib import check, lib


class Context:
    """Owns an ncm_ctx_t. Each call runs on torch's current stream of the
    context's device, so library kernels order with torch's own work."""

    def __init__(self, device: int = 0):
        self.device = device
        h = C.c_void_p()
        check(lib().ncm_init(device, C.byref(h)), "ncm_init")
        self.handle = h
        self._bound = None  # stream handle last passed to ncm_set_stream

    def bind_stream(self, stream=None) -> None:
        """Route library work to `stream` (a torch.cuda.Stream) or to torch's
        current stream on this device."""
        import torch

        if stream is None:
            stream = torch.cuda.current_stream(self.device)
        h = stream.cuda_stream
        if h != self._bound:
            check(lib().ncm_set_stream(self.handle, C.c_void_p(h)), "ncm_set_stream")
            self._bound = h

    def synchronize(self) -> None:
        check(lib().ncm_synchronize(self.handle), "ncm_synchronize")

    def close(self) -> None:
        if self.handle:
            lib().ncm_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_tls = threading.local()


def default_context(device: int = 0) -> Context:
    ctxs = getattr(_tls, "ctxs", None)
    if ctxs is None:
        ctxs = _tls.ctxs = {}
    if device not in ctxs:
        ctxs[device] = Context(device)
    return ctxs[device]
