"""MI355X (gfx950) neural-texture train/decode hot path.

The product is libnt_hip.so, a C-ABI library (include/nt/nt.h) of hand-written HIP kernels.
This package loads it with ctypes and offers helpers that lay out latent grids, networks
and reference textures in torch (device) or numpy (host) memory for that ABI.

Import torch before the library is loaded so that both share torch's HIP runtime
(libamdhip64.so.7 is resolved once per process); load() does this itself.
"""
from __future__ import annotations

import ctypes
import os

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(HERE, "libnt_hip.so")

_lib = None


class NtError(RuntimeError):
    """A C-ABI call returned a non-zero nt_status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def load() -> ctypes.CDLL:
    """Loads libnt_hip.so (built by neural_textures_amd.build). Raises if it is missing:
    there is no fallback path."""
    global _lib
    if _lib is None:
        try:
            import torch  # noqa: F401  (shares torch's HIP runtime)
        except ImportError:
            pass
        if not os.path.exists(LIBRARY_PATH):
            raise RuntimeError(
                f"{LIBRARY_PATH} is not built; run `python -m neural_textures_amd.build`")
        _lib = abi.bind(ctypes.CDLL(LIBRARY_PATH))
        if _lib.nt_abi_version() != abi.NT_ABI_VERSION:
            raise RuntimeError("libnt_hip.so ABI version does not match abi.py")
    return _lib


def check(status: int) -> None:
    """Raises NtError for a non-zero status, with the library's message."""
    if status != abi.NT_OK:
        lib = load()
        msg = lib.nt_last_error().decode()
        raise NtError(status, f"{lib.nt_status_string(status).decode()}: {msg}")


def stream_handle(stream=None) -> ctypes.c_void_p:
    """hipStream_t of a torch stream (the current one by default) as a void*."""
    import torch

    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)
