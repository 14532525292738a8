"""ctypes binding of ``libmhc_hip.so`` (the C ABI declared in ``include/mhc_abi.h``).

The library is built in-tree by ``make -C mhc-triton_amd`` (or
``__graft_entry__.build()``) and loaded lazily on the first kernel call.  There
is no fallback: if the library is missing, or a tensor is not on a ROCm GPU,
the call raises.  ``import torch`` always precedes loading the library so that
the HIP runtime torch ships (soname ``libamdhip64.so.7``) is the one the
library binds to; pointers and streams are therefore shared with torch.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmhc_hip.so")

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/mhc_abi.h
_SIGNATURES = {
    "mhc_abi_version": (_I, []),
    "mhc_last_error": (ctypes.c_char_p, []),
    "mhc_sinkhorn_forward": (_I, [_P, _P, _I64, _I, _I, _F, _P]),
    "mhc_sinkhorn_backward": (_I, [_P, _I, _P, _I, _P, _I64, _I, _F, _P]),
    "mhc_stream_mix_forward": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "mhc_stream_mix_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "mhc_stream_mix_backward": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ, _P]),
    "mhc_add_residual_forward": (_I, [_P, _I, _P, _I, _P, _P, _I64, _I64, _I64, _P]),
    "mhc_add_residual_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "mhc_add_residual_backward": (_I, [_P, _I, _P, _I, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mhc_dynamic_weights_workspace_bytes": (_SZ, [_I64, _I64]),
    "mhc_dynamic_weights_forward": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _F, _P, _SZ, _P]),
    "mhc_dynamic_weights_backward_workspace_bytes": (_SZ, [_I64, _I64]),
    "mhc_dynamic_weights_backward": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _F, _P, _SZ, _P]),
    "mhc_layer_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "mhc_stream_expand": (_I, [_P, _I, _P, _I, _I64, _I64, _I64, _F, _P]),
    "mhc_stream_collapse": (_I, [_P, _I, _P, _I, _I64, _I64, _I64, _F, _P]),
    "mhc_mean_pool_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I]),
    "mhc_mean_pool": (_I, [_P, _I, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mhc_layer_dynamic_forward": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _F, _P, _SZ, _P]),
    "mhc_layer_dynamic_forward_noalloc": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _F, _P]),
    "mhc_layer_static_forward": (_I, [_P, _I, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P]),
    "mhc_layer_branch_input": (_I, [_P, _I, _P, _P, _I64, _I64, _I64, _P]),
    "mhc_layer_mix_backward": (_I, [_P, _I, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mhc_layer_mix_dh": (_I, [_P, _P, _I, _P, _P, _P, _I64, _I64, _I64, _P]),
    "mhc_layer_add_forward": (_I, [_P, _I, _P, _I, _P, _P, _I64, _I64, _I64, _P]),
    "mhc_layer_add_backward": (_I, [_P, _I, _P, _I, _P, _P, _P, _I64, _I64, _I64, _P, _SZ, _P]),
    "mhc_layer_dynamic_backward": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
             _I64, _I64, _I64, _I, _F, _P, _SZ, _P]),
    "mhc_layer_static_backward": (
        _I, [_P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _SZ, _P]),
}

ABI_VERSION = 3

_lib = None
_lock = threading.Lock()


class MHCError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the HIP library, with argument types bound."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MHCError(
                    f"mhc: HIP library not built ({LIB_PATH} missing); run "
                    "`make -C mhc-triton_amd` or `python -c 'import __graft_entry__ as g; g.build()'`")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.mhc_abi_version() != ABI_VERSION:
                raise MHCError(f"mhc: library ABI {lib.mhc_abi_version()} != expected {ABI_VERSION}; rebuild")
            _lib = lib
    return _lib


def check(rc: int, name: str) -> None:
    if rc != 0:
        msg = load().mhc_last_error().decode(errors="replace")
        raise MHCError(f"mhc: {name} failed (status {rc}): {msg}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise TypeError(f"mhc: unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def require_gpu(*tensors) -> torch.device:
    """All tensors must live on the same ROCm GPU; returns that device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                f"mhc: the HIP kernels need tensors on a ROCm GPU, got device '{t.device}' "
                "(the *_torch baselines run on CPU)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"mhc: tensors on different devices ({dev} and {t.device})")
    if dev is None:
        raise RuntimeError("mhc: no tensor arguments")
    return dev


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(dev: torch.device) -> int:
    """The handle of torch's current stream on `dev` (the stream every launch goes to).  The raw
    getter skips building a torch.cuda.Stream object (about 5 us of host time per call)."""
    if _raw_stream is not None:
        return _raw_stream(dev.index if dev.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(dev).cuda_stream


def workspace(nbytes: int, dev: torch.device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(int(nbytes), dtype=torch.uint8, device=dev)


class on_device:
    """Make `dev` the current HIP device for the duration of a call."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev: torch.device):
        self.dev = dev.index if dev.index is not None else torch.cuda.current_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.dev:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False
