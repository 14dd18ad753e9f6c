"""Loader for libnaylis_mom.so, the C-ABI library of HIP kernels.

The library is built in-tree (``naylis_amd/_lib/libnaylis_mom.so``, see
``naylis_amd/build.py``) and loaded with ctypes; argument types of every
entry point are declared here from ``include/naylis_mom.h``.  There is no
fallback: a missing or stale library raises ``RuntimeError``.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
import threading

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libnaylis_mom.so")
ABI_VERSION = 17

NAYLIS_OK = 0
NAYLIS_ERR_ARG = 1
NAYLIS_ERR_WORKSPACE = 2
NAYLIS_ERR_HIP = 3

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_size_t = ctypes.c_size_t
_pp = ctypes.POINTER(ctypes.c_void_p)  # host array of device pointers
_int = ctypes.c_int
_float = ctypes.c_float

# name -> (restype, argtypes); mirrors include/naylis_mom.h
SIGNATURES = {
    "naylis_mom_abi_version": (_int, []),
    "naylis_mom_last_error": (ctypes.c_char_p, []),
    "naylis_mom_read_workspace_bytes": (_size_t, [_i64] * 7),
    "naylis_mom_read_side_bytes": (_size_t, [_i64] * 7),
    "naylis_mom_read_fwd": (_int, [_c_void_p] * 9 + [_c_void_p, _size_t] + [_i64] * 7 + [_c_void_p]),
    "naylis_mom_read_bwd": (_int, [_c_void_p] * 14 + [_c_void_p, _size_t] + [_i64] * 7 + [_c_void_p]),
    "naylis_mom_read_bwd_noalloc": (_int, [_c_void_p] * 14 + [_i64] * 7 + [_c_void_p]),
    "naylis_mom_read_order_words": (_i64, [_i64] * 4),
    "naylis_mom_read_order_workspace_bytes": (_size_t, [_i64] * 4),
    "naylis_mom_read_order": (_int, [_c_void_p, _c_void_p, _c_void_p, _size_t] + [_i64] * 4 + [_c_void_p]),
    "naylis_mom_router_workspace_bytes": (_size_t, [_i64] * 6),
    "naylis_mom_router_fwd": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _int, _float]
                              + [_c_void_p] * 6 + [_c_void_p, _size_t] + [_i64] * 6 + [_c_void_p]),
    "naylis_mom_spin_limit": (_int, [_int]),
    "naylis_mom_router_bwd": (_int, [_c_void_p, _int] + [_c_void_p] * 8 + [_i64] + [_c_void_p] * 2 + [_int]
                              + [_c_void_p] * 2 + [_c_void_p, _size_t] + [_i64] * 6 + [_c_void_p]),
    "naylis_mom_router_stats_workspace_bytes": (_size_t, [_i64] * 2),
    "naylis_mom_router_stats": (_int, [_c_void_p] * 4 + [_size_t] + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_bank_kv_fwd": (_int, [_c_void_p] * 5 + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_rmsnorm_fwd": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _float,
                                      _c_void_p]),
    "naylis_mom_rmsnorm_workspace_bytes": (_size_t, [_i64] * 2),
    "naylis_mom_add_rmsnorm_fwd": (_int, [_c_void_p, _c_void_p, _int] + [_c_void_p] * 4 + [_int, _i64, _i64, _float,
                                                                                          _c_void_p]),
    "naylis_mom_add_rmsnorm_bwd": (_int, [_c_void_p] * 8 + [_size_t, _int, _i64, _i64, _c_void_p]),
    "naylis_mom_rope": (_int, [_c_void_p] * 6 + [_int, _int] + [_i64] * 5 + [_c_void_p]),
    "naylis_mom_swiglu_fwd": (_int, [_c_void_p] * 3 + [_int, _i64, _c_void_p]),
    "naylis_mom_xent_fwd": (_int, [_c_void_p] * 4 + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_xent_bwd": (_int, [_c_void_p] * 4 + [_i64, _c_void_p] + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_swiglu_bwd": (_int, [_c_void_p] * 5 + [_int, _i64, _c_void_p]),
    "naylis_mom_rmsnorm_bwd": (_int, [_c_void_p, _int] + [_c_void_p] * 6 + [_size_t, _i64, _i64, _c_void_p]),
    "naylis_mom_linear_wgrad_workspace_bytes": (_size_t, [_i64] * 3),
    "naylis_mom_rezero_workspace_bytes": (_size_t, [_i64]),
    "naylis_mom_rezero_fwd": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _i64, _c_void_p]),
    "naylis_mom_rezero_bwd": (_int, [_c_void_p, _int, _c_void_p, _int] + [_c_void_p] * 4 + [_size_t, _i64, _c_void_p]),
    "naylis_mom_rezero_scale": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _int, _i64, _c_void_p]),
    "naylis_mom_linear_wgrad": (_int, [_c_void_p] * 3 + [_int, _c_void_p, _size_t] + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_gated_wgrad_workspace_bytes": (_size_t, [_i64] * 3),
    "naylis_mom_gated_wgrad": (_int, [_c_void_p] * 7 + [_size_t] + [_i64] * 3 + [_c_void_p]),
    "naylis_mom_bank_kv_bwd": (_int, [_c_void_p] * 6 + [_int, _c_void_p, _c_void_p, _int] + [_i64] * 3
                               + [_c_void_p]),
    "naylis_mom_bank_kv_fwd_grouped": (_int, [_c_void_p] + [_pp] * 4 + [_i64] * 4 + [_c_void_p]),
    "naylis_mom_bank_kv_bwd_grouped_workspace_bytes": (_size_t, [_i64] * 4),
    "naylis_mom_bank_kv_bwd_grouped": (_int, [_c_void_p] + [_pp] * 4 + [_c_void_p, _int] + [_pp] * 2
                                       + [_int, _c_void_p, _size_t] + [_i64] * 4 + [_c_void_p]),
    "naylis_mom_bank_quant_fp8": (_int, [_c_void_p] * 6 + [_i64] * 2 + [_c_void_p]),
    "naylis_mom_decode_step": (_int, [_c_void_p] * 4 + [_int] + [_c_void_p] * 10 + [_i64] * 7 + [_c_void_p]),
    "naylis_mom_timing_enable": (None, [_int]),
    "naylis_mom_timing_reset": (None, []),
    "naylis_mom_timing_get": (_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                     ctypes.POINTER(ctypes.c_int64)]),
    "naylis_mom_timing_names": (_int, [ctypes.c_char_p, _size_t]),
}

_lock = threading.Lock()
_lib = None


class NaylisError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def load():
    """Load (once) and return the ctypes handle; raises if unavailable."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"naylis_amd: HIP library not built ({LIB_PATH} missing). "
                "Run `python -c 'import __graft_entry__ as g; g.build()'` or "
                "`python -m naylis_amd.build` first.")
        # global visibility: the torch extension of the fused layer node
        # (naylis_amd/_torch_ext.py) binds its calls to this instance
        lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.naylis_mom_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"naylis_amd: library ABI {ver} != expected {ABI_VERSION}; rebuild it")
        _lib = lib
        return lib


def check(rc):
    """Raise NaylisError for a non-zero status code."""
    if rc != NAYLIS_OK:
        msg = load().naylis_mom_last_error()
        msg = msg.decode() if msg else "unknown error"
        raise NaylisError(rc, msg)


class KernelTimer:
    """Per-kernel HIP-event totals collected by the library while enabled."""

    def __enter__(self):
        lib = load()
        lib.naylis_mom_timing_reset()
        lib.naylis_mom_timing_enable(1)
        return self

    def __exit__(self, *exc):
        load().naylis_mom_timing_enable(0)
        return False

    @staticmethod
    def results():
        """{kernel name: (total_ms, launches)} (waits for the recorded events)."""
        lib = load()
        buf = ctypes.create_string_buffer(8192)
        check(lib.naylis_mom_timing_names(buf, len(buf)))
        out = {}
        for name in filter(None, buf.value.decode().split(",")):
            ms = ctypes.c_double()
            n = ctypes.c_int64()
            check(lib.naylis_mom_timing_get(name.encode(), ctypes.byref(ms), ctypes.byref(n)))
            out[name] = (ms.value, n.value)
        return out


def available():
    try:
        load()
        return True
    except (RuntimeError, OSError):
        return False


_NULL_CTX = contextlib.nullcontext()


def on_device(device):
    """Context making `device` current only when it is not already: a switch
    costs two runtime calls per launch, and the layer's tensors normally sit
    on the current device."""
    import torch
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if torch.cuda.current_device() == idx:
        return _NULL_CTX
    return torch.cuda.device(idx)


def stream_of(device):
    """Raw handle of torch's current stream on `device` (where launches go)."""
    import torch
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
