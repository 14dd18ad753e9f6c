"""Naylis MoM kernels on MI355X: public API and backend selection.

Drop-in for the reference's ``mom_kernels`` package
(mom_kernels/__init__.py:1-117): ``preflight``, ``resolve_mode``,
``mom_read`` and ``announce`` keep their names, arguments and fail-loud
behaviour.  The one backend is ``"hip"`` — hand-written gfx950 kernels behind
the C ABI of ``libnaylis_mom.so``.  On ROCm, torch reports GPU devices as
``"cuda"``; those resolve to ``"hip"``.  Anything else raises: there is no
silent eager fallback (the eager maths lives only in the test oracle).

New entry points beyond the reference (it has no kernel boundary for them):
``mom_route`` (fused prefix-mean router) and ``mom_bank_kv`` (bank K/V
projection), used by ``naylis_amd.layer.MoMLayer``; ``quantize_bank_fp8`` and
``decode_step``, the one-token inference step over an fp8 bank (the reference
has no decode path).
"""
from __future__ import annotations

import torch

from .. import _lib
from .hip_read import mom_read as _hip_mom_read

__all__ = ["HAS_HIP", "preflight", "resolve_mode", "mom_read", "announce", "mom_route",
           "mom_bank_kv", "mom_bank_kv_grouped", "mom_linear", "mom_rezero", "mom_gated_linear", "has_hip", "quantize_bank_fp8", "decode_step",
           "mom_router_stats"]

_ANNOUNCED = {"backend": None}


def has_hip() -> bool:
    """True when torch is a ROCm build and the HIP library loads."""
    return torch.version.hip is not None and _lib.available()


HAS_HIP = _lib.available()


def _device_type(device) -> str:
    if isinstance(device, torch.device):
        return device.type
    return str(device).split(":")[0].lower()


def preflight(device_type: str) -> None:
    """Fail fast at startup if the requested device has no kernel backend
    (mom_kernels/__init__.py:37-53)."""
    if device_type == "cuda":
        if torch.version.hip is None:
            raise RuntimeError("use_kernel=true: this build targets ROCm (MI355X); torch is not a ROCm build.")
        if not _lib.available():
            raise RuntimeError(
                "use_kernel=true on ROCm requires libnaylis_mom.so "
                "(build it with `python -m naylis_amd.build`).")
        return
    raise RuntimeError(
        f"use_kernel=true requires a ROCm GPU device (HIP read); this process resolved to "
        f"{device_type!r}. The eager SDPA path is the test oracle, not a product backend.")


def resolve_mode(device, dtype, *, head_dim=None) -> str:
    """Pick the kernel backend and check its contract (mom_kernels/__init__.py:56-84).

    Requires bf16 activations and head_dim a power of two in [16, 128];
    violations raise instead of falling back to eager.
    """
    device_type = _device_type(device)
    if device_type == "cuda":
        if torch.version.hip is None or not _lib.available():
            raise RuntimeError("use_kernel=true: the HIP backend is not available on this box.")
        if dtype != torch.bfloat16:
            raise RuntimeError(
                f"use_kernel=true (hip) requires bf16 activations; got {dtype}.")
        if head_dim is not None:
            if head_dim > 128 or head_dim < 16 or head_dim & (head_dim - 1) != 0:
                raise RuntimeError(
                    f"use_kernel=true (hip): head_dim {head_dim} must be a power of two in [16, 128].")
        return "hip"
    raise RuntimeError(
        f"use_kernel=true: no kernel backend for device {device_type!r} (ROCm GPU -> HIP read).")


def mom_read(q_sh, k, v, top_idx, top_gates, *, num_blocks, block_size, mode: str):
    """MoM memory read with the per-token gate bias on the selected backend
    (mom_kernels/__init__.py:87-102).  Returns (B, S, H, hd)."""
    if mode == "hip":
        return _hip_mom_read(q_sh, k, v, top_idx, top_gates, num_blocks=num_blocks, block_size=block_size)
    raise RuntimeError(f"unknown kernel mode {mode!r}")


def announce(backend: str) -> None:
    """Print the backend banner once per process (mom_kernels/__init__.py:105-117)."""
    if _ANNOUNCED["backend"] != backend:
        _ANNOUNCED["backend"] = backend
        if backend == "hip":
            print("[MoM] use_kernel=true -> backend 'hip': gfx950 flash read with "
                  "in-register gate bias and block skipping, fused prefix-mean router, "
                  "MFMA bank K/V; deterministic backward.")


def mom_route(*args, **kwargs):
    from .hip_router import mom_route as _route
    return _route(*args, **kwargs)


def mom_router_stats(*args, **kwargs):
    from .hip_router import mom_router_stats as _stats
    return _stats(*args, **kwargs)


def mom_bank_kv(*args, **kwargs):
    from .hip_bank import mom_bank_kv as _bank
    return _bank(*args, **kwargs)


def mom_bank_kv_grouped(*args, **kwargs):
    from .hip_bank import mom_bank_kv_grouped as _grouped
    return _grouped(*args, **kwargs)


def mom_linear(*args, **kwargs):
    from .hip_linear import mom_linear as _linear
    return _linear(*args, **kwargs)


def mom_rezero(*args, **kwargs):
    from .hip_rezero import mom_rezero as _rezero
    return _rezero(*args, **kwargs)


def mom_gated_linear(*args, **kwargs):
    from .hip_rezero import mom_gated_linear as _gated
    return _gated(*args, **kwargs)


def quantize_bank_fp8(*args, **kwargs):
    from .hip_decode import quantize_bank_fp8 as _quant
    return _quant(*args, **kwargs)


def decode_step(*args, **kwargs):
    from .hip_decode import decode_step as _step
    return _step(*args, **kwargs)
