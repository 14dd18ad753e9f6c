"""Fused RMSNorm of the Naylis decoder (C ABI: naylis_mom_rmsnorm_*).

The reference builds every norm of its decoder layer — the MoM layer's
pre-norm ``mom_norm`` and the Llama block's two norms — as LlamaRMSNorm, or
as Liger's fused RMSNorm with ``use_liger`` (model.py:304-305):
``h = fp32(x) * rsqrt(mean(fp32(x)^2) + eps); y = weight * h.to(x.dtype)``.
``NaylisRMSNorm`` keeps that module's parameter (``weight``) and ``eps`` and
runs forward and backward as one library pass each.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


def rmsnorm_supported(x, weight):
    """True when the fused kernels apply: same-dtype bf16 / fp32 x and weight on
    a ROCm device, D a multiple of 512 in [512, 4096]."""
    D = x.shape[-1]
    return (torch.version.hip is not None and x.is_cuda and x.dtype in _DT and weight.dtype == x.dtype
            and weight.device == x.device and D % 512 == 0 and 512 <= D <= 4096 and weight.shape == (D,))


class RMSNormFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, weight, eps):
        lib = _lib.load()
        D = x.shape[-1]
        x2 = x.contiguous().view(-1, D)
        N = x2.shape[0]
        dev = x.device
        y = torch.empty_like(x2)
        rstd = torch.empty(N, device=dev, dtype=torch.float32)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_rmsnorm_fwd(x2.data_ptr(), _DT[x.dtype], weight.data_ptr(), y.data_ptr(),
                                                  rstd.data_ptr(), N, D, float(eps), _lib.stream_of(dev)))
        ctx.save_for_backward(x2, weight, rstd)
        ctx.shape = x.shape
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.load()
        x2, weight, rstd = ctx.saved_tensors
        N, D = x2.shape
        dev = x2.device
        dy2 = dy.to(x2.dtype).contiguous().view(N, D)
        dx = torch.empty_like(x2)
        dw = torch.empty_like(weight)
        ws = torch.empty(max(lib.naylis_mom_rmsnorm_workspace_bytes(N, D), 1), dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_rmsnorm_bwd(x2.data_ptr(), _DT[x2.dtype], weight.data_ptr(), rstd.data_ptr(),
                                                  dy2.data_ptr(), dx.data_ptr(), dw.data_ptr(), ws.data_ptr(),
                                                  ws.numel(), N, D, _lib.stream_of(dev)))
        return dx.view(ctx.shape), dw, None


def rms_norm(x, weight, eps=1e-6):
    """Fused RMSNorm; raises when ``rmsnorm_supported`` is false."""
    if not rmsnorm_supported(x, weight):
        raise RuntimeError(f"rms_norm: needs bf16 / fp32 x and weight of one dtype on a ROCm device with D a "
                           f"multiple of 512 in [512, 4096]; got x {tuple(x.shape)} {x.dtype} on {x.device}, "
                           f"weight {weight.dtype}")
    return RMSNormFunction.apply(x, weight, float(eps))


class NaylisRMSNorm(nn.Module):
    """Drop-in for LlamaRMSNorm (same ``weight`` parameter and ``eps``,
    ``variance_epsilon`` kept as an alias), computed by the fused kernels."""

    def __init__(self, hidden_size, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x):
        return rms_norm(x, self.weight, self.variance_epsilon)

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.variance_epsilon}"


class AddRMSNormFunction(torch.autograd.Function):
    """(s, y) = (x + a.to(x.dtype), RMSNorm(s)) in one pass each way."""

    @staticmethod
    def forward(ctx, x, a, weight, eps):
        lib = _lib.load()
        D = x.shape[-1]
        x2 = x.contiguous().view(-1, D)
        a2 = a.contiguous().view(-1, D)
        N = x2.shape[0]
        dev = x.device
        s = torch.empty_like(x2)
        y = torch.empty_like(x2)
        rstd = torch.empty(N, device=dev, dtype=torch.float32)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_add_rmsnorm_fwd(x2.data_ptr(), a2.data_ptr(), _DT[a.dtype], weight.data_ptr(),
                                                      s.data_ptr(), y.data_ptr(), rstd.data_ptr(), _DT[x.dtype], N, D,
                                                      float(eps), _lib.stream_of(dev)))
        ctx.save_for_backward(s, weight, rstd)
        ctx.shape = x.shape
        return s.view(x.shape), y.view(x.shape)

    @staticmethod
    def backward(ctx, ds_out, dy):
        lib = _lib.load()
        s, weight, rstd = ctx.saved_tensors
        N, D = s.shape
        dev = s.device
        if dy is None:
            dy = torch.zeros_like(s)
        dy2 = dy.to(s.dtype).contiguous().view(N, D)
        dres = ds_out.to(s.dtype).contiguous().view(N, D) if ds_out is not None else None
        ds = torch.empty_like(s)
        dw = torch.empty_like(weight)
        ws = torch.empty(max(lib.naylis_mom_rmsnorm_workspace_bytes(N, D), 1), dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_add_rmsnorm_bwd(s.data_ptr(), weight.data_ptr(), rstd.data_ptr(), dy2.data_ptr(),
                                                      dres.data_ptr() if dres is not None else None, ds.data_ptr(),
                                                      dw.data_ptr(), ws.data_ptr(), ws.numel(), _DT[s.dtype], N, D,
                                                      _lib.stream_of(dev)))
        ds = ds.view(ctx.shape)
        return ds, ds, dw, None


def add_rms_norm(x, a, norm):
    """Residual add followed by ``norm``: returns (s, norm(s)) with
    s = x + a.to(x.dtype).  One fused pass when ``norm`` is a NaylisRMSNorm and
    the kernels apply (a in x's dtype or fp32), else the two torch steps."""
    if (isinstance(norm, NaylisRMSNorm) and rmsnorm_supported(x, norm.weight) and a.shape == x.shape
            and a.device == x.device and (a.dtype == x.dtype or a.dtype == torch.float32)):
        return AddRMSNormFunction.apply(x, a, norm.weight, float(norm.variance_epsilon))
    s = x + a.to(x.dtype)
    return s, norm(s)
