"""Autograd binding of the layer's ReZero output gate (C ABI naylis_mom_rezero_*).

model.py:239 returns ``self.mom_scale * out`` (mom_scale: the (1,) parameter
of model.py:151).  Eagerly that is a multiply forward and, backward, a
multiply, a second multiply, a sum and dtype casts; here it is one kernel each
way, with the scale read on the device (no host sync) and d(mom_scale)
reduced in a fixed order.

With the o projection in front of it (model.py:251, then 239), the gate
folds into the projection's weight: s * (out W_o^T) = out (s W_o)^T.  The
layer's fp32 output is then one GEMM with an fp32 result instead of a bf16
GEMM result that is scaled, stored and read back; backward, d out = dy W',
dW' = dy^T out in fp32, and dW_o = s dW', ds = sum(dW' W_o) come from the
ReZero backward kernel run over the weight's elements
(``gated_linear_forward`` / ``gated_linear_backward``, shared by the fused
layer node and ``mom_gated_linear``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib
from .hip_linear import library_wgrad

_DT = {torch.float32: 0, torch.bfloat16: 1}


def gated_linear_forward(lib, out2, w_o, s, st):
    """(y2, w_os): y2 = out2 (s W_o)^T in fp32 and the scaled bf16 weight w_os."""
    w_os = torch.empty_like(w_o)
    _lib.check(lib.naylis_mom_rezero_scale(w_o.data_ptr(), _DT[w_o.dtype], s.data_ptr(), w_os.data_ptr(),
                                           _DT[w_os.dtype], w_o.numel(), st))
    return torch.mm(out2, w_os.t(), out_dtype=torch.float32), w_os


def gated_linear_backward(lib, dy2, out2, w_o, w_os, s, st):
    """(d out2, dW_o, ds) of y2 = out2 (s W_o)^T for the upstream gradient dy2
    (rows = tokens, rounded to bf16 for the two GEMMs)."""
    dev = out2.device
    dy2 = dy2.to(torch.bfloat16).contiguous()
    dout2 = torch.mm(dy2, w_os)
    N, D_in = out2.shape
    D_out = dy2.shape[1]
    if (out2.dtype == torch.bfloat16 and w_o.dtype == torch.bfloat16 and w_o.is_contiguous() and out2.is_contiguous()
            and N % 8 == 0 and D_in % 8 == 0 and D_out % 8 == 0):
        # dW' = dy^T out stays inside the split-K reduction, whose epilogue
        # writes dW_o = s dW' and the partials of ds = sum(dW' W_o)
        ws = torch.empty(max(int(lib.naylis_mom_gated_wgrad_workspace_bytes(N, D_in, D_out)), 1), device=dev,
                         dtype=torch.uint8)
        dw_o = torch.empty_like(w_o)
        ds = torch.empty(1, device=dev, dtype=torch.float32)
        _lib.check(lib.naylis_mom_gated_wgrad(out2.data_ptr(), dy2.data_ptr(), w_o.data_ptr(), s.data_ptr(),
                                              dw_o.data_ptr(), ds.data_ptr(), ws.data_ptr(), ws.numel(), N, D_in,
                                              D_out, st))
        return dout2, dw_o, ds
    dw_s = library_wgrad(lib, out2, dy2, torch.float32, dev, st)
    dw_o = torch.empty_like(w_o)
    ds = torch.empty(1, device=dev, dtype=torch.float32)
    ws = torch.empty(max(int(lib.naylis_mom_rezero_workspace_bytes(w_o.numel())), 1), device=dev, dtype=torch.uint8)
    _lib.check(lib.naylis_mom_rezero_bwd(dw_s.data_ptr(), _DT[dw_s.dtype], w_o.data_ptr(), _DT[w_o.dtype],
                                         s.data_ptr(), dw_o.data_ptr(), ds.data_ptr(), ws.data_ptr(), ws.numel(),
                                         w_o.numel(), st))
    return dout2, dw_o, ds


class MomReZeroFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, z, s):
        lib = _lib.load()
        y = torch.empty(z.shape, device=z.device, dtype=torch.float32)
        with _lib.on_device(z.device):
            rc = lib.naylis_mom_rezero_fwd(z.data_ptr(), _DT[z.dtype], s.data_ptr(), y.data_ptr(), z.numel(),
                                           _lib.stream_of(z.device))
        _lib.check(rc)
        ctx.save_for_backward(z, s)
        return y

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.load()
        z, s = ctx.saved_tensors
        dy = dy.contiguous()
        if dy.dtype not in _DT:
            dy = dy.float()
        dz = torch.empty_like(z) if ctx.needs_input_grad[0] else None
        ds = torch.empty(1, device=z.device, dtype=torch.float32)
        ws = torch.empty(lib.naylis_mom_rezero_workspace_bytes(z.numel()), device=z.device, dtype=torch.uint8)
        with _lib.on_device(z.device):
            rc = lib.naylis_mom_rezero_bwd(dy.data_ptr(), _DT[dy.dtype], z.data_ptr(), _DT[z.dtype], s.data_ptr(),
                                           dz.data_ptr() if dz is not None else None, ds.data_ptr(), ws.data_ptr(),
                                           ws.numel(), z.numel(), _lib.stream_of(z.device))
        _lib.check(rc)
        return dz, ds.view(s.shape).to(s.dtype)


def mom_rezero(z, s):
    """y = s * z for the (1,) fp32 gate s on a ROCm device (one kernel each way);
    any other combination is the eager product."""
    if (z.is_cuda and torch.version.hip is not None and s.dtype == torch.float32 and s.numel() == 1
            and z.dtype in _DT and s.device == z.device and z.is_contiguous()):
        return MomReZeroFunction.apply(z, s)
    return s * z


class MomGatedLinearFunction(torch.autograd.Function):
    """y = s * (out W_o^T) in fp32, as out (s W_o)^T (see the module notes)."""

    @staticmethod
    def forward(ctx, out, w_o, s):
        lib = _lib.load()
        D = w_o.shape[1]
        with _lib.on_device(out.device):
            y2, w_os = gated_linear_forward(lib, out.reshape(-1, D), w_o, s, _lib.stream_of(out.device))
        ctx.save_for_backward(out, w_o, w_os, s)
        return y2.view(*out.shape[:-1], w_o.shape[0])

    @staticmethod
    def backward(ctx, dy):
        lib = _lib.load()
        out, w_o, w_os, s = ctx.saved_tensors
        D = w_o.shape[1]
        with _lib.on_device(out.device):
            dout2, dw_o, ds = gated_linear_backward(lib, dy.reshape(-1, w_o.shape[0]), out.reshape(-1, D), w_o, w_os,
                                                    s, _lib.stream_of(out.device))
        return dout2.view(out.shape), dw_o, ds.view(s.shape)


def mom_gated_linear(out, w_o, s):
    """s * (out W_o^T) for the layer's o projection and ReZero gate
    (model.py:251, 239): one GEMM with the gate folded into the weight, for
    bf16 activations and weight and the (1,) fp32 gate on a ROCm device with
    dimensions that are multiples of 8; any other combination is the eager
    composition."""
    D_out, D_in = w_o.shape
    if (out.is_cuda and torch.version.hip is not None and out.dtype == torch.bfloat16
            and w_o.dtype == torch.bfloat16 and s.dtype == torch.float32 and s.numel() == 1
            and out.device == w_o.device == s.device and out.shape[-1] == D_in and D_in % 8 == 0
            and D_out % 8 == 0 and (out.numel() // D_in) % 8 == 0):
        return MomGatedLinearFunction.apply(out.contiguous(), w_o, s)
    return s * F.linear(out, w_o)
