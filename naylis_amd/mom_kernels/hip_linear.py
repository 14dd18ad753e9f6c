"""Autograd binding of the layer's bias-free q/o projections with the weight
gradient on the library's split-K MFMA GEMM (C ABI: naylis_mom_linear_wgrad).

model.py:239 (`q_proj`) and model.py:251 (`o_proj`) are nn.Linear(d, d,
bias=False); the reference takes their weight gradient from autograd, a
dy^T x reduction over all B*T tokens.  Here the forward product and the input
gradient stay torch GEMMs (hipBLASLt); the weight gradient is
naylis_mom_linear_wgrad, deterministic (fixed-order split-K reduction).

The decoder trunk's projections (the Llama attention's q/k/v/o and the MLP's
gate/up/down inside every Naylis decoder layer, model.py:279-345) are the same
bias-free nn.Linear; ``NaylisLinear`` / ``use_library_wgrad`` give them this
weight gradient too.  At the config-3 shapes (16384 tokens) hipBLASLt's
weight-gradient GEMM runs d x d at about 340 TFLOP/s and d x 2816 at about
620, the library's split-K kernel at about 680 and 750.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


def _library_wgrad(x2, dy2, weight):
    """dW = dy2^T x2 (rows = tokens) on the library's split-K GEMM."""
    lib = _lib.load()
    D_out, D_in = weight.shape
    N = x2.shape[0]
    dev = x2.device
    ws = torch.empty(lib.naylis_mom_linear_wgrad_workspace_bytes(N, D_in, D_out), device=dev, dtype=torch.uint8)
    dw = torch.empty((D_out, D_in), device=dev, dtype=weight.dtype)
    with _lib.on_device(dev):
        rc = lib.naylis_mom_linear_wgrad(x2.data_ptr(), dy2.data_ptr(), dw.data_ptr(), _DT[weight.dtype],
                                         ws.data_ptr(), ws.numel(), N, D_in, D_out, _lib.stream_of(dev))
    _lib.check(rc)
    return dw


def library_wgrad(lib, xin, dy, dtype, dev, st):
    """dW = dy^T xin over all rows (C ABI naylis_mom_linear_wgrad; its split-K
    kernel needs N, D_in, D_out multiples of 8 — otherwise the torch product
    that autograd would use for nn.Linear's weight gradient)."""
    N, D_in = xin.shape
    D_out = dy.shape[1]
    if N % 8 or D_in % 8 or D_out % 8:
        if dtype == torch.float32:
            return torch.mm(dy.t(), xin, out_dtype=torch.float32)
        return torch.mm(dy.t(), xin).to(dtype)
    ws = torch.empty(max(int(lib.naylis_mom_linear_wgrad_workspace_bytes(N, D_in, D_out)), 1), dtype=torch.uint8,
                     device=dev)
    dw = torch.empty((D_out, D_in), device=dev, dtype=dtype)
    _lib.check(lib.naylis_mom_linear_wgrad(xin.data_ptr(), dy.data_ptr(), dw.data_ptr(),
                                           _DT[dtype], ws.data_ptr(), ws.numel(),
                                           N, D_in, D_out, st))
    return dw


class MomLinearFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, weight):
        ctx.save_for_backward(x, weight)
        return F.linear(x, weight)

    @staticmethod
    def backward(ctx, dy):
        x, weight = ctx.saved_tensors
        D_out, D_in = weight.shape
        dy2 = dy.reshape(-1, D_out).contiguous()
        dx = None
        if ctx.needs_input_grad[0]:
            dx = torch.mm(dy2, weight).view(x.shape)
        dw = None
        if ctx.needs_input_grad[1]:
            dw = _library_wgrad(x.reshape(-1, D_in).contiguous(), dy2, weight)
        return dx, dw


def mom_linear(x, weight):
    """y = x W^T (no bias).  For bf16 activations and weights on a ROCm device
    with dimensions that are multiples of 8 the weight gradient runs on the
    library's GEMM; any other combination is the plain torch linear."""
    D_out, D_in = weight.shape
    if (x.is_cuda and torch.version.hip is not None and x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16
            and D_in % 8 == 0 and D_out % 8 == 0 and (x.numel() // D_in) % 8 == 0 and torch.is_grad_enabled()
            and weight.requires_grad):
        return MomLinearFunction.apply(x, weight)
    return F.linear(x, weight)


def _library_ok(x, weight):
    D_out, D_in = weight.shape
    return (x.is_cuda and torch.version.hip is not None and x.dtype == torch.bfloat16
            and weight.dtype == torch.bfloat16 and weight.device == x.device and D_in % 8 == 0 and D_out % 8 == 0
            and x.shape[-1] == D_in and (x.numel() // D_in) % 8 == 0)


class SharedInputLinearFunction(torch.autograd.Function):
    """y_i = x W_i^T for several bias-free projections of one input (the
    attention's q/k/v, the MLP's gate/up).  Autograd would sum their input
    gradients with separate elementwise adds; here each further product
    accumulates into the first in the GEMM's epilogue (``addmm_``, one
    rounding of the sum).  Weight gradients: the library's split-K GEMM."""

    @staticmethod
    def forward(ctx, x, *weights):
        ctx.save_for_backward(x, *weights)
        return tuple(F.linear(x, w) for w in weights)

    @staticmethod
    def backward(ctx, *dys):
        x, *weights = ctx.saved_tensors
        x2 = x.reshape(-1, x.shape[-1]).contiguous() if any(ctx.needs_input_grad[1:]) else None
        dx, dws = None, []
        for i, (dy, w) in enumerate(zip(dys, weights)):
            dy2 = dy.reshape(-1, w.shape[0]).contiguous()
            if ctx.needs_input_grad[0]:
                dx = torch.mm(dy2, w) if dx is None else dx.addmm_(dy2, w)
            dws.append(_library_wgrad(x2, dy2, w) if ctx.needs_input_grad[1 + i] else None)
        return (dx.view(x.shape) if dx is not None else None, *dws)


def shared_input_linear(x, linears):
    """The outputs of several bias-free linear layers applied to one input,
    as a tuple.  One autograd node (``SharedInputLinearFunction``) for bf16
    activations and weights on a ROCm device with dimensions that are
    multiples of 8; otherwise each layer applied in turn."""
    if (torch.is_grad_enabled() and all(m.bias is None and _library_ok(x, m.weight) for m in linears)
            and any(m.weight.requires_grad for m in linears)):
        return SharedInputLinearFunction.apply(x, *(m.weight for m in linears))
    return tuple(m(x) for m in linears)


class NaylisLinear(nn.Linear):
    """nn.Linear (same parameters and state-dict keys) whose bias-free form
    runs through ``mom_linear``; with a bias it is nn.Linear's forward."""

    def forward(self, x):
        if self.bias is not None:
            return super().forward(x)
        return mom_linear(x, self.weight)


def use_library_wgrad(module):
    """Turn every bias-free nn.Linear inside ``module`` into a NaylisLinear in
    place (its parameters are untouched).  Returns ``module``."""
    for m in module.modules():
        if type(m) is nn.Linear and m.bias is None:
            m.__class__ = NaylisLinear
    return module
