"""Fused SwiGLU of the decoder MLP (C ABI: naylis_mom_swiglu_*).

transformers' LlamaMLP (inside each Naylis decoder layer, model.py:279-345)
computes ``down(silu(gate(x)) * up(x))``; the activation and the product are
two elementwise launches forward and three backward.  ``swiglu`` does them in
one library pass each way; ``NaylisMLP`` is LlamaMLP with it (same
parameters).
"""
from __future__ import annotations

import torch
from transformers.models.llama.modeling_llama import LlamaMLP

from .. import _lib
from .hip_linear import shared_input_linear

_DT = {torch.float32: 0, torch.bfloat16: 1}


def swiglu_supported(g, u):
    return (torch.version.hip is not None and g.is_cuda and g.dtype in _DT and u.dtype == g.dtype
            and u.shape == g.shape and u.device == g.device and g.numel() % 8 == 0)


class SwiGLUFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, g, u):
        lib = _lib.load()
        g = g.contiguous()
        u = u.contiguous()
        h = torch.empty_like(g)
        with _lib.on_device(g.device):
            _lib.check(lib.naylis_mom_swiglu_fwd(g.data_ptr(), u.data_ptr(), h.data_ptr(), _DT[g.dtype], g.numel(),
                                                 _lib.stream_of(g.device)))
        ctx.save_for_backward(g, u)
        return h

    @staticmethod
    def backward(ctx, dh):
        lib = _lib.load()
        g, u = ctx.saved_tensors
        dh = dh.to(g.dtype).contiguous()
        dg = torch.empty_like(g)
        du = torch.empty_like(u)
        with _lib.on_device(g.device):
            _lib.check(lib.naylis_mom_swiglu_bwd(g.data_ptr(), u.data_ptr(), dh.data_ptr(), dg.data_ptr(),
                                                 du.data_ptr(), _DT[g.dtype], g.numel(), _lib.stream_of(g.device)))
        return dg, du


def swiglu(g, u):
    """silu(g) * u in one pass; raises when ``swiglu_supported`` is false."""
    if not swiglu_supported(g, u):
        raise RuntimeError(f"swiglu: unsupported inputs {tuple(g.shape)} {g.dtype} / {tuple(u.shape)} {u.dtype} "
                           f"on {g.device}")
    return SwiGLUFunction.apply(g, u)


class NaylisMLP(LlamaMLP):
    """LlamaMLP with the fused activation where it applies (SiLU, ROCm,
    bf16 / fp32); transformers' forward otherwise."""

    def forward(self, x):
        if self.config.hidden_act != "silu":
            return super().forward(x)
        g, u = shared_input_linear(x, (self.gate_proj, self.up_proj))
        if not swiglu_supported(g, u):
            return self.down_proj(self.act_fn(g) * u)
        return self.down_proj(swiglu(g, u))
