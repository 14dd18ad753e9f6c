"""Autograd binding of the layer's ReZero output gate (C ABI naylis_mom_rezero_*).

model.py:239 returns ``self.mom_scale * out`` (mom_scale: the (1,) parameter
of model.py:151).  Eagerly that is a multiply forward and, backward, a
multiply, a second multiply, a sum and dtype casts; here it is one kernel each
way, with the scale read on the device (no host sync) and d(mom_scale)
reduced in a fixed order.
"""
from __future__ import annotations

import torch

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


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
