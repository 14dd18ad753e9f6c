"""Autograd binding of the bank K/V projection (C ABI: naylis_mom_bank_kv_*).

Replaces the two ``nn.Linear`` calls of model.py:253-256
(``k_proj(M_blocks.view(L, D))``, ``v_proj(...)``) with one MFMA launch;
gradients flow to M_blocks, k_proj.weight and v_proj.weight.
"""
from __future__ import annotations

import torch

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


class MomBankKVFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, slots_in, w_k_in, w_v_in):
        # bf16 operands are made here, outside autograd, so the gradients can
        # be produced directly in the parameters' own dtype (fp32 master
        # weights keep fp32 gradients with no bf16 round trip).
        lib = _lib.load()
        slots_grad_dtype = slots_in.dtype if slots_in.dtype in _DT else torch.float32
        w_grad_dtype = w_k_in.dtype if w_k_in.dtype in _DT else torch.float32
        slots = slots_in.to(torch.bfloat16).contiguous()
        w_k = w_k_in.to(torch.bfloat16).contiguous()
        w_v = w_v_in.to(torch.bfloat16).contiguous()
        L, D_in = slots.shape
        D_out = w_k.shape[0]
        dev = slots.device
        k = torch.empty((L, D_out), device=dev, dtype=torch.bfloat16)
        v = torch.empty((L, D_out), device=dev, dtype=torch.bfloat16)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_bank_kv_fwd(slots.data_ptr(), w_k.data_ptr(), w_v.data_ptr(), k.data_ptr(),
                                            v.data_ptr(), L, D_in, D_out, _lib.stream_of(dev))
        _lib.check(rc)
        ctx.save_for_backward(slots, w_k, w_v)
        ctx.gdt = (slots_grad_dtype, w_grad_dtype)
        return k, v

    @staticmethod
    def backward(ctx, dk, dv):
        lib = _lib.load()
        slots, w_k, w_v = ctx.saved_tensors
        sdt, wdt = ctx.gdt
        L, D_in = slots.shape
        D_out = w_k.shape[0]
        dev = slots.device
        dk = torch.zeros((L, D_out), device=dev, dtype=torch.bfloat16) if dk is None else dk.to(torch.bfloat16).contiguous()
        dv = torch.zeros((L, D_out), device=dev, dtype=torch.bfloat16) if dv is None else dv.to(torch.bfloat16).contiguous()
        d_slots = torch.empty((L, D_in), device=dev, dtype=sdt)
        dw_k = torch.empty((D_out, D_in), device=dev, dtype=wdt)
        dw_v = torch.empty((D_out, D_in), device=dev, dtype=wdt)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_bank_kv_bwd(slots.data_ptr(), w_k.data_ptr(), w_v.data_ptr(), dk.data_ptr(),
                                            dv.data_ptr(), d_slots.data_ptr(), _DT[sdt], dw_k.data_ptr(),
                                            dw_v.data_ptr(), _DT[wdt], L, D_in, D_out, _lib.stream_of(dev))
        _lib.check(rc)
        return d_slots, dw_k, dw_v


def mom_bank_kv(M_blocks, w_k, w_v, mem_slots=None):
    """K, V = slots W_k^T, slots W_v^T with slots = M_blocks.view(L, D) (bf16 MFMA,
    fp32 accumulation, bf16 outputs).  fp32 parameters are cast to bf16 for
    the product, as autocast does; their gradients come back in their own
    dtype."""
    D_in = w_k.shape[1]
    if w_k.shape != w_v.shape:
        raise RuntimeError(f"mom_bank_kv: k/v weights differ in shape {tuple(w_k.shape)} vs {tuple(w_v.shape)}")
    if M_blocks.numel() % D_in != 0:
        raise RuntimeError(f"mom_bank_kv: bank of {M_blocks.numel()} values is not a whole number of {D_in}-wide slots")
    slots = M_blocks.reshape(-1, D_in)
    if mem_slots is not None and slots.shape[0] != mem_slots:
        raise RuntimeError(f"mom_bank_kv: bank holds {slots.shape[0]} slots, layer expects {mem_slots}")
    if slots.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"mom_bank_kv: needs a ROCm device tensor, got {slots.device}")
    return MomBankKVFunction.apply(slots, w_k, w_v)
