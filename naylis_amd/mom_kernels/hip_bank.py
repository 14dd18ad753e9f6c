"""Autograd binding of the bank K/V projection (C ABI: naylis_mom_bank_kv_*).

Replaces the two ``nn.Linear`` calls of model.py:253-256
(``k_proj(M_blocks.view(L, D))``, ``v_proj(...)``) with one MFMA launch;
gradients flow to M_blocks, k_proj.weight and v_proj.weight.
"""
from __future__ import annotations

import ctypes

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


def _ptrs(tensors):
    return (ctypes.c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


class MomBankKVGroupedFunction(torch.autograd.Function):
    """K_i, V_i of n layers that project one bank (naylis_mom_bank_kv_*_grouped):
    inputs (slots, w_k_0, w_v_0, w_k_1, w_v_1, ...), outputs (k_0, v_0, k_1, ...).
    The backward adds every layer's bank gradient in one fp32 accumulation."""

    @staticmethod
    def forward(ctx, slots_in, *weights):
        lib = _lib.load()
        n = len(weights) // 2
        slots_grad_dtype = slots_in.dtype if slots_in.dtype in _DT else torch.float32
        w_grad_dtype = weights[0].dtype if weights[0].dtype in _DT else torch.float32
        slots = slots_in.to(torch.bfloat16).contiguous()
        ws = [w.to(torch.bfloat16).contiguous() for w in weights]
        L, D_in = slots.shape
        D_out = ws[0].shape[0]
        dev = slots.device
        outs = [torch.empty((L, D_out), device=dev, dtype=torch.bfloat16) for _ in range(2 * n)]
        with _lib.on_device(dev):
            rc = lib.naylis_mom_bank_kv_fwd_grouped(slots.data_ptr(), _ptrs(ws[0::2]), _ptrs(ws[1::2]),
                                                    _ptrs(outs[0::2]), _ptrs(outs[1::2]), n, L, D_in, D_out,
                                                    _lib.stream_of(dev))
        _lib.check(rc)
        ctx.save_for_backward(slots, *ws)
        ctx.gdt = (slots_grad_dtype, w_grad_dtype)
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        lib = _lib.load()
        slots, *ws = ctx.saved_tensors
        sdt, wdt = ctx.gdt
        n = len(ws) // 2
        L, D_in = slots.shape
        D_out = ws[0].shape[0]
        dev = slots.device
        g = [torch.zeros((L, D_out), device=dev, dtype=torch.bfloat16) if d is None
             else d.to(torch.bfloat16).contiguous() for d in grads]
        d_slots = torch.empty((L, D_in), device=dev, dtype=sdt)
        dws = [torch.empty((D_out, D_in), device=dev, dtype=wdt) for _ in range(2 * n)]
        nbytes = lib.naylis_mom_bank_kv_bwd_grouped_workspace_bytes(n, L, D_in, D_out)
        wsp = torch.empty(max(nbytes, 1), device=dev, dtype=torch.uint8)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_bank_kv_bwd_grouped(slots.data_ptr(), _ptrs(ws[0::2]), _ptrs(ws[1::2]),
                                                    _ptrs(g[0::2]), _ptrs(g[1::2]), d_slots.data_ptr(), _DT[sdt],
                                                    _ptrs(dws[0::2]), _ptrs(dws[1::2]), _DT[wdt], wsp.data_ptr(),
                                                    wsp.numel(), n, L, D_in, D_out, _lib.stream_of(dev))
        _lib.check(rc)
        return (d_slots, *dws)


GROUP_MAX_LAYERS = 24  # NAYLIS_BANK_GROUP_MAX_LAYERS


def mom_bank_kv_grouped(M_blocks, w_k_list, w_v_list, mem_slots=None):
    """[(K_i, V_i)] for layers i that all project the bank M_blocks: per
    layer the result of ``mom_bank_kv(M_blocks, w_k_list[i], w_v_list[i])``,
    computed in one grouped launch per up to 24 layers (the backward adds the
    bank gradients of a group in one fp32 accumulation).  Shapes the grouped
    GEMM does not take (D_out not a multiple of 64) run layer by layer."""
    if len(w_k_list) != len(w_v_list) or not w_k_list:
        raise RuntimeError("mom_bank_kv_grouped: needs one k and one v weight per layer")
    shape = tuple(w_k_list[0].shape)
    for w in (*w_k_list, *w_v_list):
        if tuple(w.shape) != shape:
            raise RuntimeError(f"mom_bank_kv_grouped: weights differ in shape: {tuple(w.shape)} vs {shape}")
    D_out, D_in = shape
    if D_out % 64 or D_in % 8:
        return [mom_bank_kv(M_blocks, wk, wv, mem_slots) for wk, wv in zip(w_k_list, w_v_list)]
    if M_blocks.numel() % D_in != 0:
        raise RuntimeError(f"mom_bank_kv: bank of {M_blocks.numel()} values is not a whole number of {D_in}-wide slots")
    slots = M_blocks.reshape(-1, D_in)
    if mem_slots is not None and slots.shape[0] != mem_slots:
        raise RuntimeError(f"mom_bank_kv: bank holds {slots.shape[0]} slots, layer expects {mem_slots}")
    if slots.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"mom_bank_kv: needs a ROCm device tensor, got {slots.device}")
    out = []
    for i0 in range(0, len(w_k_list), GROUP_MAX_LAYERS):
        ws = []
        for wk, wv in zip(w_k_list[i0:i0 + GROUP_MAX_LAYERS], w_v_list[i0:i0 + GROUP_MAX_LAYERS]):
            ws += [wk, wv]
        kv = MomBankKVGroupedFunction.apply(slots, *ws)
        out += [(kv[2 * j], kv[2 * j + 1]) for j in range(len(ws) // 2)]
    return out
