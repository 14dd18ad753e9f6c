"""Inference decode step of the MoM read (C ABI naylis_mom_decode_step).

The reference has no decode path (`use_cache=False`, pretrain.py:198): its
router recomputes the causal prefix mean over the whole sequence on every
forward (model.py:169-176), and the O(1) running-sum form is only described
in a docstring (model.py:172-173).  This module is that form: per sequence a
running sum of the tokens so far (fp64, so the prefix mean of the new token
is bit-identical to the full-sequence fp32 cumsum / (t+1)), the fp32 router,
and the gated read of the new token's top-k blocks from a bank whose K / V
are stored as fp8 e4m3 (OCP) with one fp32 scale per slot — one kernel per
step.  The bank projection (mom_bank_kv) and the q projection stay outside.
"""
from __future__ import annotations

from typing import NamedTuple

import torch

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}


class Fp8Bank(NamedTuple):
    """Bank K / V as fp8 e4m3 codes (L, D) uint8 with per-slot fp32 scales (L,):
    k_n = k_scale[n] * e4m3(k8[n]), likewise v."""
    k8: torch.Tensor
    v8: torch.Tensor
    k_scale: torch.Tensor
    v_scale: torch.Tensor

    def dequantize(self):
        """(k, v) fp32 (L, D): the values the decode step reads."""
        k = self.k8.view(torch.float8_e4m3fn).float() * self.k_scale.view(-1, 1)
        v = self.v8.view(torch.float8_e4m3fn).float() * self.v_scale.view(-1, 1)
        return k, v


def quantize_bank_fp8(k, v) -> Fp8Bank:
    """Quantize the bank's (L, D) bf16 K / V once per bank: per slot row
    scale = max|row| / 448, code = e4m3fn(x / scale), round to nearest even."""
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or k.dim() != 2 or k.shape != v.shape:
        raise RuntimeError("quantize_bank_fp8: k and v must be (L, D) bf16 tensors of one shape")
    if not k.is_cuda or v.device != k.device:
        raise RuntimeError("quantize_bank_fp8: k and v must be on one ROCm device")
    lib = _lib.load()
    k, v = k.contiguous(), v.contiguous()
    L, D = k.shape
    dev = k.device
    k8 = torch.empty((L, D), device=dev, dtype=torch.uint8)
    v8 = torch.empty_like(k8)
    ks = torch.empty(L, device=dev, dtype=torch.float32)
    vs = torch.empty_like(ks)
    with _lib.on_device(dev):
        _lib.check(lib.naylis_mom_bank_quant_fp8(k.data_ptr(), v.data_ptr(), k8.data_ptr(), v8.data_ptr(),
                                                 ks.data_ptr(), vs.data_ptr(), L, D, _lib.stream_of(dev)))
    return Fp8Bank(k8, v8, ks, vs)


def decode_step(sum_state, t_prev, x_new, w_down, w_up, top_k, q_new, bank: Fp8Bank, num_blocks, block_size,
                out_state=None):
    """One decode step for B sequences (one new token each).

    sum_state (B, D) fp64: sum of each sequence's earlier tokens; t_prev (B,)
    int: their number; x_new (B, D) bf16 / fp32: the new tokens; w_down
    (R, D), w_up (E, R) fp32 router weights (E = num_blocks); q_new (B, H, hd)
    bf16: the new tokens' queries; bank: the fp8 bank (quantize_bank_fp8).
    Returns (out (B, H, hd) bf16, new_state (B, D) fp64, top_idx (B, top_k)
    int32, top_gates (B, top_k) fp32).  new_state is written to out_state when
    given (it must not be sum_state: every workgroup of a sequence reads the
    old state); the caller ping-pongs two buffers across steps.
    """
    lib = _lib.load()
    if x_new.dim() != 2 or q_new.dim() != 3:
        raise RuntimeError("decode_step: x_new must be (B, D) and q_new (B, H, head_dim)")
    B, D = x_new.shape
    H = q_new.shape[1]
    R, E = w_down.shape[0], w_up.shape[0]
    if E != num_blocks:
        raise RuntimeError(f"decode_step: the router has {E} experts but the bank {num_blocks} blocks")
    if q_new.shape != (B, H, D // H) or q_new.dtype != torch.bfloat16:
        raise RuntimeError("decode_step: q_new must be (B, H, D / H) bf16")
    if x_new.dtype not in _DT:
        raise RuntimeError(f"decode_step: x_new dtype {x_new.dtype} (bf16 or fp32 expected)")
    if bank.k8.shape != (num_blocks * block_size, D):
        raise RuntimeError("decode_step: the bank's shape does not match num_blocks * block_size x D")
    dev = x_new.device
    sum_state = sum_state.to(torch.float64).contiguous()
    t_prev = t_prev.to(device=dev, dtype=torch.int32).contiguous()
    if out_state is None:
        out_state = torch.empty_like(sum_state)
    elif out_state.data_ptr() == sum_state.data_ptr() or out_state.dtype != torch.float64:
        raise RuntimeError("decode_step: out_state must be a separate fp64 buffer")
    x_new = x_new.contiguous()
    q_new = q_new.contiguous()
    w_down = w_down.float().contiguous()
    w_up = w_up.float().contiguous()
    out = torch.empty((B, H, D // H), device=dev, dtype=torch.bfloat16)
    top_idx = torch.empty((B, top_k), device=dev, dtype=torch.int32)
    gates = torch.empty((B, top_k), device=dev, dtype=torch.float32)
    with _lib.on_device(dev):
        _lib.check(lib.naylis_mom_decode_step(
            sum_state.data_ptr(), out_state.data_ptr(), t_prev.data_ptr(), x_new.data_ptr(), _DT[x_new.dtype],
            w_down.data_ptr(), w_up.data_ptr(), q_new.data_ptr(), bank.k8.data_ptr(), bank.v8.data_ptr(),
            bank.k_scale.data_ptr(), bank.v_scale.data_ptr(), out.data_ptr(), top_idx.data_ptr(), gates.data_ptr(),
            B, D, H, R, E, block_size, top_k, _lib.stream_of(dev)))
    return out, out_state, top_idx, gates
