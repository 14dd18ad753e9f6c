"""Fused rotary position embedding of the decoder attention (C ABI: naylis_mom_rope).

transformers' ``apply_rotary_pos_emb`` (called by the Llama attention of each
Naylis decoder layer, model.py:279-345) rotates q and k with five elementwise
ops per tensor; ``rope`` does q and k in one library pass each way with the
same roundings (bitwise equal in bf16 and fp32).  ``NaylisAttention`` is the
Llama attention with that rotation, the same parameters and the same
attention backend (SDPA).
"""
from __future__ import annotations

import torch
from transformers.models.llama.modeling_llama import ALL_ATTENTION_FUNCTIONS, LlamaAttention, eager_attention_forward

from .. import _lib
from .hip_linear import shared_input_linear

_DT = {torch.float32: 0, torch.bfloat16: 1}


def _shape_ok(dtype, device, B, S, hd, cos, sin):
    if torch.version.hip is None or device.type != "cuda" or dtype not in _DT or hd not in (32, 64, 128):
        return False
    for t in (cos, sin):
        if t.dtype != dtype or t.device != device or t.dim() != 3 or t.shape[1:] != (S, hd) \
                or t.shape[0] not in (1, B):
            return False
    return True


def rope_supported(q, k, cos, sin):
    """q, k (B, S, H, hd) of one dtype on a ROCm device, hd 32 / 64 / 128,
    cos / sin (1 or B, S, hd) of the same dtype."""
    if q.dim() != 4 or k.shape != q.shape or k.dtype != q.dtype:
        return False
    B, S, _, hd = q.shape
    return _shape_ok(q.dtype, q.device, B, S, hd, cos, sin)


def _launch(q, k, cos, sin, backward):
    lib = _lib.load()
    B, S, H, hd = q.shape
    q = q.contiguous()
    k = k.contiguous()
    cos = cos.contiguous()
    sin = sin.contiguous()
    qo = torch.empty_like(q)
    ko = torch.empty_like(k)
    with _lib.on_device(q.device):
        _lib.check(lib.naylis_mom_rope(q.data_ptr(), k.data_ptr(), cos.data_ptr(), sin.data_ptr(), qo.data_ptr(),
                                       ko.data_ptr(), _DT[q.dtype], int(backward), B, S, H, hd, cos.shape[0],
                                       _lib.stream_of(q.device)))
    return qo, ko


class RopeFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        ctx.save_for_backward(cos, sin)
        return _launch(q, k, cos, sin, False)

    @staticmethod
    def backward(ctx, dq, dk):
        cos, sin = ctx.saved_tensors
        if dq is None:
            dq = torch.zeros_like(dk)
        if dk is None:
            dk = torch.zeros_like(dq)
        gq, gk = _launch(dq, dk, cos, sin, True)
        return gq, gk, None, None


def rope(q, k, cos, sin):
    """(q', k') = rotary embedding of q, k (B, S, H, hd) with cos / sin
    (1 or B, S, hd); raises when ``rope_supported`` is false."""
    if not rope_supported(q, k, cos, sin):
        raise RuntimeError(f"rope: unsupported inputs q {tuple(q.shape)} {q.dtype} on {q.device}, cos "
                           f"{tuple(cos.shape)} {cos.dtype}")
    return RopeFunction.apply(q, k, cos.detach(), sin.detach())


class NaylisAttention(LlamaAttention):
    """LlamaAttention with the fused rotation (no cache: the decoder trains and
    evaluates full sequences); other cases run transformers' forward."""

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                **kwargs):
        B, S, _ = hidden_states.shape
        shape = (B, S, -1, self.head_dim)
        cos, sin = position_embeddings
        same_heads = self.q_proj.out_features == self.k_proj.out_features
        dtype = torch.promote_types(hidden_states.dtype, self.q_proj.weight.dtype)
        if past_key_values is not None or not same_heads or \
                not _shape_ok(dtype, hidden_states.device, B, S, self.head_dim, cos, sin):
            return super().forward(hidden_states, position_embeddings=position_embeddings,
                                   attention_mask=attention_mask, past_key_values=past_key_values, **kwargs)
        q, k, v = shared_input_linear(hidden_states, (self.q_proj, self.k_proj, self.v_proj))
        q, k, v = q.view(shape), k.view(shape), v.view(shape).transpose(1, 2)
        q, k = rope(q, k, cos, sin)
        interface = ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation, eager_attention_forward)
        out, weights = interface(self, q.transpose(1, 2), k.transpose(1, 2), v, attention_mask,
                                 dropout=0.0 if not self.training else self.attention_dropout, scaling=self.scaling,
                                 **kwargs)
        return self.o_proj(out.reshape(B, S, -1).contiguous()), weights
