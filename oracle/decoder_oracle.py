"""Eager CPU restatement of the Naylis decoder (model.py:279-567).

TEST INFRASTRUCTURE ONLY: the checker for ``naylis_amd.decoder``.  The
module tree mirrors the reference's parameter names (``model.embed_tokens``,
``model.layers.<i>.{self_attn,mlp,input_layernorm,mom_norm,
post_attention_layernorm,mom}``, ``model.M_blocks``, ``model.norm``, tied
``lm_head``) so a product state dict loads with ``strict=True``; the
arithmetic is written out here in plain torch (no transformers code):

* RMSNorm as LlamaRMSNorm: fp32 mean of squares, rsqrt(var + eps), cast back,
  times the weight.
* RoPE: inverse frequencies theta^(-2i/hd), cos/sin of pos * inv_freq
  repeated over both halves, q' = q cos + rotate_half(q) sin.
* Causal softmax attention with an explicit triangular mask.
* SwiGLU MLP: down(silu(gate(x)) * up(x)).
* MoM read: ``OracleMoMLayer`` / ``layer_forward`` (mom_oracle.py).
* Loss: sum cross-entropy of the shifted logits / number of valid labels,
  plus aux_weight * (mean over layers of the load-balance term) in training.

Pinning: with every ``mom_scale`` = 0 (the ReZero init) the decoder is a
stock Llama, which the tests check against transformers' LlamaForCausalLM on
the same weights; the MoM term itself is pinned by the layer oracle.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .mom_oracle import OracleMoMLayer, aux_loss, layer_forward

__all__ = ["OracleDecoder", "rms_norm", "rope_cos_sin", "apply_rope"]


def rms_norm(x, weight, eps):
    """LlamaRMSNorm (transformers modeling_llama, used at model.py:304)."""
    x32 = x.float()
    var = x32.pow(2).mean(-1, keepdim=True)
    return weight * (x32 * torch.rsqrt(var + eps)).to(x.dtype)


def rope_cos_sin(seq_len, head_dim, theta, dtype=torch.float32):
    """Default RoPE tables: (S, hd) cos and sin, frequencies repeated over both halves."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    pos = torch.arange(seq_len, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(t, cos, sin):
    """t (B, H, S, hd): t cos + rotate_half(t) sin, rotate_half(a|b) = (-b|a)."""
    half = t.shape[-1] // 2
    rot = torch.cat([-t[..., half:], t[..., :half]], dim=-1)
    return t * cos + rot * sin


class _Attn(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.q_proj = nn.Linear(d, d, bias=False)
        self.k_proj = nn.Linear(d, d, bias=False)
        self.v_proj = nn.Linear(d, d, bias=False)
        self.o_proj = nn.Linear(d, d, bias=False)


class _Mlp(nn.Module):
    def __init__(self, d, ffn):
        super().__init__()
        self.gate_proj = nn.Linear(d, ffn, bias=False)
        self.up_proj = nn.Linear(d, ffn, bias=False)
        self.down_proj = nn.Linear(ffn, d, bias=False)


class _Norm(nn.Module):
    def __init__(self, d):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))


class _Layer(nn.Module):
    def __init__(self, d, h, ffn, mem_size, block_size, top_blocks, rank):
        super().__init__()
        self.self_attn = _Attn(d)
        self.mlp = _Mlp(d, ffn)
        self.input_layernorm = _Norm(d)
        self.post_attention_layernorm = _Norm(d)
        self.mom_norm = _Norm(d)
        self.mom = OracleMoMLayer(d, h, mem_size, block_size, top_blocks, rank)


class _Trunk(nn.Module):
    def __init__(self, vocab, d, n_layers, h, ffn, mem_size, block_size, top_blocks, rank):
        super().__init__()
        self.embed_tokens = nn.Embedding(vocab, d)
        self.M_blocks = nn.Parameter(torch.zeros(mem_size // block_size, block_size * d))
        self.layers = nn.ModuleList([_Layer(d, h, ffn, mem_size, block_size, top_blocks, rank)
                                     for _ in range(n_layers)])
        self.norm = _Norm(d)


class OracleDecoder(nn.Module):
    """Reference decoder restated for the CPU (model.py:279-567), tied LM head."""

    def __init__(self, vocab, d, n_layers, n_heads, ffn, mem_size, block_size, top_blocks, rank, eps=1e-5,
                 rope_theta=500000.0, aux_weight=0.01):
        super().__init__()
        self.model = _Trunk(vocab, d, n_layers, n_heads, ffn, mem_size, block_size, top_blocks, rank)
        self.lm_head = nn.Linear(d, vocab, bias=False)
        self.lm_head.weight = self.model.embed_tokens.weight
        self.n_heads, self.eps, self.theta, self.aux_weight = n_heads, eps, rope_theta, aux_weight
        for layer in self.model.layers:
            layer.mom.noise_scale = 0.0

    def _attention(self, a, x, cos, sin):
        B, S, D = x.shape
        H = self.n_heads
        hd = D // H
        q = a.q_proj(x).view(B, S, H, hd).transpose(1, 2)
        k = a.k_proj(x).view(B, S, H, hd).transpose(1, 2)
        v = a.v_proj(x).view(B, S, H, hd).transpose(1, 2)
        q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        s = (q @ k.transpose(-1, -2)) * hd ** -0.5
        mask = torch.ones(S, S, dtype=torch.bool, device=x.device).triu(1)
        p = torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1)
        o = (p @ v).transpose(1, 2).reshape(B, S, D)
        return a.o_proj(o)

    def forward(self, input_ids, labels=None, noise=None, train=True, routing=None, capture=None):
        """Returns (loss or None, logits of the full sequence, aux term).
        ``noise``: optional list (one per layer) of additive router noise;
        the aux term enters the loss in training only (model.py:550-561).
        ``routing``: optional list (one per layer) of forced top-k ids;
        ``capture``: optional list that receives each MoM layer's
        (input, output, top_idx)."""
        m = self.model
        h = m.embed_tokens(input_ids)
        B, S, D = h.shape
        cos, sin = rope_cos_sin(S, D // self.n_heads, self.theta, h.dtype)  # tables computed on the host
        cos, sin = cos.to(h.device), sin.to(h.device)
        aux_terms = []
        for i, layer in enumerate(m.layers):
            h = h + self._attention(layer.self_attn, rms_norm(h, layer.input_layernorm.weight, self.eps), cos, sin)
            xm = rms_norm(h, layer.mom_norm.weight, self.eps)
            out, probs, idx, _ = layer_forward(xm, layer.mom, m.M_blocks, noise=None if noise is None else noise[i],
                                               force_idx=None if routing is None else routing[i])
            if capture is not None:
                capture.append((xm.detach(), out.detach(), idx.detach()))
            aux_terms.append(aux_loss(probs, idx, layer.mom.num_blocks))
            h = h + out.to(h.dtype)
            x = rms_norm(h, layer.post_attention_layernorm.weight, self.eps)
            h = h + layer.mlp.down_proj(F.silu(layer.mlp.gate_proj(x)) * layer.mlp.up_proj(x))
        h = rms_norm(h, m.norm.weight, self.eps)
        logits = self.lm_head(h)
        aux = torch.stack(aux_terms).mean() if aux_terms else torch.zeros(())
        if labels is None:
            return None, logits, aux
        shift_logits = logits[:, :-1].reshape(-1, logits.shape[-1])
        shift_labels = labels[:, 1:].reshape(-1)
        loss = F.cross_entropy(shift_logits.float(), shift_labels, reduction="sum")
        loss = loss / (shift_labels != -100).sum().clamp_min(1)
        return (loss + self.aux_weight * aux if train else loss), logits, aux
