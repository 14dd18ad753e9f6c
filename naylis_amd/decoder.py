"""The Naylis decoder with its MoM reads on the HIP kernels (model.py:279-567).

The Llama trunk (embedding, RoPE attention, SwiGLU MLP, RMSNorm, LM head) is
transformers' Llama, as in the reference; every decoder layer adds the MoM
read between attention and MLP, pre-normed by ``mom_norm`` and residual-wired,
and all layers read the one bank ``model.M_blocks`` (num_blocks,
block_size * hidden) that the model owns.  Module and parameter names are the
reference's (``model.layers.<i>.mom.*``, ``model.layers.<i>.mom_norm.*``,
``model.M_blocks``), so checkpoints load unchanged (see
``naylis_amd.checkpoint``).

What differs from the reference is where the MoM work runs: ``self.mom`` is
``naylis_amd.layer.MoMLayer`` (router, read, ReZero on the library's kernels,
one autograd node per layer), the bank's K and V for every layer come from one
grouped projection per forward (``mom_kernels.mom_bank_kv_grouped``: one
launch for all layers' K/V, and in the backward one fp32 accumulation of all
layers' bank gradients where the reference sums 20 per-layer gradients in
autograd), and the load-balance aux loss consumes the router probabilities
the layer kernel emits (``naylis_amd.layer.mom_aux_loss``).
There is no eager MoM path: off ROCm the MoM layers raise.  The norms
(``mom_norm``, the block's two norms, the final norm) are the library's fused
RMSNorm (``NaylisRMSNorm``, the role of the reference's ``use_liger`` norm)
when the hidden size is a multiple of 512 up to 4096, LlamaRMSNorm otherwise;
the attention applies the rotary embedding with the library's fused kernel
(``NaylisAttention``, same parameters and SDPA backend), the MLP its fused
SwiGLU (``NaylisMLP``), the bias-free projections of both take their
weight gradient from the library's split-K GEMM (``use_library_wgrad``), and
the LM loss reads the bf16 logits once (``cross_entropy_rows``) when the
vocabulary is a multiple of 2048.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from transformers import LlamaConfig
from transformers.modeling_outputs import BaseModelOutputWithPast, CausalLMOutputWithPast
from transformers.models.llama.modeling_llama import (LlamaDecoderLayer, LlamaForCausalLM, LlamaModel,
                                                      LlamaRMSNorm)

from . import mom_kernels
from .layer import MoMLayer, cast_mom_layer, mom_aux_loss
from .mom_kernels.hip_norm import NaylisRMSNorm, add_rms_norm
from .mom_kernels.hip_linear import use_library_wgrad
from .mom_kernels.hip_mlp import NaylisMLP
from .mom_kernels.hip_rope import NaylisAttention
from .mom_kernels.hip_xent import cross_entropy_rows, xent_supported

__all__ = ["naylis_config", "NaylisDecoderLayer", "NaylisLlamaModel", "NaylisLlamaForCausalLM",
           "cast_for_training"]


def _norm(config):
    """RMSNorm module for the hidden size: the fused library norm where its
    kernels apply (hidden a multiple of 512 in [512, 4096]), else LlamaRMSNorm;
    both hold one ``weight`` (hidden,) and compute the same function."""
    d = config.hidden_size
    if d % 512 == 0 and 512 <= d <= 4096:
        return NaylisRMSNorm(d, eps=config.rms_norm_eps)
    return LlamaRMSNorm(d, eps=config.rms_norm_eps)


def naylis_config(vocab_size=32768, d_model=1024, n_layers=20, n_heads=16, intermediate_size=2816, seq_len=2048,
                  mem_size=1024, mom_block_size=128, mom_top_blocks=2, mom_router_rank=32, mom_aux_weight=0.01,
                  mom_grad_ckpt=False):
    """A LlamaConfig carrying the MoM keys, built as pretrain.py:185-210 builds
    it (rms eps 1e-5, RoPE theta 5e5, tied embeddings, SDPA attention, no
    cache).  The defaults are the 300M-class decoder of config 3."""
    config = LlamaConfig(vocab_size=vocab_size, hidden_size=d_model, intermediate_size=intermediate_size,
                         num_hidden_layers=n_layers, num_attention_heads=n_heads, num_key_value_heads=n_heads,
                         max_position_embeddings=seq_len, rms_norm_eps=1e-5, rope_theta=500000.0,
                         attention_bias=False, tie_word_embeddings=True, attn_implementation="sdpa",
                         use_cache=False)
    config.variant = "naylis"
    config.mem_size = mem_size
    config.mom_block_size = mom_block_size
    config.mom_top_blocks = mom_top_blocks
    config.mom_router_rank = mom_router_rank
    config.mom_aux_weight = mom_aux_weight
    config.mom_grad_ckpt = mom_grad_ckpt
    return config


class NaylisDecoderLayer(LlamaDecoderLayer):
    """Llama block + MoM read between attention and MLP (model.py:279-345):

        h = h + attn(input_layernorm(h))
        h = h + mom(mom_norm(h), M_blocks)
        h = h + mlp(post_attention_layernorm(h))

    With ``mom_grad_ckpt`` the attention and the MLP run in checkpoint
    regions (no RNG inside either, so the recompute is exact) and the MoM
    layer checkpoints its read.

    Every residual add is followed by a norm (the next sub-block's, or the
    next layer's ``input_layernorm``, or the final norm), so the layer hands
    its MLP output on un-added (``pending``) and each add runs fused with the
    norm after it (``add_rms_norm``): forward(h, M, pos, pending) returns
    (h, mlp_out); h + mlp_out is the reference layer's output.
    """

    def __init__(self, config, layer_idx, mem_size, mom_block_size, mom_top_blocks, mom_router_rank,
                 mom_grad_ckpt=False):
        super().__init__(config, layer_idx)
        self.self_attn = use_library_wgrad(NaylisAttention(config, layer_idx))
        self.mlp = use_library_wgrad(NaylisMLP(config))
        self.input_layernorm = _norm(config)
        self.post_attention_layernorm = _norm(config)
        self.mom_norm = _norm(config)
        self.mom = MoMLayer(d_model=config.hidden_size, n_heads=config.num_attention_heads, mem_size=mem_size,
                            block_size=mom_block_size, top_blocks=mom_top_blocks, router_rank=mom_router_rank,
                            mom_grad_ckpt=mom_grad_ckpt)
        self._grad_ckpt = mom_grad_ckpt

    def _maybe_ckpt(self, fn, *tensors):
        if self._grad_ckpt and self.training and torch.is_grad_enabled():
            return torch.utils.checkpoint.checkpoint(fn, *tensors, use_reentrant=False, preserve_rng_state=False)
        return fn(*tensors)

    def forward(self, hidden_states, M_blocks=None, position_embeddings=None, pending=None, bank_kv=None,
                **kwargs):
        if M_blocks is None:
            raise ValueError("M_blocks is required: the MoM layer cannot run without the shared memory bank")
        h = hidden_states
        if pending is None:
            x = self.input_layernorm(h)
        else:
            h, x = add_rms_norm(h, pending, self.input_layernorm)
        a = self._maybe_ckpt(lambda t: self.self_attn(hidden_states=t, position_embeddings=position_embeddings,
                                                      **kwargs)[0], x)
        h, x = add_rms_norm(h, a, self.mom_norm)
        # the ReZero product promotes to the fp32 scale's dtype; the add rounds
        # it to the residual stream's (bf16 in bf16 training, fp32 under autocast)
        h, x = add_rms_norm(h, self.mom(x, M_blocks, bank_kv), self.post_attention_layernorm)
        return h, self._maybe_ckpt(self.mlp, x)


class NaylisLlamaModel(LlamaModel):
    """Llama backbone owning the bank shared by every layer (model.py:348-420)."""

    def __init__(self, config, mem_size, mom_block_size, mom_top_blocks, mom_router_rank, mom_grad_ckpt=False):
        super().__init__(config)
        if mem_size % mom_block_size:
            raise ValueError(f"mem_size ({mem_size}) must be a multiple of mom_block_size ({mom_block_size})")
        num_blocks = mem_size // mom_block_size
        self.M_blocks = nn.Parameter(torch.randn(num_blocks, mom_block_size * config.hidden_size) * 0.02)
        self.norm = _norm(config)
        self.layers = nn.ModuleList([
            NaylisDecoderLayer(config, i, mem_size, mom_block_size, mom_top_blocks, mom_router_rank, mom_grad_ckpt)
            for i in range(config.num_hidden_layers)])

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, inputs_embeds=None, **kwargs):
        """The attention mask, if any, goes to the attention as given (the MoM
        read is causal over the whole sequence and takes no mask)."""
        h = self.embed_tokens(input_ids) if inputs_embeds is None else inputs_embeds
        B, S = h.shape[:2]
        if position_ids is None:
            position_ids = torch.arange(S, device=h.device).unsqueeze(0).expand(B, -1)
        pos = self.rotary_emb(h, position_ids)
        # every layer projects the one bank (model.py:409-416, 253-256): one grouped launch for all
        # layers' K and V, and one accumulation of their bank gradients in the backward
        moms = [layer.mom for layer in self.layers]
        kv = mom_kernels.mom_bank_kv_grouped(self.M_blocks, [m.k_proj.weight for m in moms],
                                             [m.v_proj.weight for m in moms], mem_slots=moms[0].mem_slots)
        pending = None
        for layer, bank_kv in zip(self.layers, kv):
            h, pending = layer(h, M_blocks=self.M_blocks, position_embeddings=pos, pending=pending,
                               bank_kv=bank_kv, attention_mask=attention_mask, **kwargs)
        out = self.norm(h) if pending is None else add_rms_norm(h, pending, self.norm)[1]
        return BaseModelOutputWithPast(last_hidden_state=out)


class NaylisLlamaForCausalLM(LlamaForCausalLM):
    """LM head, next-token cross-entropy and the MoM load-balance aux loss
    (model.py:423-567): loss = CE_sum / n_valid (or / num_items_in_batch)
    + mom_aux_weight * aux, the aux term added in training mode only."""

    def __init__(self, config, mem_size=None, mom_block_size=None, mom_top_blocks=None, mom_router_rank=None,
                 mom_aux_weight=None, mom_grad_ckpt=None):
        super().__init__(config)

        def pick(value, name, default=None):
            return getattr(config, name, default) if value is None else value

        self.model = NaylisLlamaModel(config, pick(mem_size, "mem_size"), pick(mom_block_size, "mom_block_size"),
                                      pick(mom_top_blocks, "mom_top_blocks"), pick(mom_router_rank, "mom_router_rank"),
                                      bool(pick(mom_grad_ckpt, "mom_grad_ckpt", False)))
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight
        self.mom_aux_weight = float(pick(mom_aux_weight, "mom_aux_weight"))
        self.mom_aux_normalize = False
        self.mom_aux_accum_steps = None
        self.last_aux_loss = None
        self.post_init()

    def set_noise_scale(self, scale):
        """Gumbel scale of every router (the reference's annealing hook)."""
        for layer in self.model.layers:
            layer.mom.noise_scale = float(scale)

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, labels=None, num_items_in_batch=None,
                **kwargs):
        h = self.model(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                       **kwargs).last_hidden_state
        if labels is None:
            return CausalLMOutputWithPast(loss=None, logits=self.lm_head(h))
        shift_h = h[:, :-1, :].contiguous()
        shift_labels = labels[:, 1:].contiguous().view(-1)
        logits = self.lm_head(shift_h).view(-1, self.config.vocab_size)
        if xent_supported(logits, shift_labels):
            # the library's one-pass loss over the bf16 logits (same sum as below)
            loss = cross_entropy_rows(logits, shift_labels).sum()
        else:
            loss = F.cross_entropy(logits.float(), shift_labels, reduction="sum")
        if num_items_in_batch is not None:
            loss = loss / num_items_in_batch
        else:
            loss = loss / (shift_labels != -100).sum().clamp_min(1)
        if self.training:
            aux = mom_aux_loss(self.modules()).to(loss.device)
            if self.mom_aux_normalize:
                if not self.mom_aux_accum_steps or self.mom_aux_accum_steps < 1:
                    raise RuntimeError("mom_aux_normalize is set but mom_aux_accum_steps is not: the accumulation "
                                       "cycle length is unknown")
                aux = aux / self.mom_aux_accum_steps
            self.last_aux_loss = aux.detach()
            loss = loss + self.mom_aux_weight * aux
        return CausalLMOutputWithPast(loss=loss, logits=None)


def cast_for_training(model, dtype=torch.bfloat16):
    """Cast the model to ``dtype`` except what the MoM layer keeps in fp32 —
    the router weights and the ReZero scale ("routing and the prefix mean are
    in fp32") — so every MoM layer runs as one fused autograd node."""
    model.to(dtype)
    for m in model.modules():
        if isinstance(m, MoMLayer):
            cast_mom_layer(m, dtype)
    return model
