"""MoMLayer on MI355X: the reference's layer with every hot op on HIP kernels.

Same constructor, parameter names and forward contract as model.py:71-276
(``MoMLayer(d_model, n_heads, mem_size, block_size, top_blocks,
router_rank, use_kernel, mom_grad_ckpt)``; parameters router_down,
router_up, q_proj, k_proj, v_proj, o_proj, mom_scale), so state dicts move
between the two unchanged.  The forward is

    logits, probs, idx, gates = mom_route(x)            # fused router kernel
    K, V  = mom_bank_kv(M_blocks)                       # MFMA bank projection
    out   = mom_read(q_proj(x), K, V, idx, gates)       # gated flash read
    y     = mom_scale * o_proj(out)

q_proj / o_proj run their forward and input gradient as torch GEMMs
(hipBLASLt) and their weight gradient on the library's split-K GEMM.  In the
common training case (bf16 activations and projection weights, no gradient
checkpointing) the whole forward is one autograd node
(``mom_kernels.hip_layer``) whose backward orders the library calls so the
router's input gradient accumulates into the q projection's.  There is one backend: the
HIP kernels (``use_kernel`` is accepted for signature compatibility).  The
eager SDPA path of model.py:262-275 is the parity oracle and lives in
``oracle/``, outside the product.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import mom_kernels
from .mom_kernels.hip_layer import fused_layer_supported, mom_layer

__all__ = ["MoMLayer", "mom_aux_loss"]


def cast_mom_layer(layer, dtype):
    """Cast a MoMLayer for the fused HIP node: the q/k/v/o projections to
    ``dtype``, the router weights and the ReZero scale kept in fp32 (routing
    and the prefix mean run in fp32, model.py:169-187)."""
    for lin in (layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
        lin.to(dtype)
    layer.router_down.float()
    layer.router_up.float()
    layer.mom_scale.data = layer.mom_scale.data.float()
    return layer


class MoMLayer(nn.Module):
    """Mixture-of-Memory read over a shared learnable bank, causal routing."""

    def __init__(self, d_model: int, n_heads: int, mem_size: int, block_size: int, top_blocks: int,
                 router_rank: int, use_kernel: bool = True, mom_grad_ckpt: bool = False):
        super().__init__()
        # contract checks of model.py:125-133
        if d_model % n_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by n_heads ({n_heads})")
        if mem_size % block_size != 0:
            raise ValueError(f"mem_size ({mem_size}) must be a multiple of block_size ({block_size})")
        if top_blocks > mem_size // block_size:
            raise ValueError(
                f"top_blocks ({top_blocks}) exceeds the number of memory blocks "
                f"({mem_size // block_size} = mem_size {mem_size} // block_size {block_size})")
        self.num_blocks = mem_size // block_size
        self.block_size = block_size
        self.top_blocks = top_blocks
        self.mem_slots = mem_size
        self.n_heads = n_heads
        self.head_dim = d_model // n_heads

        self.router_down = nn.Linear(d_model, router_rank, bias=False)
        self.router_up = nn.Linear(router_rank, self.num_blocks, bias=False)
        self.q_proj = nn.Linear(d_model, d_model, bias=False)
        self.k_proj = nn.Linear(d_model, d_model, bias=False)
        self.v_proj = nn.Linear(d_model, d_model, bias=False)
        self.o_proj = nn.Linear(d_model, d_model, bias=False)
        self.mom_scale = nn.Parameter(torch.zeros(1))

        self.last_router_probs = None
        self.last_top_idx = None
        self.last_entropy = None
        self.last_dead_frac = None
        self.noise_scale = 1.0
        self.use_kernel = use_kernel
        self.mom_grad_ckpt = mom_grad_ckpt
        self._kernel_mode = None

    def _resolve_kernel(self, x):
        mode = mom_kernels.resolve_mode(x.device, x.dtype, head_dim=self.head_dim)
        mom_kernels.announce(mode)
        return mode

    def route(self, x, noise=None, noise_is_uniform=False):
        """Router outputs (logits, probs, top_idx, top_gates) — model.py:207-220.
        ``noise``: additive logit noise, or with ``noise_is_uniform`` the
        uniform draw that the kernel turns into the Gumbel sample."""
        return mom_kernels.mom_route(x, self.router_down.weight, self.router_up.weight, self.top_blocks,
                                     noise=noise, noise_scale=self.noise_scale, noise_is_uniform=noise_is_uniform)

    def forward(self, x, M_blocks, bank_kv=None):
        """``bank_kv``: this layer's (K, V) of the bank, when the caller
        projected the bank for several layers at once
        (``mom_kernels.mom_bank_kv_grouped``); else the layer projects
        M_blocks itself."""
        B, S, D = x.shape
        if self._kernel_mode is None:
            self._kernel_mode = self._resolve_kernel(x)
        noise = None
        if self.training and self.noise_scale > 0:
            # the uniform draw of model.py:210 (torch.rand_like of the fp32 logits: same shape,
            # dtype and position in the RNG stream); the router kernel applies
            # g = -log(-log(u + 1e-9) + 1e-9) and logits + noise_scale * g
            noise = torch.rand((B, S, self.num_blocks), device=x.device, dtype=torch.float32)
        ckpt = self.mom_grad_ckpt and self.training and torch.is_grad_enabled()
        if not ckpt and fused_layer_supported(x, M_blocks, self.router_down.weight, self.router_up.weight,
                                              self.q_proj.weight, self.k_proj.weight, self.v_proj.weight,
                                              self.o_proj.weight, self.mom_scale, bank_kv):
            # one autograd node for router + bank + q + read + o + ReZero
            y, router_probs, top_idx = mom_layer(
                x, M_blocks, self.router_down.weight, self.router_up.weight, self.q_proj.weight,
                self.k_proj.weight, self.v_proj.weight, self.o_proj.weight, self.mom_scale,
                n_heads=self.n_heads, num_blocks=self.num_blocks, block_size=self.block_size,
                top_k=self.top_blocks, noise=noise, noise_scale=self.noise_scale, noise_is_uniform=True,
                bank_kv=bank_kv)
            if self.training:
                # plain attributes (not parameters, buffers or modules): set
                # without nn.Module.__setattr__'s registry checks
                self.__dict__["last_router_probs"] = router_probs.reshape(-1, self.num_blocks)
                self.__dict__["last_top_idx"] = top_idx.reshape(-1, self.top_blocks)
            return y
        _, router_probs, top_idx, top_gates = self.route(x, noise, noise_is_uniform=True)
        if self.training:
            self.last_router_probs = router_probs.reshape(-1, self.num_blocks)
            self.last_top_idx = top_idx.reshape(-1, self.top_blocks)
        k, v = bank_kv if bank_kv is not None else (None, None)
        if ckpt:
            out = torch.utils.checkpoint.checkpoint(
                self._read, x, top_idx, top_gates, M_blocks, k, v, use_reentrant=False, preserve_rng_state=False)
        else:
            out = self._read(x, top_idx, top_gates, M_blocks, k, v)
        # o projection and ReZero gate (model.py:251, 239): one GEMM, the gate folded into the weight
        return mom_kernels.mom_gated_linear(out, self.o_proj.weight, self.mom_scale)

    def _read(self, x, top_idx, top_gates, M_blocks, k=None, v=None):
        """q projection, bank K/V (unless given), gated flash read (model.py:241-274)."""
        B, S, D = x.shape
        q_sh = mom_kernels.mom_linear(x, self.q_proj.weight).view(B, S, self.n_heads, self.head_dim)
        if k is None:
            k, v = mom_kernels.mom_bank_kv(M_blocks, self.k_proj.weight, self.v_proj.weight, mem_slots=self.mem_slots)
        out = mom_kernels.mom_read(q_sh, k, v, top_idx, top_gates, num_blocks=self.num_blocks,
                                   block_size=self.block_size, mode=self._kernel_mode)
        return out.reshape(B, S, D)


def mom_aux_loss(layers):
    """Load-balance aux loss averaged over MoM layers, plus per-layer router
    entropy / dead-block fraction — model.py:476-517 (`_collect_mom_aux_loss`).
    Each layer's statistics come from one library pass over the router probs
    and top_idx it stashed (``mom_kernels.mom_router_stats``); the aux gradient
    returns to the router as one row per layer, never an (N, E) tensor."""
    aux = None
    count = 0
    for m in layers:
        if not isinstance(m, MoMLayer) or m.last_router_probs is None or m.last_top_idx is None:
            continue
        E = m.num_blocks
        stats = mom_kernels.mom_router_stats(m.last_router_probs, m.last_top_idx)
        term = stats[2 * E]
        aux = term if aux is None else aux + term
        m.last_entropy = stats[2 * E + 1].detach()
        m.last_dead_frac = stats[2 * E + 2].detach()
        m.last_router_probs = None
        m.last_top_idx = None
        count += 1
    if count == 0:
        return torch.zeros(())
    return aux / count
