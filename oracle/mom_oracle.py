"""Eager CPU restatement of the Naylis Mixture-of-Memory (MoM) read.

TEST INFRASTRUCTURE ONLY: the checker for the HIP path (and the timed CPU
baseline in bench.py). The product package ``naylis_amd`` never imports it.

Every function states the reference lines it follows (paths relative to the
OpenRootdev/Naylis tree). All arithmetic is plain torch on the CPU in the
dtype of the inputs (fp32 for the parity oracle, fp64 for the pinning checks),
using the same library routines the reference calls (``torch.cumsum``,
``F.linear``, ``softmax``, ``topk``) so that "restatement == reference" holds
bit-for-bit where the reference's own tests demand it (tests/test_parity.py §1,
§2a).

Pinning (what checks each function, beyond retyping it):

* ``prefix_mean``      — closed form fp32(sum_fp64(x[0..t])) / fp32(t+1),
                         h[:,0] == x[:,0], causality, golden fixtures.
* ``router``           — fp64 evaluation as the decider for top-k indices,
                         softmax identities, golden fixtures.
* ``build_gate_bias``  — brute-force loops incl. duplicate ids, fixtures.
* ``mom_attention``    — brute-force gather over the active slots in fp64,
                         convex-hull and gate-independence invariants,
                         fixtures.
* ``mom_read`` backward— fp64 finite differences, sum_t dlog_gates == 0.
* ``bank_kv``          — fp64 matmul.
* ``layer_forward``    — golden fixtures written from the reference's own
                         ``mom_full_reference`` (tests/golden/make_golden.py).
* ``aux_loss``         — uniform-routing closed form (== 2.0 at top-2) and
                         the scatter formulation.
* ``decode_step``      — equals the last row of the full-sequence read.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

__all__ = [
    "build_gate_bias", "prefix_mean", "router", "mom_attention", "mom_read",
    "bank_kv", "aux_loss", "router_stats", "OracleMoMLayer", "layer_forward",
    "active_tile_blocks", "read_flops_tile_basis", "decode_step",
]


def build_gate_bias(top_idx, top_gates, num_blocks, block_size, mask_dtype):
    """Dense per-token slot bias (B, S, num_blocks*block_size), fp32.

    Follows mom_kernels/reference.py:14-29: log(max(gate, 1e-9)) summed over
    the k selections that hit a block (duplicate ids add), finfo(mask_dtype).min
    on blocks no selection hits, repeated over the block's slots.
    """
    log_gates = top_gates.clamp_min(1e-9).log().float()
    onehot = F.one_hot(top_idx.long(), num_blocks)
    sel = onehot.any(dim=2)
    bias_blocks = torch.einsum("bsk,bske->bse", log_gates, onehot.to(log_gates.dtype))
    bias_blocks = bias_blocks.masked_fill(~sel, float(torch.finfo(mask_dtype).min))
    return bias_blocks.repeat_interleave(block_size, dim=-1)


def prefix_mean(x):
    """Causal prefix mean h_t = mean(x_0..x_t) in fp32.

    Follows mom_kernels/reference.py:32-36 and model.py:169-176: cumsum of
    x.float() over the sequence axis, divided by (t+1) in fp32. On the CPU,
    torch accumulates an fp32 cumsum in fp64 and rounds each prefix once,
    so h == fp32(sum_fp64) / fp32(t+1) exactly.
    """
    cs = torch.cumsum(x.float(), dim=1)
    denom = torch.arange(1, x.shape[1] + 1, device=x.device, dtype=cs.dtype)
    return cs / denom.view(1, -1, 1)


def router(x, w_down, w_up, top_k, noise=None, noise_scale=1.0, force_idx=None):
    """Prefix-mean router: (logits, probs, top_idx, top_gates, h).

    Follows model.py:178-187 (h cast to the router weight dtype, two bias-free
    linears around tanh, ``.float()``) and model.py:209-220 (optional additive
    noise before topk only, softmax probs of the clean logits, topk sorted
    descending, softmax of the selected values). ``noise`` is the
    already-drawn perturbation (the Gumbel sample of model.py:210 or any
    additive logit bias); ``noise_scale`` multiplies it as model.py:211 does.
    ``force_idx`` (B, S, k) replaces the top-k selection (gates are still the
    softmax of the selected noisy logits): whole-model comparisons use it to
    give both sides the same routing when bf16 differences in a layer's input
    move tokens across a selection boundary.
    """
    h = prefix_mean(x).to(w_down.dtype)
    logits = F.linear(torch.tanh(F.linear(h, w_down)), w_up).float()
    noisy = logits if noise is None else logits + noise_scale * noise
    probs = F.softmax(logits, dim=-1)
    if force_idx is None:
        top_values, top_idx = noisy.topk(top_k, dim=-1)
    else:
        top_idx = force_idx.long()
        top_values = noisy.gather(-1, top_idx)
    top_gates = F.softmax(top_values, dim=-1)
    return logits, probs, top_idx, top_gates, h


def mom_attention(q_sh, k, v, bias):
    """Multi-head read of the bank with an additive per-token slot bias.

    Follows mom_kernels/reference.py:39-61 (softmax(q k^T / sqrt(hd) + bias) v,
    not causal over the sequence, shared (L, D) or batched (B, L, D) K/V),
    written as explicit matmuls in the input dtype instead of SDPA so the
    same code runs in fp64 for the pinning checks. The bias is applied in
    the input dtype (reference.py:59 casts it to q's dtype).
    """
    B, S, H, hd = q_sh.shape
    if k.dim() == 2:
        L = k.shape[0]
        kk = k.reshape(1, L, H, hd).transpose(1, 2)
        vv = v.reshape(1, L, H, hd).transpose(1, 2)
    else:
        L = k.shape[1]
        kk = k.reshape(B, L, H, hd).transpose(1, 2)
        vv = v.reshape(B, L, H, hd).transpose(1, 2)
    q = q_sh.transpose(1, 2)                                   # (B, H, S, hd)
    scale = 1.0 / math.sqrt(hd)
    scores = torch.matmul(q, kk.transpose(-1, -2)) * scale
    scores = scores + bias.to(q_sh.dtype).unsqueeze(1)
    p = torch.softmax(scores, dim=-1)
    return torch.matmul(p, vv).transpose(1, 2)


def mom_read(q_sh, k, v, top_idx, top_gates, *, num_blocks, block_size):
    """The structured-routing read: mom_kernels/__init__.py:87-102 semantics.

    Builds the dense bias (reference.py:14-29, fp32) and runs the attention
    (reference.py:39-61). Differentiable in q, k, v and top_gates, which is
    the gradient set the Triton backward returns (triton_gpu.py:409).
    """
    bias = build_gate_bias(top_idx, top_gates, num_blocks, block_size, torch.float32)
    if q_sh.dtype == torch.float64:
        bias = bias.double()
    return mom_attention(q_sh, k, v, bias)


def bank_kv(M_blocks, w_k, w_v):
    """Bank K/V projection, once per layer: model.py:253-256.

    slots = M_blocks.view(L, D); K = slots W_k^T; V = slots W_v^T.
    """
    D = w_k.shape[1]
    slots = M_blocks.reshape(-1, D)
    return F.linear(slots, w_k), F.linear(slots, w_v)


def aux_loss(probs, top_idx, num_blocks):
    """Load-balance aux term of one MoM layer: model.py:476-517
    (``_collect_mom_aux_loss``, the per-layer term at model.py:494-503).

    num_blocks * sum_e frac_selected_e * mean_prob_e, with the selection mask
    built by comparison + any (model.py:498-499).
    """
    probs = probs.reshape(-1, num_blocks).float()
    top_idx = top_idx.reshape(probs.shape[0], -1)
    blocks = torch.arange(num_blocks, device=top_idx.device)
    sel_mask = (top_idx.unsqueeze(2) == blocks.view(1, 1, -1)).any(1)
    frac_selected = sel_mask.to(probs.dtype).mean(dim=0)
    mean_prob = probs.mean(dim=0)
    return num_blocks * (frac_selected * mean_prob).sum()


def router_stats(probs, top_idx, num_blocks):
    """Router entropy and dead-block fraction: model.py:505-507."""
    probs = probs.reshape(-1, num_blocks).float()
    top_idx = top_idx.reshape(probs.shape[0], -1)
    blocks = torch.arange(num_blocks, device=top_idx.device)
    sel_mask = (top_idx.unsqueeze(2) == blocks.view(1, 1, -1)).any(1)
    entropy = -(probs * probs.clamp_min(1e-9).log()).sum(-1).mean()
    dead = (~sel_mask.any(0)).to(probs.dtype).mean()
    return entropy, dead


class OracleMoMLayer(nn.Module):
    """Eager MoM layer with the reference's parameter names.

    Mirrors model.py:71-276 (``MoMLayer``) with the read always on the eager
    path (model.py:262-275): router_down, router_up, q_proj, k_proj, v_proj,
    o_proj, mom_scale, so a state_dict moves between this oracle and the HIP
    layer unchanged.
    """

    def __init__(self, d_model, n_heads, mem_size, block_size, top_blocks, router_rank):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by n_heads ({n_heads})")
        if mem_size % block_size != 0:
            raise ValueError(f"mem_size ({mem_size}) must be a multiple of block_size ({block_size})")
        if top_blocks > mem_size // block_size:
            raise ValueError("top_blocks exceeds the number of memory blocks")
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
        self.noise_scale = 1.0

    def forward(self, x, M_blocks, noise=None):
        out, _, _, _ = layer_forward(x, self, M_blocks, noise=noise)
        return out


def layer_forward(x, layer, M_blocks, noise=None, force_idx=None):
    """Full causal layer forward: mom_kernels/reference.py:64-95.

    Returns (output, router_probs, top_idx, top_gates) with the router stats
    flattened to (B*S, ...) rows as the reference returns them. ``noise`` is
    the additive logit perturbation drawn by the caller (Gumbel in training,
    reference.py:77-79), applied with ``layer.noise_scale``; ``force_idx`` as
    in ``router``.
    """
    B, S, D = x.shape
    q_sh = layer.q_proj(x).view(B, S, layer.n_heads, layer.head_dim)
    _, probs, top_idx, top_gates, _ = router(
        x, layer.router_down.weight, layer.router_up.weight, layer.top_blocks,
        noise=noise, noise_scale=layer.noise_scale, force_idx=force_idx)
    k, v = bank_kv(M_blocks, layer.k_proj.weight, layer.v_proj.weight)
    bias = build_gate_bias(top_idx, top_gates, layer.num_blocks, layer.block_size, q_sh.dtype)
    out = mom_attention(q_sh, k, v, bias)
    out = layer.mom_scale * layer.o_proj(out.reshape(B, S, D))
    return out, probs, top_idx, top_gates


def active_tile_blocks(top_idx, num_blocks, tile=128):
    """A = sum over (b, tile of `tile` tokens) of the number of distinct blocks
    any token of the tile selects — the block-skipping work count of a read
    that tiles tokens by `tile` (the reference's BLOCK_M, triton_gpu.py:50)."""
    B, S, k = top_idx.shape
    n_tiles = (S + tile - 1) // tile
    pad = n_tiles * tile - S
    idx = top_idx.long()
    onehot = F.one_hot(idx, num_blocks).any(dim=2)             # (B, S, E)
    if pad:
        onehot = torch.cat([onehot, onehot.new_zeros(B, pad, num_blocks)], dim=1)
    return int(onehot.view(B, n_tiles, tile, num_blocks).any(dim=2).sum())


def read_flops_tile_basis(top_idx, num_blocks, block_size, d_model, tile=128):
    """Algorithmic read fwd+bwd MFMA FLOP on the tile-active basis:
    14 * d * block_size * tile * A (4 forward + 10 backward flop per
    (token, slot, feature) for QK^T, PV | QK^T, dP, dV, dK, dQ)."""
    A = active_tile_blocks(top_idx, num_blocks, tile)
    return 14.0 * d_model * block_size * tile * A, A


def decode_step(sum_state, t_prev, x_new, w_down, w_up, top_k, q_new, k, v,
                num_blocks, block_size):
    """One decode step of the read with a running prefix-sum state.

    The O(1) form of model.py:172-173: the state holds sum_{s<t} x_s (fp64
    here so it equals the fp32 cumsum the CPU computes), the new token's h is
    fp32(state + x_t) / (t+1), then router + read over its top-k blocks.
    Returns (out (B,H,hd), new_state, top_idx, top_gates).
    """
    B, D = x_new.shape
    state = sum_state.double() + x_new.double()
    denom = (t_prev + 1).to(torch.float32).view(B, 1)
    h = state.float() / denom
    h = h.to(w_down.dtype)
    logits = F.linear(torch.tanh(F.linear(h, w_down)), w_up).float()
    vals, idx = logits.topk(top_k, dim=-1)
    gates = F.softmax(vals, dim=-1)
    H = q_new.shape[1]
    bias = build_gate_bias(idx.view(B, 1, -1), gates.view(B, 1, -1),
                           num_blocks, block_size, torch.float32)
    out = mom_attention(q_new.view(B, 1, H, -1).float(), k.float(), v.float(), bias)
    return out.view(B, H, -1), state, idx, gates
