"""Autograd binding of the fused prefix-mean router (C ABI: naylis_mom_router_*).

The reference computes the router with eager torch ops and no kernel boundary
(model.py:169-187, 209-220).  ``mom_route`` returns the same tensors in one
fused launch sequence: (router_logits, router_probs, top_idx, top_gates) and,
on request, the fp32 prefix mean h.  Gradients flow to x, router_down.weight
and router_up.weight from top_gates (the LM path through the read),
router_probs (the aux loss) and router_logits.

``mom_router_stats`` computes the load-balance statistics of a routing
(model.py:476-517) in one library pass; its gradient reaches router_probs as
one (E,) row expanded over the tokens, which the router backward reads with
row stride 0 instead of materialising an (N, E) tensor.
"""
from __future__ import annotations

import torch

from .. import _lib

_DT = {torch.float32: 0, torch.bfloat16: 1}
NOISE_ADDITIVE, NOISE_GUMBEL_UNIFORM = 0, 1


def d_probs_arg(d_probs, E):
    """(tensor kept alive, device pointer, row stride) for the router
    backward's d_probs: an fp32 (..., E) gradient expanded from one row
    (strides 0 except the last) goes in as that row with stride 0; anything
    else as a dense fp32 copy with stride E."""
    if d_probs is None:
        return None, None, E
    if (d_probs.dtype == torch.float32 and d_probs.stride(-1) == 1
            and all(s == 0 for s in d_probs.stride()[:-1])):
        return d_probs, d_probs.data_ptr(), 0
    dense = d_probs.float().contiguous()
    return dense, dense.data_ptr(), E


class MomRouteFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, w_down, w_up, noise, noise_scale, top_k, want_h, noise_kind=NOISE_ADDITIVE):
        lib = _lib.load()
        B, T, D = x.shape
        R, E = w_down.shape[0], w_up.shape[0]
        dev = x.device
        f32 = dict(device=dev, dtype=torch.float32)
        logits = torch.empty((B, T, E), **f32)
        probs = torch.empty((B, T, E), **f32)
        top_idx = torch.empty((B, T, top_k), device=dev, dtype=torch.int32)
        top_gates = torch.empty((B, T, top_k), **f32)
        act = torch.empty((B, T, R), **f32)
        h = torch.empty((B, T, D), **f32) if want_h else None
        nbytes = lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k)
        if nbytes == 0:
            _lib.check(_lib.NAYLIS_ERR_ARG)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_router_fwd(
                x.data_ptr(), _DT[x.dtype], w_down.data_ptr(), w_up.data_ptr(),
                noise.data_ptr() if noise is not None else None, int(noise_kind), float(noise_scale),
                logits.data_ptr(), probs.data_ptr(), top_idx.data_ptr(), top_gates.data_ptr(), act.data_ptr(),
                h.data_ptr() if h is not None else None, ws.data_ptr(), ws.numel(),
                B, T, D, R, E, top_k, _lib.stream_of(dev))
        _lib.check(rc)
        ctx.save_for_backward(x, w_down, w_up, act, probs, top_idx, top_gates)
        ctx.mark_non_differentiable(top_idx)
        if h is not None:
            ctx.mark_non_differentiable(h)
            return logits, probs, top_idx, top_gates, h
        return logits, probs, top_idx, top_gates

    @staticmethod
    def backward(ctx, d_logits, d_probs, _d_idx, d_gates, *_rest):
        lib = _lib.load()
        x, w_down, w_up, act, probs, top_idx, top_gates = ctx.saved_tensors
        B, T, D = x.shape
        R, E = w_down.shape[0], w_up.shape[0]
        top_k = top_idx.shape[-1]
        dev = x.device

        def opt(t):
            return t.float().contiguous() if t is not None else None

        d_logits, d_gates = opt(d_logits), opt(d_gates)
        d_probs, dp_ptr, dp_stride = d_probs_arg(d_probs, E)
        dx = torch.empty_like(x)
        dw_down = torch.empty((R, D), device=dev, dtype=torch.float32)
        dw_up = torch.empty((E, R), device=dev, dtype=torch.float32)
        nbytes = lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_router_bwd(
                x.data_ptr(), _DT[x.dtype], w_down.data_ptr(), w_up.data_ptr(), act.data_ptr(),
                probs.data_ptr(), top_idx.data_ptr(), top_gates.data_ptr(),
                d_gates.data_ptr() if d_gates is not None else None,
                dp_ptr, dp_stride,
                d_logits.data_ptr() if d_logits is not None else None,
                dx.data_ptr(), 0, dw_down.data_ptr(), dw_up.data_ptr(), ws.data_ptr(), ws.numel(),
                B, T, D, R, E, top_k, _lib.stream_of(dev))
        _lib.check(rc)
        return dx, dw_down, dw_up, None, None, None, None, None


def mom_route(x, w_down, w_up, top_k, noise=None, noise_scale=1.0, return_h=False, noise_is_uniform=False):
    """Fused causal prefix-mean router.

    x (B, T, D) bf16 or fp32 on a ROCm device; w_down (R, D), w_up (E, R)
    (cast to fp32: the router computes in fp32 as with fp32 master weights,
    model.py:181-187); noise (B, T, E) or None — added as
    ``noise_scale * noise`` to the logits before top-k only (model.py:209-216).
    With ``noise_is_uniform`` the noise tensor is the uniform draw u of
    model.py:210 and the kernel applies g = -log(-log(u + 1e-9) + 1e-9)
    itself.  Returns (router_logits, router_probs, top_idx int32, top_gates[, h]).
    """
    if x.dim() != 3:
        raise RuntimeError(f"mom_route: x must be (B, T, D), got {tuple(x.shape)}")
    if x.dtype not in _DT:
        raise RuntimeError(f"mom_route: x must be fp32 or bf16, got {x.dtype}")
    if x.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"mom_route: needs a ROCm device tensor, got {x.device}")
    B, T, D = x.shape
    if w_down.dim() != 2 or w_down.shape[1] != D:
        raise RuntimeError(f"mom_route: router_down weight must be (R, {D}), got {tuple(w_down.shape)}")
    R = w_down.shape[0]
    if w_up.dim() != 2 or w_up.shape[1] != R:
        raise RuntimeError(f"mom_route: router_up weight must be (E, {R}), got {tuple(w_up.shape)}")
    E = w_up.shape[0]
    if noise is not None:
        if noise.shape != (B, T, E):
            raise RuntimeError(f"mom_route: noise must be ({B}, {T}, {E}), got {tuple(noise.shape)}")
        noise = noise.detach().float().contiguous()
    x = x.contiguous()
    w_down = w_down.float().contiguous()
    w_up = w_up.float().contiguous()
    return MomRouteFunction.apply(x, w_down, w_up, noise, float(noise_scale), int(top_k), bool(return_h),
                                  NOISE_GUMBEL_UNIFORM if noise_is_uniform else NOISE_ADDITIVE)


class RouterStatsFunction(torch.autograd.Function):
    """stats = [mean_prob (E), frac (E), aux, entropy, dead] of a routing.
    Only mean_prob and aux carry gradient (frac comes from the selection mask;
    the reference logs entropy and dead fraction detached)."""

    @staticmethod
    def forward(ctx, probs, top_idx):
        lib = _lib.load()
        E = probs.shape[-1]
        N = probs.numel() // E
        k = top_idx.shape[-1]
        dev = probs.device
        stats = torch.empty(2 * E + 3, device=dev, dtype=torch.float32)
        nbytes = lib.naylis_mom_router_stats_workspace_bytes(N, E)
        if nbytes == 0:
            _lib.check(_lib.NAYLIS_ERR_ARG)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_router_stats(probs.data_ptr(), top_idx.data_ptr(), stats.data_ptr(),
                                                   ws.data_ptr(), ws.numel(), N, E, k, _lib.stream_of(dev)))
        ctx.save_for_backward(stats)
        ctx.shape = tuple(probs.shape)
        return stats

    @staticmethod
    def backward(ctx, d_stats):
        (stats,) = ctx.saved_tensors
        E = ctx.shape[-1]
        N = 1
        for s in ctx.shape[:-1]:
            N *= s
        # d mean_prob_e = d_stats[e] + d_aux * E * frac_e; every token gets 1/N of it
        row = (d_stats[:E] + d_stats[2 * E] * E * stats[E:2 * E]) / N
        return row.expand(ctx.shape), None


def mom_router_stats(probs, top_idx):
    """Load-balance statistics of one routing: probs (..., E) fp32 router
    softmax, top_idx (..., k) int.  Returns a (2E + 3,) fp32 tensor:
    [0:E] mean prob per block, [E:2E] fraction of tokens selecting it, [2E]
    the aux term E * sum(frac * mean_prob) (model.py:500-503), [2E+1] mean
    router entropy, [2E+2] dead-block fraction (model.py:505-507)."""
    if probs.dtype != torch.float32:
        probs = probs.float()
    if probs.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"mom_router_stats: needs a ROCm device tensor, got {probs.device}")
    E = probs.shape[-1]
    if top_idx.shape[:-1] != probs.shape[:-1]:
        raise RuntimeError(f"mom_router_stats: top_idx {tuple(top_idx.shape)} does not match probs "
                           f"{tuple(probs.shape)}")
    return RouterStatsFunction.apply(probs.contiguous(), top_idx.to(torch.int32).contiguous())
