"""One autograd node for the whole MoM layer (model.py:189-276): router, bank
K/V, q projection, gated read, o projection and the ReZero gate.

The layer's separate autograd Functions (hip_router, hip_bank, hip_read,
hip_linear, hip_rezero) give autograd a graph in which x feeds both the router
and the q projection, so autograd sums the two input gradients with an extra
elementwise kernel, and materialises zero gradients for router outputs the
loss does not use.  Here the backward runs the library calls in a fixed
order instead: the q projection's input gradient is written first and the
router's backward accumulates into it (C ABI dx_accumulate, one bf16 rounding
of the fp32 sum), and absent output gradients are passed as NULL.  The
ReZero gate is folded into the o projection's weight, s * (out W_o^T) =
out (s W_o)^T, so the layer's fp32 output is one GEMM with an fp32 result
(no bf16 z to scale, store and read back); its backward takes dW' = dy^T out
in fp32 and gets dW_o = s dW' and ds = sum(dW' W_o) from one pass over the
weight.  Results equal the modular path's to bf16 rounding (W' is rounded
where the modular path rounds o W_o^T); the modular Functions stay the
public drop-in API (mom_read etc.) and serve gradient checkpointing.

The node's host work -- about fifteen library and torch calls each way --
runs in C++ (the torch extension of csrc/torch_layer.cpp, one call per
direction) when ``USE_TORCH_EXT`` is set, as it is by default; the Python
statement of the same calls below stays as its specification and for the
tests that compare the two bitwise.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import _lib, _torch_ext
from .hip_linear import library_wgrad as _wgrad
from .hip_read import _ptr, read_order, read_side
from .hip_rezero import gated_linear_backward, gated_linear_forward
from .hip_router import d_probs_arg

_F32, _BF16 = 0, 1

# run the node's host side in the torch extension (one C++ call per direction)
USE_TORCH_EXT = True
# the node itself in C++ (the extension's mom_layer: a torch::autograd::Function
# whose forward / backward make the calls of MomLayerFunction's extension path)
USE_CPP_NODE = True


def _ws(nbytes, dev):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def fused_layer_supported(x, M_blocks, w_down, w_up, w_q, w_k, w_v, w_o, scale, bank_kv=None):
    """True when the fused node applies: bf16 activations and projection
    weights, fp32 router weights and gate, D a multiple of 128 (the router's
    accumulating backward), all on one ROCm device.  With ``bank_kv`` the
    bank's K and V come from the caller (bf16, contiguous)."""
    if torch.version.hip is None or not x.is_cuda:
        return False
    if x.dim() != 3 or x.dtype != torch.bfloat16 or x.shape[-1] % 128 != 0:
        return False
    dev = x.device
    for w in (w_q, w_k, w_v, w_o):
        if w.dtype != torch.bfloat16 or w.device != dev or w.dim() != 2:
            return False
    if w_q.shape != (x.shape[-1], x.shape[-1]) or w_o.shape != w_q.shape:
        return False
    if w_down.dtype != torch.float32 or w_up.dtype != torch.float32 or w_down.shape[0] > 64:
        return False
    if scale.dtype != torch.float32 or scale.numel() != 1 or scale.device != dev:
        return False
    if bank_kv is not None:
        return all(t.dtype == torch.bfloat16 and t.device == dev and t.is_contiguous() and t.dim() == 2
                   and t.shape[1] == x.shape[-1] for t in bank_kv)
    return M_blocks.device == dev and M_blocks.dtype in (torch.bfloat16, torch.float32)


class MomLayerFunction(torch.autograd.Function):
    """y, probs, top_idx = layer(x, M_blocks, ...); y fp32 (ReZero promotes),
    probs the router softmax (for the load-balance aux loss), top_idx int32."""

    @staticmethod
    def forward(ctx, x, M_blocks, w_down, w_up, w_q, w_k, w_v, w_o, scale, noise, noise_scale, geom, k_ext=None,
                v_ext=None):
        n_heads, num_blocks, block_size, top_k, noise_kind = geom
        lib = _lib.load()
        B, T, D = x.shape
        R, E = w_down.shape[0], w_up.shape[0]
        H, HD = n_heads, D // n_heads
        dev = x.device
        st = _lib.stream_of(dev)
        x = x.contiguous()
        if USE_TORCH_EXT:
            (y, probs, top_idx, act, gates, slots, k, v, q, order, out, side, lse, w_os) = _torch_ext.load().layer_fwd(
                x, M_blocks if k_ext is None else None, w_down, w_up, w_q, w_k, w_v, w_o, scale, noise,
                float(noise_scale), n_heads, num_blocks, block_size, top_k, int(noise_kind), k_ext, v_ext, st)
            ctx.save_for_backward(x, slots, w_down, w_up, w_q, w_k, w_v, w_o, scale, act, probs, top_idx, gates, k, v,
                                  q, order, out, side, lse, w_os)
            ctx.geom = geom
            ctx.external_bank = k_ext is not None
            ctx.m_shape = None if k_ext is not None else (tuple(M_blocks.shape), M_blocks.dtype)
            ctx.mark_non_differentiable(top_idx)
            ctx.set_materialize_grads(False)
            return y, probs, top_idx
        f32 = dict(device=dev, dtype=torch.float32)
        with _lib.on_device(dev):
            # ---- router (model.py:169-220)
            logits = torch.empty((B, T, E), **f32)
            probs = torch.empty((B, T, E), **f32)
            top_idx = torch.empty((B, T, top_k), device=dev, dtype=torch.int32)
            gates = torch.empty((B, T, top_k), **f32)
            act = torch.empty((B, T, R), **f32)
            rws = _ws(lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k), dev)
            _lib.check(lib.naylis_mom_router_fwd(
                x.data_ptr(), _BF16, w_down.data_ptr(), w_up.data_ptr(),
                noise.data_ptr() if noise is not None else None, int(noise_kind), float(noise_scale),
                logits.data_ptr(),
                probs.data_ptr(), top_idx.data_ptr(), gates.data_ptr(), act.data_ptr(), None, rws.data_ptr(),
                rws.numel(), B, T, D, R, E, top_k, st))
            del rws
            # ---- bank K/V (model.py:253-256), unless the caller projected the bank (grouped over layers)
            if k_ext is None:
                slots = M_blocks.reshape(-1, D)
                m_dtype = slots.dtype
                slots = slots.to(torch.bfloat16).contiguous()
                L = slots.shape[0]
                k = torch.empty((L, D), device=dev, dtype=torch.bfloat16)
                v = torch.empty((L, D), device=dev, dtype=torch.bfloat16)
                _lib.check(lib.naylis_mom_bank_kv_fwd(slots.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
                                                      k.data_ptr(), v.data_ptr(), L, D, D, st))
            else:
                slots, m_dtype, k, v = None, None, k_ext, v_ext
            # ---- q projection, gated read, o projection (model.py:251, 258-276)
            q = F.linear(x, w_q)
            order = read_order(top_idx, num_blocks)
            out = torch.empty_like(q)
            side = read_side(lib, out.view(B, T, H, HD), num_blocks, block_size, top_k)
            lse = torch.empty((H, B, T), **f32)
            _lib.check(lib.naylis_mom_read_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr(), gates.data_ptr(), order.data_ptr(),
                out.data_ptr(), _ptr(side), lse.data_ptr(), None, 0, B, T, H, HD, num_blocks, block_size, top_k,
                st))
            # ---- o projection and ReZero gate (model.py:251, 239): one GEMM, the gate
            # folded into the weight
            y, w_os = gated_linear_forward(lib, out.view(B * T, D), w_o, scale, st)
            y = y.view(B, T, D)
        ctx.save_for_backward(x, slots, w_down, w_up, w_q, w_k, w_v, w_o, scale, act, probs, top_idx, gates, k, v,
                              q, order, out, side, lse, w_os)
        ctx.geom = geom
        ctx.external_bank = k_ext is not None
        ctx.m_shape = None if k_ext is not None else (tuple(M_blocks.shape), m_dtype)
        ctx.mark_non_differentiable(top_idx)
        ctx.set_materialize_grads(False)
        return y, probs, top_idx

    @staticmethod
    def backward(ctx, dy, d_probs, _d_idx):
        (x, slots, w_down, w_up, w_q, w_k, w_v, w_o, scale, act, probs, top_idx, gates, k, v, q, order, out, side,
         lse, w_os) = ctx.saved_tensors
        n_heads, num_blocks, block_size, top_k, _ = ctx.geom
        lib = _lib.load()
        B, T, D = x.shape
        R, E = w_down.shape[0], w_up.shape[0]
        H, HD = n_heads, D // n_heads
        L = k.shape[0]
        dev = x.device
        st = _lib.stream_of(dev)
        f32 = dict(device=dev, dtype=torch.float32)
        N = B * T
        if USE_TORCH_EXT:
            m_shape, m_dtype = ctx.m_shape if ctx.m_shape is not None else ((), None)
            (dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds, dk_ext, dv_ext) = _torch_ext.load().layer_bwd(
                dy, d_probs, x, slots, w_down, w_up, w_q, w_k, w_v, w_o, scale, act, probs, top_idx, gates, k, v, q,
                order, out, side, lse, w_os, n_heads, num_blocks, block_size, top_k, ctx.external_bank,
                list(m_shape), m_dtype == torch.bfloat16, st)
            return (dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds.view(scale.shape), None, None, None, dk_ext,
                    dv_ext)
        with _lib.on_device(dev):
            # ---- o projection with the folded gate (d out, dW_o, ds)
            if dy is None:
                dy = torch.zeros((B, T, D), device=dev, dtype=torch.bfloat16)
            dout, dw_o, ds = gated_linear_backward(lib, dy.reshape(N, D), out.view(N, D), w_o, w_os, scale, st)
            dout = dout.view(B, T, H, HD)
            # ---- gated read
            dq = torch.empty_like(q)
            dk = torch.empty_like(k)
            dv = torch.empty_like(v)
            dgates = torch.empty_like(gates)
            nbytes = lib.naylis_mom_read_workspace_bytes(B, T, H, HD, num_blocks, block_size, top_k)
            if nbytes == 0:
                _lib.check(_lib.NAYLIS_ERR_ARG)
            rws = _ws(nbytes, dev)
            _lib.check(lib.naylis_mom_read_bwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr(), gates.data_ptr(), order.data_ptr(),
                out.data_ptr(), _ptr(side), lse.data_ptr(), dout.data_ptr(), dq.data_ptr(), dk.data_ptr(),
                dv.data_ptr(),
                dgates.data_ptr(), rws.data_ptr(), rws.numel(), B, T, H, HD, num_blocks, block_size, top_k, st))
            del rws, dout
            # ---- bank K/V (the caller's grouped node takes dK, dV when it projected the bank)
            if ctx.external_bank:
                d_m, dw_k, dw_v, dk_ext, dv_ext = None, None, None, dk, dv
            else:
                m_shape, m_dtype = ctx.m_shape
                sdt = _BF16 if m_dtype == torch.bfloat16 else _F32
                d_slots = torch.empty((L, D), device=dev, dtype=m_dtype)
                dw_k = torch.empty_like(w_k)
                dw_v = torch.empty_like(w_v)
                _lib.check(lib.naylis_mom_bank_kv_bwd(slots.data_ptr(), w_k.data_ptr(), w_v.data_ptr(),
                                                      dk.data_ptr(), dv.data_ptr(), d_slots.data_ptr(), sdt,
                                                      dw_k.data_ptr(), dw_v.data_ptr(), _BF16, L, D, D, st))
                d_m, dk_ext, dv_ext = d_slots.view(m_shape), None, None
            # ---- q projection: dx = dq W_q (the router adds its part below), dW_q = dq^T x
            dq2 = dq.view(N, D)
            dx = torch.mm(dq2, w_q).view(B, T, D)
            dw_q = _wgrad(lib, x.view(N, D), dq2, w_q.dtype, dev, st)
            # ---- router, accumulating into dx
            d_probs, dp_ptr, dp_stride = d_probs_arg(d_probs, E)
            dw_down = torch.empty((R, D), **f32)
            dw_up = torch.empty((E, R), **f32)
            rws = _ws(lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, top_k), dev)
            _lib.check(lib.naylis_mom_router_bwd(
                x.data_ptr(), _BF16, w_down.data_ptr(), w_up.data_ptr(), act.data_ptr(), probs.data_ptr(),
                top_idx.data_ptr(), gates.data_ptr(), dgates.data_ptr(),
                dp_ptr, dp_stride, None, dx.data_ptr(), 1, dw_down.data_ptr(),
                dw_up.data_ptr(), rws.data_ptr(), rws.numel(), B, T, D, R, E, top_k, st))
        return (dx, d_m, dw_down, dw_up, dw_q, dw_k, dw_v, dw_o, ds.view(scale.shape), None, None, None, dk_ext,
                dv_ext)


def mom_layer(x, M_blocks, w_down, w_up, w_q, w_k, w_v, w_o, scale, *, n_heads, num_blocks, block_size, top_k,
              noise=None, noise_scale=1.0, noise_is_uniform=False, bank_kv=None):
    """The fused layer node; callers check fused_layer_supported() first.
    ``noise_is_uniform``: noise is the uniform draw and the router kernel
    applies the Gumbel transform.  ``bank_kv``: the bank's (K, V) projected by
    the caller (M_blocks, w_k and w_v then get no gradient here; K and V do).
    Returns (y fp32, router probs, top_idx int32)."""
    if noise is not None:
        noise = noise.detach().float().contiguous()
    k_ext, v_ext = bank_kv if bank_kv is not None else (None, None)
    if USE_TORCH_EXT and USE_CPP_NODE:
        y, probs, top_idx = _torch_ext.load().mom_layer(
            x, M_blocks if bank_kv is None else None, w_down.float().contiguous(), w_up.float().contiguous(), w_q,
            w_k, w_v, w_o, scale, noise, float(noise_scale), int(n_heads), int(num_blocks), int(block_size),
            int(top_k), 1 if noise_is_uniform else 0, k_ext, v_ext, _lib.stream_of(x.device))
        return y, probs, top_idx
    return MomLayerFunction.apply(x, M_blocks if bank_kv is None else None, w_down.float().contiguous(),
                                  w_up.float().contiguous(), w_q, w_k, w_v, w_o, scale, noise, float(noise_scale),
                                  (int(n_heads), int(num_blocks), int(block_size), int(top_k),
                                   1 if noise_is_uniform else 0), k_ext, v_ext)
