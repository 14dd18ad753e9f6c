"""Autograd binding of the HIP gated flash read (C ABI: naylis_mom_read_*).

Drop-in for mom_kernels/triton_gpu.py:323-439 of the reference: same
``mom_read(q_sh, k, v, top_idx, top_gates, *, num_blocks, block_size)``
signature, same preconditions (triton_gpu.py:420-429), same gradient set
(dq, dk, dv, d top_gates; triton_gpu.py:409 plus the log-gate transform of
triton_gpu.py:435, which the kernels fold in).
"""
from __future__ import annotations

import torch

from .. import _lib


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def read_order(top_idx, num_blocks):
    """The token order the read uses for this routing (C ABI:
    naylis_mom_read_order): an int32 tensor of naylis_mom_read_order_words()
    words, word 0 = 1 when words 1..B*S hold the grouped position -> token
    table, 0 for sequence order, followed (top-2 over at most 32 blocks) by
    the pair plan of the pair-tiled kernels.  Launched on the current stream;
    top_idx must be int32 (B, S, k)."""
    lib = _lib.load()
    B, S, topk = top_idx.shape
    dev = top_idx.device
    words = int(lib.naylis_mom_read_order_words(B, S, num_blocks, topk))
    if words <= 0:
        _lib.check(_lib.NAYLIS_ERR_ARG)
    order = torch.empty((words,), device=dev, dtype=torch.int32)
    ows = _workspace(lib.naylis_mom_read_order_workspace_bytes(B, S, num_blocks, topk), dev)
    with _lib.on_device(dev):
        rc = lib.naylis_mom_read_order(top_idx.data_ptr(), order.data_ptr(), ows.data_ptr(), ows.numel(),
                                       B, S, num_blocks, topk, _lib.stream_of(dev))
    _lib.check(rc)
    return order


class MomReadFunction(torch.autograd.Function):
    """Forward computes the token order (tokens grouped by selected blocks, or
    sequence order when that does not pay, plus the pair plan) and saves (q,
    k, v, top_idx, top_gates, order, o, the pair path's side buffer when
    it is used, lse); backward runs the library's backward with the same order."""

    @staticmethod
    def forward(ctx, q_sh, k, v, top_idx, top_gates, num_blocks, block_size):
        lib = _lib.load()
        B, S, H, HD = q_sh.shape
        topk = top_idx.shape[-1]
        dev = q_sh.device
        out = torch.empty_like(q_sh)
        side = read_side(lib, out, num_blocks, block_size, topk)
        lse = torch.empty((H, B, S), device=dev, dtype=torch.float32)
        order = read_order(top_idx, num_blocks)  # mode word + table (+ pair plan)
        with _lib.on_device(dev):
            st = _lib.stream_of(dev)
            rc = lib.naylis_mom_read_fwd(
                q_sh.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr(), top_gates.data_ptr(),
                order.data_ptr(), out.data_ptr(), _ptr(side), lse.data_ptr(), None, 0,
                B, S, H, HD, num_blocks, block_size, topk, st)
        _lib.check(rc)
        ctx.save_for_backward(q_sh, k, v, top_idx, top_gates, order, out, side, lse)
        ctx.geom = (num_blocks, block_size)
        return out

    @staticmethod
    def backward(ctx, dout):
        lib = _lib.load()
        q_sh, k, v, top_idx, top_gates, order, out, side, lse = ctx.saved_tensors
        num_blocks, block_size = ctx.geom
        B, S, H, HD = q_sh.shape
        topk = top_idx.shape[-1]
        dev = q_sh.device
        dout = dout.contiguous()
        if dout.dtype != q_sh.dtype:
            dout = dout.to(q_sh.dtype)
        dq = torch.empty_like(q_sh)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        dgates = torch.empty_like(top_gates)
        nbytes = lib.naylis_mom_read_workspace_bytes(B, S, H, HD, num_blocks, block_size, topk)
        if nbytes == 0:
            _lib.check(_lib.NAYLIS_ERR_ARG)
        ws = _workspace(nbytes, dev)
        with _lib.on_device(dev):
            rc = lib.naylis_mom_read_bwd(
                q_sh.data_ptr(), k.data_ptr(), v.data_ptr(), top_idx.data_ptr(), top_gates.data_ptr(),
                order.data_ptr(), out.data_ptr(), _ptr(side), lse.data_ptr(), dout.data_ptr(), dq.data_ptr(),
                dk.data_ptr(),
                dv.data_ptr(),
                dgates.data_ptr(), ws.data_ptr(), ws.numel(),
                B, S, H, HD, num_blocks, block_size, topk, _lib.stream_of(dev))
        _lib.check(rc)
        return dq, dk, dv, None, dgates, None, None


def read_side(lib, out, num_blocks, block_size, top_k):
    """The side buffer the pair-tiled forward leaves for its backward (each
    row's biases minus lse, block-a share and selection bits), when the read
    takes that path both ways (naylis_mom_read_side_bytes > 0), else None."""
    B, S, H, HD = out.shape
    nbytes = int(lib.naylis_mom_read_side_bytes(B, S, H, HD, num_blocks, block_size, top_k))
    if nbytes > 0:
        return torch.empty(nbytes, dtype=torch.uint8, device=out.device)
    return None


def _ptr(t):
    return t.data_ptr() if t is not None else None


def mom_read(q_sh, k, v, top_idx, top_gates, *, num_blocks, block_size):
    """Flash MoM read with the in-register gate bias (ROCm, bf16).

    q_sh (B, S, H, hd) bf16; shared k/v (L, D) bf16; per-token (top_idx,
    top_gates) (B, S, k); returns (B, S, H, hd) bf16.  Raises RuntimeError
    on the reference's preconditions (triton_gpu.py:420-429) and when the
    HIP library is missing — there is no eager fallback.
    """
    if k.dim() != 2 or v.dim() != 2:
        raise RuntimeError("hip mom_read: shared K/V (L, D) only, got batched inputs")
    if q_sh.dtype != torch.bfloat16:
        raise RuntimeError(f"hip mom_read requires bf16 activations, got {q_sh.dtype}")
    if k.shape[0] != num_blocks * block_size:
        raise RuntimeError(
            f"hip mom_read: bank is {k.shape[0]} slots but num_blocks "
            f"({num_blocks}) x block_size ({block_size}) disagrees")
    if q_sh.dim() != 4:
        raise RuntimeError(f"hip mom_read: q_sh must be (B, S, H, hd), got {tuple(q_sh.shape)}")
    B, S, H, HD = q_sh.shape
    if k.shape[1] != H * HD or v.shape != k.shape:
        raise RuntimeError(
            f"hip mom_read: k/v must be (L, H*hd) = ({k.shape[0]}, {H * HD}), got {tuple(k.shape)} / {tuple(v.shape)}")
    if top_idx.shape[:2] != (B, S) or top_gates.shape != top_idx.shape:
        raise RuntimeError("hip mom_read: top_idx / top_gates must both be (B, S, top_k)")
    if q_sh.device.type != "cuda" or torch.version.hip is None:
        raise RuntimeError(f"hip mom_read: needs a ROCm device tensor, got {q_sh.device}")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        k = k.to(torch.bfloat16)
        v = v.to(torch.bfloat16)
    q_sh = q_sh.contiguous()
    k = k.contiguous()
    v = v.contiguous()
    top_idx = top_idx.to(torch.int32).contiguous()
    top_gates = top_gates.float().contiguous()
    return MomReadFunction.apply(q_sh, k, v, top_idx, top_gates, int(num_blocks), int(block_size))
