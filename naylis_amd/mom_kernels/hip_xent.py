"""Fused next-token cross-entropy of the decoder (C ABI: naylis_mom_xent_*).

The reference computes ``F.cross_entropy(shift_logits.float(), labels,
reduction="sum")`` (model.py:536-545): an fp32 copy of the (N, V) logits,
log_softmax and the label pick, and the same passes backward.
``cross_entropy_rows`` reads the bf16 logits once forward and once backward
and returns each row's loss (0 for ignore_index rows); summing and dividing
by the number of valid labels stays with the caller, as in the reference.
A label outside [0, V) that is not ignore_index, which F.cross_entropy
rejects with an error, gives that row a NaN loss and NaN gradient, so the
summed loss shows it instead of dropping the row silently.
"""
from __future__ import annotations

import torch

from .. import _lib


def xent_supported(logits, labels):
    return (torch.version.hip is not None and logits.is_cuda and logits.dtype == torch.bfloat16
            and logits.dim() == 2 and logits.shape[1] % 2048 == 0 and labels.shape == logits.shape[:1]
            and labels.device == logits.device)


class XentFunction(torch.autograd.Function):

    @staticmethod
    def forward(ctx, logits, labels, ignore_index):
        lib = _lib.load()
        logits = logits.contiguous()
        labels = labels.to(torch.int64).contiguous()
        N, V = logits.shape
        dev = logits.device
        loss = torch.empty(N, device=dev, dtype=torch.float32)
        lse = torch.empty(N, device=dev, dtype=torch.float32)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_xent_fwd(logits.data_ptr(), labels.data_ptr(), loss.data_ptr(), lse.data_ptr(),
                                               N, V, int(ignore_index), _lib.stream_of(dev)))
        ctx.save_for_backward(logits, labels, lse)
        ctx.ignore_index = int(ignore_index)
        ctx.mark_non_differentiable(lse)
        return loss

    @staticmethod
    def backward(ctx, d_loss):
        lib = _lib.load()
        logits, labels, lse = ctx.saved_tensors
        N, V = logits.shape
        dev = logits.device
        d_loss = d_loss.float()
        if d_loss.dim() == 1 and d_loss.stride(0) == 0:
            g, stride = d_loss, 0          # one gradient for every row (the sum's backward)
        else:
            g, stride = d_loss.contiguous(), 1
        dlogits = torch.empty_like(logits)
        with _lib.on_device(dev):
            _lib.check(lib.naylis_mom_xent_bwd(logits.data_ptr(), labels.data_ptr(), lse.data_ptr(), g.data_ptr(),
                                               stride, dlogits.data_ptr(), N, V, ctx.ignore_index,
                                               _lib.stream_of(dev)))
        return dlogits, None, None


def cross_entropy_rows(logits, labels, ignore_index=-100):
    """Per-row next-token loss of bf16 logits (N, V); raises when
    ``xent_supported`` is false."""
    if not xent_supported(logits, labels):
        raise RuntimeError(f"cross_entropy_rows: needs bf16 logits (N, V) on a ROCm device with V a multiple of "
                           f"2048; got {tuple(logits.shape)} {logits.dtype} on {logits.device}")
    return XentFunction.apply(logits, labels, ignore_index)
