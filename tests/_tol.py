"""Tolerance helpers shared by the parity tests.

The bar: bf16 outputs and gradients within
rtol 2e-2 / atol 2e-3 of the eager fp32 oracle on identical inputs, i.e.
|got - ref| <= 2e-3 + 2e-2 * |ref| elementwise.  The reference's own parity
metric, scaled_max = max|a - b| / max|b| (tests/test_parity.py:64-67), is
reported beside it.
"""
import torch

RTOL = 2e-2
ATOL = 2e-3


def scaled_max(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max()) / max(float(b.abs().max()), 1e-6)


def assert_close(got, ref, name, rtol=RTOL, atol=ATOL):
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, f"{name}: shape {tuple(g.shape)} != {tuple(r.shape)}"
    assert torch.isfinite(g).all(), f"{name}: non-finite values"
    diff = (g - r).abs()
    bound = atol + rtol * r.abs()
    bad = diff > bound
    if bad.any():
        i = int(torch.argmax((diff - bound).flatten()))
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{bad.numel()} elements outside rtol={rtol} atol={atol}; "
            f"worst got={float(g.flatten()[i]):.6g} ref={float(r.flatten()[i]):.6g}; "
            f"max_abs={float(diff.max()):.3e} scaled_max={scaled_max(g, r):.3e}")
