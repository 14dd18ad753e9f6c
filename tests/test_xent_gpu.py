"""Fused next-token cross-entropy (naylis_mom_xent_*) against the reference's
F.cross_entropy(logits.float(), labels, reduction="sum") (model.py:536-545)
on the same GPU inputs: loss and the bf16 gradient of the logits."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,V", [(4095, 32768), (7, 2048), (300, 6144)])
def test_xent_matches_cross_entropy(N, V, dev):
    from naylis_amd.mom_kernels.hip_xent import cross_entropy_rows
    g = torch.Generator().manual_seed(N)
    logits = (torch.randn(N, V, generator=g) * 4).bfloat16().to(dev)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[::5] = -100                                  # ignored rows
    labels = labels.to(dev)
    n_valid = (labels != -100).sum()
    lr = logits.clone().requires_grad_(True)
    want = F.cross_entropy(lr.float(), labels, reduction="sum") / n_valid
    want.backward()
    lg = logits.clone().requires_grad_(True)
    rows = cross_entropy_rows(lg, labels)
    got = rows.sum() / n_valid
    got.backward()
    torch.cuda.synchronize()
    assert abs(float(got) - float(want)) <= 1e-5 * abs(float(want))
    assert bool((rows[labels == -100] == 0).all())
    # per-row: the fp32 log-sum-exp to a few ulps, then one bf16 rounding of the gradient
    err = (lg.grad.float() - lr.grad.float()).abs()
    bound = lr.grad.float().abs() * 2.0 ** -7 + 1e-9
    assert bool((err <= bound).all()), float((err - bound).max())
    assert bool((lg.grad[labels == -100] == 0).all())


def test_xent_out_of_range_label_is_nan(dev):
    """A label outside [0, V) that is not ignore_index (F.cross_entropy
    raises on it) makes that row's loss and gradient NaN; the other rows are
    unaffected, so the summed loss is NaN rather than silently smaller."""
    from naylis_amd.mom_kernels.hip_xent import cross_entropy_rows
    g = torch.Generator().manual_seed(3)
    N, V = 6, 2048
    logits = (torch.randn(N, V, generator=g) * 4).bfloat16().to(dev)
    labels = torch.randint(0, V, (N,), generator=g)
    labels[1], labels[4] = V, -100                       # one out of range, one ignored
    labels = labels.to(dev)
    lg = logits.clone().requires_grad_(True)
    rows = cross_entropy_rows(lg, labels)
    rows.sum().backward()
    torch.cuda.synchronize()
    assert torch.isnan(rows[1]) and torch.isnan(rows.sum())
    assert float(rows[4]) == 0.0
    ok = torch.tensor([0, 2, 3, 5], device=dev)
    want = F.cross_entropy(logits[ok].float(), labels[ok], reduction="none")
    assert torch.allclose(rows[ok], want, rtol=1e-5, atol=1e-5)
    assert bool(torch.isnan(lg.grad[1]).all()) and bool((lg.grad[4] == 0).all())
    assert bool(torch.isfinite(lg.grad[ok]).all())


def test_xent_rejects_unsupported(dev):
    from naylis_amd.mom_kernels.hip_xent import cross_entropy_rows
    with pytest.raises(RuntimeError, match="multiple of"):
        cross_entropy_rows(torch.randn(4, 1000, device=dev).bfloat16(), torch.zeros(4, dtype=torch.long, device=dev))
