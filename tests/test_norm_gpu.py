"""Fused RMSNorm (naylis_mom_rmsnorm_*) against transformers' LlamaRMSNorm,
the module model.py:304-305 builds, on the same GPU inputs and weights."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _pair(D, dtype, dev, seed):
    from transformers.models.llama.modeling_llama import LlamaRMSNorm

    from naylis_amd.mom_kernels.hip_norm import NaylisRMSNorm
    g = torch.Generator().manual_seed(seed)
    w = (1.0 + 0.5 * torch.randn(D, generator=g)).to(dtype)
    ref = LlamaRMSNorm(D, eps=1e-5).to(dev, dtype)
    got = NaylisRMSNorm(D, eps=1e-5).to(dev, dtype)
    with torch.no_grad():
        ref.weight.copy_(w)
        got.weight.copy_(w)
    return ref, got


def _rel(a, b):
    return float((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("N,D", [(16384, 1024), (333, 512), (7, 1536), (64, 4096), (1, 2048)])
def test_rmsnorm_matches_llama_rmsnorm(N, D, dtype, dev):
    ref, got = _pair(D, dtype, dev, seed=N + D)
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(N, D, generator=g) * 3.0).to(dtype).to(dev)
    dy = torch.randn(N, D, generator=g).to(dtype).to(dev)
    xr = x.clone().requires_grad_(True)
    xg = x.clone().requires_grad_(True)
    yr = ref(xr)
    yg = got(xg)
    yr.backward(dy)
    yg.backward(dy)
    torch.cuda.synchronize()
    assert yg.dtype == yr.dtype and yg.shape == yr.shape
    if dtype == torch.float32:
        assert torch.allclose(yg, yr, rtol=1e-5, atol=1e-6)
        assert torch.allclose(xg.grad, xr.grad, rtol=1e-4, atol=1e-6)
        assert _rel(got.weight.grad, ref.weight.grad) <= 1e-5
    else:
        # forward: the same bf16 roundings; the fp32 sum of squares may differ in
        # its last bit from torch's mean, which can move bf16(h) by one ulp where
        # h sits on a rounding boundary, and w * bf16(h) then by up to two ulps of
        # y (measured: 75 of 16.8 M outputs at N=16384, D=1024)
        two_ulp = (yr.float().abs() * 2.0 ** -6).clamp_min(1e-30)
        assert bool(((yg.float() - yr.float()).abs() <= two_ulp).all())
        assert float((yg != yr).float().mean()) < 1e-3
        # backward: torch rounds dy * w and dy * T(h) to bf16 before its sums; the
        # fused kernel keeps fp32 products, so compare at bf16 resolution
        assert _rel(xg.grad, xr.grad) <= 1e-2
        assert _rel(got.weight.grad, ref.weight.grad) <= 1e-2


def test_rmsnorm_deterministic_and_3d(dev):
    _, got = _pair(1024, torch.bfloat16, dev, seed=3)
    x = torch.randn(4, 100, 1024, device=dev).bfloat16().requires_grad_(True)
    dy = torch.randn(4, 100, 1024, device=dev).bfloat16()
    outs = []
    for _ in range(2):
        x.grad = None
        got.weight.grad = None
        y = got(x)
        y.backward(dy)
        outs.append((y.detach().clone(), x.grad.clone(), got.weight.grad.clone()))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert outs[0][0].shape == (4, 100, 1024)


def test_rmsnorm_rejects_unsupported(dev):
    from naylis_amd.mom_kernels.hip_norm import rms_norm
    w = torch.ones(1000, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 512"):
        rms_norm(torch.randn(4, 1000, device=dev), w)


@pytest.mark.parametrize("a_dtype", [torch.bfloat16, torch.float32])
def test_add_rmsnorm_matches_add_then_norm(a_dtype, dev):
    """s = x + a.to(x.dtype); y = norm(s) fused, against the two torch steps
    the decoder block would run (model.py:330-345), forward and backward."""
    from naylis_amd.mom_kernels.hip_norm import add_rms_norm
    ref, got = _pair(1024, torch.bfloat16, dev, seed=9)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4096, 1024, generator=g).bfloat16().to(dev)
    a = torch.randn(4096, 1024, generator=g).to(a_dtype).to(dev)
    ds = torch.randn(4096, 1024, generator=g).bfloat16().to(dev)
    dy = torch.randn(4096, 1024, generator=g).bfloat16().to(dev)
    xr, ar = x.clone().requires_grad_(True), a.clone().requires_grad_(True)
    sr = xr + ar.to(torch.bfloat16)
    yr = ref(sr)
    torch.autograd.backward((sr, yr), (ds, dy))
    xg, ag = x.clone().requires_grad_(True), a.clone().requires_grad_(True)
    sg, yg = add_rms_norm(xg, ag, got)
    torch.autograd.backward((sg, yg), (ds, dy))
    torch.cuda.synchronize()
    assert torch.equal(sg, sr)                                   # the add rounds like torch's
    two_ulp = (yr.float().abs() * 2.0 ** -6).clamp_min(1e-30)
    assert bool(((yg.float() - yr.float()).abs() <= two_ulp).all())
    # torch rounds the norm's input gradient to bf16 before adding ds; the kernel adds first
    assert _rel(xg.grad, xr.grad) <= 1e-2 and _rel(ag.grad, ar.grad) <= 1e-2
    assert ag.grad.dtype == a_dtype
    assert _rel(got.weight.grad, ref.weight.grad) <= 1e-2
