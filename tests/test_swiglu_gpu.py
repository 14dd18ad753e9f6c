"""Fused SwiGLU (naylis_mom_swiglu_*) against transformers' LlamaMLP
activation, silu(gate) * up, on the same GPU inputs (model.py:279-345)."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(16384, 2816), (3, 7, 64), (8,)])
def test_swiglu_matches_silu_times_up(shape, dtype, dev):
    from naylis_amd.mom_kernels.hip_mlp import swiglu
    g0 = torch.Generator().manual_seed(sum(shape))
    g = (torch.randn(shape, generator=g0) * 3).to(dtype).to(dev)
    u = torch.randn(shape, generator=g0).to(dtype).to(dev)
    dh = torch.randn(shape, generator=g0).to(dtype).to(dev)
    gr, ur = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    hr = F.silu(gr) * ur
    hr.backward(dh)
    gg, ug = g.clone().requires_grad_(True), u.clone().requires_grad_(True)
    hg = swiglu(gg, ug)
    hg.backward(dh)
    torch.cuda.synchronize()
    if dtype == torch.bfloat16:
        # the same bf16 roundings; silu's fp32 value may differ in its last bit
        # from torch's (separately compiled exp / division), which can move a
        # bf16 rounding by one ulp
        for got, want in ((hg, hr), (gg.grad, gr.grad), (ug.grad, ur.grad)):
            ulp2 = (want.float().abs() * 2.0 ** -6).clamp_min(1e-30)
            assert bool(((got.float() - want.float()).abs() <= ulp2).all())
            assert float((got != want).float().mean()) < 1e-3
    else:
        assert torch.allclose(hg, hr, rtol=1e-6, atol=1e-7)
        assert torch.allclose(gg.grad, gr.grad, rtol=1e-5, atol=1e-6)
        assert torch.allclose(ug.grad, ur.grad, rtol=1e-6, atol=1e-7)


def test_swiglu_rejects_unsupported(dev):
    from naylis_amd.mom_kernels.hip_mlp import swiglu
    with pytest.raises(RuntimeError, match="unsupported"):
        swiglu(torch.randn(7, device=dev), torch.randn(7, device=dev))
