"""Fused rotary embedding (naylis_mom_rope) against transformers'
apply_rotary_pos_emb, which the Llama attention of every decoder layer calls
(model.py:279-345): same inputs on the GPU, outputs and gradients bitwise."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("B,S,H,hd,cb", [(2, 300, 4, 64, 2), (1, 128, 16, 64, 1), (3, 77, 2, 128, 3),
                                         (2, 64, 8, 32, 1)])
def test_rope_matches_transformers(B, S, H, hd, cb, dtype, dev):
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    from naylis_amd.mom_kernels.hip_rope import rope
    g = torch.Generator().manual_seed(B * S + hd)
    q = torch.randn(B, S, H, hd, generator=g).to(dtype).to(dev)
    k = torch.randn(B, S, H, hd, generator=g).to(dtype).to(dev)
    ang = torch.rand(cb, S, hd // 2, generator=g) * 6.28
    ang = torch.cat([ang, ang], -1)
    cos, sin = ang.cos().to(dtype).to(dev), ang.sin().to(dtype).to(dev)
    dq = torch.randn(B, S, H, hd, generator=g).to(dtype).to(dev)
    dk = torch.randn(B, S, H, hd, generator=g).to(dtype).to(dev)

    qr, kr = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    # transformers works on (B, H, S, hd) with cos / sin unsqueezed at dim 1
    a, b = apply_rotary_pos_emb(qr.transpose(1, 2), kr.transpose(1, 2), cos, sin)
    a, b = a.transpose(1, 2), b.transpose(1, 2)
    (a * dq).sum().backward(retain_graph=True)
    (b * dk).sum().backward()
    qg, kg = q.clone().requires_grad_(True), k.clone().requires_grad_(True)
    c, d = rope(qg, kg, cos, sin)
    torch.autograd.backward((c, d), (dq, dk))
    torch.cuda.synchronize()
    assert torch.equal(c, a) and torch.equal(d, b)
    if dtype == torch.float32:
        # the reference's autograd accumulates the two paths of q in fp32; one rounding each way
        assert torch.allclose(qg.grad, qr.grad, rtol=1e-6, atol=1e-7)
        assert torch.allclose(kg.grad, kr.grad, rtol=1e-6, atol=1e-7)
    else:
        assert torch.equal(qg.grad, qr.grad) and torch.equal(kg.grad, kr.grad)


def test_rope_rejects_unsupported(dev):
    from naylis_amd.mom_kernels.hip_rope import rope
    q = torch.randn(1, 8, 2, 48, device=dev)
    cs = torch.randn(1, 8, 48, device=dev)
    with pytest.raises(RuntimeError, match="unsupported"):
        rope(q, q, cs, cs)
