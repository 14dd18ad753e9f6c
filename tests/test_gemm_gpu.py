"""GPU checks of the split-K MFMA GEMM behind the q/o projection weight
gradient (C ABI naylis_mom_linear_wgrad; model.py:239,251 take it from
autograd as dy^T x over all tokens) against an fp64 product of the same bf16
inputs, plus the autograd binding against torch's own linear.

Tolerance: |got - ref| <= 2e-2 |ref| + 2e-3 max(1, max|ref|) (a sum over up to
16384 tokens has magnitudes >> 1; the atol scales with it as for the other
parameter gradients); results must be bitwise reproducible.
"""
import copy

import pytest
import torch

from tests._tol import assert_close

pytestmark = pytest.mark.gpu


def wgrad(x, dy, out_dtype):
    from naylis_amd import _lib
    lib = _lib.load()
    N, D_in = x.shape
    D_out = dy.shape[1]
    ws = torch.empty(lib.naylis_mom_linear_wgrad_workspace_bytes(N, D_in, D_out), device=x.device, dtype=torch.uint8)
    dw = torch.full((D_out, D_in), float("nan"), device=x.device, dtype=out_dtype)
    rc = lib.naylis_mom_linear_wgrad(x.data_ptr(), dy.data_ptr(), dw.data_ptr(), 0 if out_dtype == torch.float32 else 1,
                                     ws.data_ptr(), ws.numel(), N, D_in, D_out,
                                     torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    return dw


@pytest.mark.parametrize("N,D_in,D_out,out_dtype", [
    (16384, 1024, 1024, torch.bfloat16),   # config 2: B*T tokens, d x d
    (16384, 1024, 1024, torch.float32),
    (16384, 1536, 1536, torch.bfloat16),   # config 4 width
    (1000, 64, 192, torch.float32),        # ragged token count, rectangular
    (8, 24, 40, torch.float32),            # below one tile in every dimension
])
def test_linear_wgrad_matches_fp64(N, D_in, D_out, out_dtype, dev):
    g = torch.Generator().manual_seed(N + D_in)
    x = torch.randn(N, D_in, generator=g).bfloat16()
    dy = torch.randn(N, D_out, generator=g).bfloat16()
    got = wgrad(x.to(dev), dy.to(dev), out_dtype)
    torch.cuda.synchronize()
    ref = dy.double().T @ x.double()
    assert_close(got, ref, "dW", atol=2e-3 * max(1.0, float(ref.abs().max())))


def test_linear_wgrad_deterministic_and_empty(dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16384, 1024, generator=g).bfloat16().to(dev)
    dy = torch.randn(16384, 1024, generator=g).bfloat16().to(dev)
    a = wgrad(x, dy, torch.float32)
    b = wgrad(x, dy, torch.float32)
    assert torch.equal(a, b)
    z = wgrad(x[:0], dy[:0], torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(z.cpu(), torch.zeros(1024, 1024))


def test_mom_linear_autograd_matches_torch(dev):
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4, 512, 256, generator=g).bfloat16().to(dev).requires_grad_(True)
    w = (torch.randn(384, 256, generator=g) * 0.05).bfloat16().to(dev).requires_grad_(True)
    dy = torch.randn(4, 512, 384, generator=g).bfloat16().to(dev)
    y = mom_kernels.mom_linear(x, w)
    y.backward(dy)
    xr = x.detach().double().requires_grad_(True)
    wr = w.detach().double().requires_grad_(True)
    yr = torch.nn.functional.linear(xr, wr)
    yr.backward(dy.double())
    assert_close(y, yr, "y")
    assert_close(x.grad, xr.grad, "dx")
    assert_close(w.grad, wr.grad, "dW", atol=2e-3 * max(1.0, float(wr.grad.abs().max())))


def test_naylis_linear_module_swap(dev):
    """use_library_wgrad turns the bias-free nn.Linear of a block into
    NaylisLinear in place: same parameters and keys, the same forward and
    input gradient as nn.Linear, the weight gradient from the library (to the
    bf16 GEMM bound); a biased Linear is left alone."""
    from naylis_amd.mom_kernels.hip_linear import NaylisLinear, use_library_wgrad
    torch.manual_seed(7)
    block = torch.nn.Sequential(torch.nn.Linear(256, 704, bias=False), torch.nn.Linear(704, 256, bias=True))
    block = block.to(dev, torch.bfloat16)
    ref = copy.deepcopy(block)
    keys = list(block.state_dict())
    use_library_wgrad(block)
    assert type(block[0]) is NaylisLinear and type(block[1]) is torch.nn.Linear
    assert list(block.state_dict()) == keys
    x = torch.randn(2, 512, 256, device=dev, dtype=torch.bfloat16)
    dy = torch.randn(2, 512, 256, device=dev, dtype=torch.bfloat16)
    xa, xb = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    ya = block(xa)
    ya.backward(dy)
    hb = ref[0](xb)
    hb.retain_grad()
    yb = ref[1](hb)
    yb.backward(dy)
    assert torch.equal(ya, yb)
    assert_close(xa.grad, xb.grad, "dx")
    # the first layer's exact weight gradient from the bf16 gradient reaching it
    gw = torch.mm(hb.grad.reshape(-1, 704).float().t(), x.reshape(-1, 256).float())
    # bf16 output rounding (half an ulp, at most 2^-8 relative) plus the accumulation
    tol = 2.0 ** -8 * gw.abs() + 2e-3 * max(1.0, float(gw.abs().max()))
    assert bool(((block[0].weight.grad.float() - gw).abs() <= tol).all())
    assert bool(((ref[0].weight.grad.float() - gw).abs() <= tol).all())
    assert_close(block[1].weight.grad, ref[1].weight.grad, "dW (nn.Linear)")


def test_shared_input_linear_matches_separate_layers(dev):
    """shared_input_linear (q/k/v, gate/up of the decoder): the same outputs as
    applying the layers one by one; the input gradient is the sum of the
    products accumulated in one GEMM epilogue (close to autograd's sum of
    rounded products), weight gradients to the bf16 GEMM bound."""
    from naylis_amd.mom_kernels.hip_linear import shared_input_linear
    torch.manual_seed(11)
    layers = [torch.nn.Linear(256, n, bias=False).to(dev, torch.bfloat16) for n in (256, 512, 256)]
    x = torch.randn(2, 512, 256, device=dev, dtype=torch.bfloat16)
    dys = [torch.randn(2, 512, m.out_features, device=dev, dtype=torch.bfloat16) for m in layers]
    xa = x.clone().requires_grad_(True)
    outs = shared_input_linear(xa, layers)
    torch.autograd.backward(outs, dys)
    wgrads = [m.weight.grad.clone() for m in layers]
    for m in layers:
        m.weight.grad = None
    for o, m in zip(outs, layers):
        assert torch.equal(o, m(x))
    x32 = x.reshape(-1, 256).float()
    parts = [torch.mm(d.reshape(-1, m.out_features).float(), m.weight.detach().float()) for d, m in zip(dys, layers)]
    dx = sum(parts)
    # three bf16 roundings of partial sums (here, and in autograd's sum of rounded products), each at most
    # 2^-9 of the sum of the products' magnitudes, plus the GEMMs' accumulation
    tol = 2.0 ** -7 * sum(q.abs() for q in parts) + 1e-3
    assert bool(((xa.grad.reshape(-1, 256).float() - dx).abs() <= tol).all())
    # and no further from the fp32 sum than autograd's own sum over the separate layers
    xb = x.clone().requires_grad_(True)
    torch.autograd.backward([m(xb) for m in layers], dys)
    err_lib = float((xa.grad.reshape(-1, 256).float() - dx).abs().max())
    err_torch = float((xb.grad.reshape(-1, 256).float() - dx).abs().max())
    assert err_lib <= 1.5 * err_torch + 1e-3, (err_lib, err_torch)
    for d, m, g in zip(dys, layers, wgrads):
        gw = torch.mm(d.reshape(-1, m.out_features).float().t(), x32)
        tol = 2.0 ** -8 * gw.abs() + 2e-3 * max(1.0, float(gw.abs().max()))
        assert bool(((g.float() - gw).abs() <= tol).all())
    # no grad: the plain layers
    with torch.no_grad():
        outs = shared_input_linear(x, layers)
    assert all(o.grad_fn is None for o in outs)
