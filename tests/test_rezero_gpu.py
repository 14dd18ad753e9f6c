"""GPU checks of the ReZero output gate kernel (C ABI naylis_mom_rezero_*;
model.py:239 `self.mom_scale * out`) against fp64 torch on the same inputs:
y = s z, dz = s dy, ds = sum(dy z); ragged sizes, both dtypes, determinism."""
import pytest
import torch

from tests._tol import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,zdt,dydt", [
    (8 * 2048 * 1024, torch.bfloat16, torch.float32),   # config 2: o_proj output bf16, y fp32
    (1000003, torch.bfloat16, torch.bfloat16),          # ragged, bf16 upstream gradient
    (4099, torch.float32, torch.float32),
    (5, torch.float32, torch.bfloat16),
])
def test_rezero_matches_fp64(n, zdt, dydt, dev):
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(n % 1000)
    z = torch.randn(n, generator=g).to(zdt).to(dev).requires_grad_(True)
    s = torch.tensor([0.37], device=dev, requires_grad=True)
    dy = torch.randn(n, generator=g).to(dydt).to(dev)
    y = mom_kernels.mom_rezero(z, s)
    assert y.dtype == torch.float32
    y.backward(dy)
    zr = z.detach().double()
    assert_close(y, 0.37 * zr, "y", rtol=1e-6, atol=1e-7)
    assert_close(z.grad, (0.37 * dy.double()).to(zdt), "dz")
    ds_ref = (dy.double() * zr).sum()
    assert z.grad.dtype == zdt and s.grad.shape == (1,)
    assert abs(float(s.grad) - float(ds_ref)) <= 1e-5 * float((dy.double() * zr).abs().sum()) + 1e-6


def test_rezero_deterministic_and_zero_size(dev):
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(1)
    z = torch.randn(3 * 1024 * 1024, generator=g).bfloat16().to(dev)
    dy = torch.randn(3 * 1024 * 1024, generator=g).to(dev)
    grads = []
    for _ in range(2):
        zz = z.clone().requires_grad_(True)
        s = torch.tensor([1.5], device=dev, requires_grad=True)
        mom_kernels.mom_rezero(zz, s).backward(dy)
        grads.append((zz.grad.clone(), s.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    e = torch.zeros(0, device=dev, dtype=torch.bfloat16, requires_grad=True)
    s = torch.tensor([2.0], device=dev, requires_grad=True)
    mom_kernels.mom_rezero(e, s).backward(torch.zeros(0, device=dev))
    assert float(s.grad) == 0.0


@pytest.mark.parametrize("n,xdt,ydt", [
    (1024 * 1024, torch.bfloat16, torch.bfloat16),   # the o projection's weight, folded gate
    (1000003, torch.bfloat16, torch.float32),
    (4099, torch.float32, torch.bfloat16),
    (7, torch.float32, torch.float32),
])
def test_rezero_scale_matches_torch(n, xdt, ydt, dev):
    """naylis_mom_rezero_scale: y = s x rounded once to y's dtype, bitwise the
    fp32 product torch forms and rounds (round to nearest even)."""
    from naylis_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(n % 977)
    x = torch.randn(n, generator=g).to(xdt).to(dev)
    s = torch.tensor([0.37], device=dev)
    y = torch.empty(n, device=dev, dtype=ydt)
    dt = {torch.float32: 0, torch.bfloat16: 1}
    _lib.check(lib.naylis_mom_rezero_scale(x.data_ptr(), dt[xdt], s.data_ptr(), y.data_ptr(), dt[ydt], n,
                                           torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert torch.equal(y, (x.float() * s).to(ydt))


@pytest.mark.parametrize("N,D,s0", [(8 * 2048, 1024, 0.37), (300 * 8, 256, 0.0), (8, 256, 0.37), (64, 128, -0.6)])
def test_gated_linear_matches_fp64(N, D, s0, dev):
    """mom_gated_linear: y = s (o W^T) in fp32 as one GEMM on the scaled bf16
    weight W' = bf16(s W) (model.py:251 then 239), and its backward (d o, dW,
    ds) against fp64 torch on the same bf16 inputs.  The fold rounds W' where
    the reference rounds o W^T, so y's error is bounded by the weight
    rounding, 2^-9 |s| sum_j |o_j| |W_ij| per element (checked with a factor 2
    of margin), not by a fraction of |y|; d o = bf16(dy) W' adds the same
    rounding of dy and one bf16 rounding of the result.  s = 0 (the ReZero
    initial value) makes y and d o vanish while ds does not."""
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(N + D)
    o = torch.randn(N, D, generator=g).bfloat16().to(dev).requires_grad_(True)
    w = (torch.randn(D, D, generator=g) * D ** -0.5).bfloat16().to(dev).requires_grad_(True)
    s = torch.tensor([s0], device=dev, requires_grad=True)
    dy = torch.randn(N, D, generator=g).to(dev)
    y = mom_kernels.mom_gated_linear(o, w, s)
    assert y.dtype == torch.float32
    y.backward(dy)
    od, wd, dyd = o.detach().double(), w.detach().double(), dy.double()
    z = od @ wd.t()
    y_bound = 2.0 ** -8 * abs(s0) * (od.abs() @ wd.abs().t()) + 1e-6
    assert bool(((y.double() - s0 * z).abs() <= y_bound).all()), "y beyond the weight-rounding bound"
    do_ref = s0 * (dyd @ wd)
    do_bound = 2.0 ** -7 * abs(s0) * (dyd.abs() @ wd.abs()) + 2.0 ** -8 * do_ref.abs() + 1e-6
    assert bool(((o.grad.double() - do_ref).abs() <= do_bound).all()), "d o beyond its rounding bound"
    ref_dw = s0 * (dyd.t() @ od)
    assert_close(w.grad, ref_dw, "dW", atol=2e-3 * max(1.0, float(ref_dw.abs().max())))
    # ds = sum bf16(dy) . z: its error is the rounding of dy against z, at most 2^-9 sum |dy z|
    # (checked with a factor 2), plus fp32 accumulation
    ref_ds = float((dyd * z).sum())
    assert abs(float(s.grad) - ref_ds) <= 2.0 ** -8 * float((dyd * z).abs().sum()) + 1e-6


@pytest.mark.parametrize("N,D_in,D_out", [(8 * 2048, 1024, 1024), (2400, 256, 512), (0, 64, 64), (8, 256, 128),
                                          (64, 128, 256)])
def test_gated_wgrad_matches_two_steps(N, D_in, D_out, dev):
    """naylis_mom_gated_wgrad (dW' kept inside the split-K reduction, whose
    epilogue writes dw = bf16(s dW') and the partials of ds = sum(dW' w))
    against naylis_mom_linear_wgrad's fp32 dW' followed by naylis_mom_rezero_bwd
    over the weight.  dw is bitwise equal where both split K alike (config-2
    shape: 8 splits), else within one bf16 rounding; ds differs only in its
    fp32 summation order.  N = 0 gives zeros over poisoned outputs; N = 8 and
    64 fit one K split, where the gate epilogue must still run (its outputs
    start poisoned)."""
    from naylis_amd import _lib
    from naylis_amd.mom_kernels.hip_linear import library_wgrad
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(N + D_in)
    x = torch.randn(N, D_in, generator=g).bfloat16().to(dev)
    dy = torch.randn(N, D_out, generator=g).bfloat16().to(dev)
    w = (torch.randn(D_out, D_in, generator=g) * 0.05).bfloat16().to(dev)
    s = torch.tensor([0.37], device=dev)
    nb = int(lib.naylis_mom_gated_wgrad_workspace_bytes(N, D_in, D_out))
    assert nb > 0
    ws = torch.empty(nb, dtype=torch.uint8, device=dev)
    dw = torch.full((D_out, D_in), 7.0, device=dev, dtype=torch.bfloat16)
    ds = torch.full((1,), 7.0, device=dev)
    _lib.check(lib.naylis_mom_gated_wgrad(x.data_ptr() if N else None, dy.data_ptr() if N else None, w.data_ptr(),
                                          s.data_ptr(), dw.data_ptr(), ds.data_ptr(), ws.data_ptr(), nb, N, D_in,
                                          D_out, st))
    torch.cuda.synchronize()
    if N == 0:
        assert not dw.any() and float(ds) == 0.0
        return
    dwp = library_wgrad(lib, x, dy, torch.float32, dev, st)
    dw_ref = torch.empty_like(w)
    ds_ref = torch.empty(1, device=dev)
    rz = torch.empty(max(int(lib.naylis_mom_rezero_workspace_bytes(w.numel())), 1), dtype=torch.uint8, device=dev)
    _lib.check(lib.naylis_mom_rezero_bwd(dwp.data_ptr(), 0, w.data_ptr(), 1, s.data_ptr(), dw_ref.data_ptr(),
                                         ds_ref.data_ptr(), rz.data_ptr(), rz.numel(), w.numel(), st))
    torch.cuda.synchronize()
    if N == 8 * 2048:
        assert torch.equal(dw, dw_ref), f"{int((dw != dw_ref).sum())} elements differ"
    else:
        d = (dw.float() - dw_ref.float()).abs()
        # one bf16 rounding, plus the fp32 summation-order difference of dW' near zero
        assert bool((d <= 2.0 ** -7 * dw_ref.float().abs() + 1e-3).all()), f"max {float(d.max())}"
    mag = float((dwp.double() * w.double()).abs().sum())
    assert abs(float(ds) - float(ds_ref)) <= 1e-5 * mag + 1e-6
