"""GPU parity of the fused prefix-mean router (C ABI naylis_mom_router_*)
against the CPU oracle (model.py:169-220 restated in oracle.router).

* The fp32 prefix mean is bit-exact (torch.equal) with the CPU reference's
  cumsum / (t+1) — reference test_parity.py §2a/2b, probe.py A1.
* top_idx equals the oracle's on every token whose fp64 k-th / (k+1)-th
  logit margin exceeds tau = 1e-5 * max|logit| (a near-tie is decided by fp32
  GEMM rounding order, which no two implementations share); such tokens are
  counted and must be rare.
* logits / probs / gates to fp32 rounding; gradients dx, dW_down, dW_up
  against fp32 autograd of the oracle.
"""
import pytest
import torch

import oracle
from tests._tol import assert_close

pytestmark = pytest.mark.gpu


def make(B, T, D, R, E, dtype, seed=0, bias_blocks=None):
    g = torch.Generator().manual_seed(seed)
    w_down = torch.randn(R, D, generator=g) * 0.02
    w_up = torch.randn(E, R, generator=g) * 0.02
    x = torch.randn(B, T, D, generator=g)
    if dtype == torch.bfloat16:
        x = x.bfloat16()
    noise = None
    if bias_blocks is not None:
        # config-4 style additive logit bias: per (b, 128-token tile) a few
        # favoured blocks, through the additive noise hook of the router
        noise = torch.zeros(B, T, E)
        for b in range(B):
            for t0 in range(0, T, 128):
                n = int(torch.randint(bias_blocks[0], bias_blocks[1] + 1, (1,), generator=g))
                blk = torch.randperm(E, generator=g)[:n]
                noise[b, t0:t0 + 128, blk] = 1.0
    return x, w_down, w_up, noise


def fp64_margin(x, w_down, w_up, k, noise, scale):
    logits64, _, _, _, _ = oracle.router(x.double(), w_down.double(), w_up.double(), k,
                                         noise=None if noise is None else noise.double(), noise_scale=scale)
    noisy = logits64 if noise is None else logits64 + scale * noise.double()
    srt = noisy.sort(-1, descending=True).values
    return (srt[..., k - 1] - srt[..., k]), noisy.abs().max()


CASES = [
    (2, 64, 32, 8, 4, 2, torch.float32),      # reference suite shapes (router rank 8)
    (2, 512, 1024, 32, 8, 2, torch.float32),  # config 1
    (2, 300, 1024, 32, 8, 2, torch.bfloat16), # ragged T
    (8, 2048, 1024, 32, 8, 2, torch.bfloat16),# config 2
    (1, 256, 96, 16, 8, 3, torch.bfloat16),   # top-3, D not a multiple of 256
    (4, 4096, 1536, 32, 32, 2, torch.bfloat16),  # config 4: 12 K-steps per wave, two chunks per workgroup
    (2, 512, 256, 32, 32, 8, torch.bfloat16), # 32 blocks, top-8
    (1, 300, 128, 16, 64, 5, torch.bfloat16), # 64 blocks, top-5, ragged T
]


def test_router_prefix_mean_tiny_values(dev):
    """Prefix means in and near the fp32 subnormal range stay bit-exact
    (the kernel's reciprocal product hands nonzero subnormal quotients to
    the IEEE division; the fp64 partial sums of such inputs are exact, so the
    chunked summation order cannot matter)."""
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(5)
    B, T, D, R, E, k = 2, 4096, 64, 8, 4, 2
    x = torch.randn(B, T, D, generator=g) * 2.0 ** -128
    x[:, :, :8] = 0.0                                           # exact zeros
    x[0, :, 8:16] = torch.randint(-3, 4, (T, 8), generator=g).float() * 2.0 ** -149   # subnormal multiples
    w_down = torch.randn(R, D, generator=g) * 0.02
    w_up = torch.randn(E, R, generator=g) * 0.02
    *_, h = mom_kernels.mom_route(x.to(dev), w_down.to(dev), w_up.to(dev), k, return_h=True)
    torch.cuda.synchronize()
    r_h = oracle.prefix_mean(x)
    sub = (r_h != 0) & (r_h.abs() < torch.finfo(torch.float32).tiny)
    assert int(sub.sum()) > 1000, "the case must exercise subnormal prefix means"
    assert torch.equal(h.cpu(), r_h), f"{int((h.cpu() != r_h).sum())} prefix-mean values differ"


@pytest.mark.parametrize("want_h", [True, False], ids=["scan_x", "project_first"])
@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}T{c[1]}D{c[2]}R{c[3]}E{c[4]}k{c[5]}{str(c[6])[6:]}" for c in CASES])
def test_router_forward(case, want_h, dev):
    """With h requested the router scans x and h is bit-exact; without it,
    bf16 x with D % 128 == 0 takes the project-first path (y = x W_down^T on
    exact three-plane bf16 MFMA, fp64 prefix over the R-wide y); both must
    meet the same index / logit criteria."""
    from naylis_amd import mom_kernels
    B, T, D, R, E, k, dtype = case
    x, w_down, w_up, _ = make(B, T, D, R, E, dtype)
    out = mom_kernels.mom_route(x.to(dev), w_down.to(dev), w_up.to(dev), k, return_h=want_h)
    torch.cuda.synchronize()
    logits, probs, idx, gates = out[:4]
    r_logits, r_probs, r_idx, r_gates, r_h = oracle.router(x, w_down, w_up, k)
    if want_h:
        # bit-exact prefix mean
        h = out[4]
        assert torch.equal(h.cpu(), r_h), f"prefix mean differs: max {float((h.cpu() - r_h).abs().max())}"
        assert torch.equal(h[:, 0].cpu(), x[:, 0].float())
    # indices: exact outside near-ties
    margin, scale = fp64_margin(x, w_down, w_up, k, None, 1.0)
    tau = 1e-5 * float(scale)
    clear = margin > tau
    mism = (idx.cpu().long() != r_idx).any(-1)
    assert not (mism & clear).any(), f"{int((mism & clear).sum())} clear-margin tokens route differently"
    # near-ties (fp64 margin below tau) may go either way; they stay rare
    assert int(mism.sum()) <= max(2, B * T // 1000), f"{int(mism.sum())} near-tie tokens route differently"
    print(f"near-tie tokens: {int((~clear).sum())}, of which routed differently: {int(mism.sum())}")
    same = ~mism
    assert_close(logits.cpu(), r_logits, "logits", rtol=1e-4, atol=1e-6)
    assert_close(probs.cpu(), r_probs, "probs", rtol=1e-4, atol=1e-6)
    assert_close(gates.cpu()[same], r_gates[same], "gates", rtol=1e-4, atol=1e-6)


def test_router_noise_hook_and_config4_bias(dev):
    """Additive noise (Gumbel / logit bias) re-ranks top-k only; probs stay
    the clean softmax (model.py:209-220)."""
    from naylis_amd import mom_kernels
    B, T, D, R, E, k = 2, 512, 256, 32, 32, 2
    x, w_down, w_up, noise = make(B, T, D, R, E, torch.bfloat16, seed=3, bias_blocks=(3, 6))
    noise = noise * 10.0
    logits, probs, idx, gates = mom_kernels.mom_route(x.to(dev), w_down.to(dev), w_up.to(dev), k,
                                                      noise=noise.to(dev), noise_scale=0.5)
    r_logits, r_probs, r_idx, r_gates, _ = oracle.router(x, w_down, w_up, k, noise=noise, noise_scale=0.5)
    margin, scale = fp64_margin(x, w_down, w_up, k, noise, 0.5)
    clear = margin > 1e-5 * float(scale)
    mism = (idx.cpu().long() != r_idx).any(-1)
    assert not (mism & clear).any()
    assert_close(probs.cpu(), r_probs, "probs", rtol=1e-4, atol=1e-6)
    assert_close(gates.cpu()[~mism], r_gates[~mism], "gates", rtol=1e-4, atol=1e-6)
    # every selected block is among the biased ones for this tile
    assert bool((noise.gather(-1, idx.cpu().long()) > 0).all())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 64, 32, 8, 4, 2), (2, 384, 1024, 32, 8, 2), (1, 200, 96, 16, 8, 3),
                                   # T a multiple of 256 (bf16: the dx kernel forms W~ itself), R < 32
                                   (2, 512, 256, 16, 8, 2),
                                   # chunk sums staged in two blocks (143 later chunks > 4096 / R)
                                   (1, 4608, 128, 32, 8, 2)])
def test_router_backward(shape, dtype, dev):
    from naylis_amd import mom_kernels
    B, T, D, R, E, k = shape
    x, w_down, w_up, _ = make(B, T, D, R, E, dtype, seed=5)
    g = torch.Generator().manual_seed(9)
    dg = torch.randn(B, T, k, generator=g)
    dp = torch.randn(B, T, E, generator=g) * 0.1
    dlg = torch.randn(B, T, E, generator=g) * 0.1

    xd = x.to(dev).requires_grad_(True)
    wdd = w_down.to(dev).requires_grad_(True)
    wud = w_up.to(dev).requires_grad_(True)
    logits, probs, idx, gates = mom_kernels.mom_route(xd, wdd, wud, k)
    (gates * dg.to(dev)).sum().add((probs * dp.to(dev)).sum()).add((logits * dlg.to(dev)).sum()).backward()

    xr = x.float().requires_grad_(True)
    wdr = w_down.clone().requires_grad_(True)
    wur = w_up.clone().requires_grad_(True)
    r_logits, r_probs, r_idx, r_gates, _ = oracle.router(xr, wdr, wur, k)
    assert torch.equal(idx.cpu().long(), r_idx), "routing differs; pick another seed for this check"
    (r_gates * dg).sum().add((r_probs * dp).sum()).add((r_logits * dlg).sum()).backward()

    assert_close(xd.grad, xr.grad.to(x.dtype) if dtype == torch.bfloat16 else xr.grad, "dx")
    smax = float(wdr.grad.abs().max())
    assert_close(wdd.grad, wdr.grad, "dW_down", rtol=1e-3, atol=1e-4 * smax)
    umax = float(wur.grad.abs().max())
    assert_close(wud.grad, wur.grad, "dW_up", rtol=1e-3, atol=1e-4 * umax)


def test_router_causal(dev):
    """Routing of tokens <= t ignores tokens > t (test_parity.py §3a)."""
    from naylis_amd import mom_kernels
    x, w_down, w_up, _ = make(2, 512, 256, 32, 8, torch.bfloat16, seed=11)
    a = mom_kernels.mom_route(x.to(dev), w_down.to(dev), w_up.to(dev), 2, return_h=True)
    x2 = x.clone()
    x2[:, 301:] += 1.0
    b = mom_kernels.mom_route(x2.to(dev), w_down.to(dev), w_up.to(dev), 2, return_h=True)
    for ta, tb in zip(a, b):
        assert torch.equal(ta[:, :301], tb[:, :301])


def test_router_backward_accumulates_dx(dev):
    """dx_accumulate = 1 adds the router's input gradient to the dx the
    caller passes (the layer folds the query projection's dx in this way);
    it matches the plain gradient plus that dx to one bf16 rounding."""
    from naylis_amd import _lib, mom_kernels
    lib = _lib.load()
    B, T, D, R, E, k = 2, 384, 1024, 32, 8, 2
    x, w_down, w_up, _ = make(B, T, D, R, E, torch.bfloat16, seed=5)
    g = torch.Generator().manual_seed(9)
    dg = torch.randn(B, T, k, generator=g).to(dev)
    xd = x.to(dev)
    wd, wu = w_down.to(dev), w_up.to(dev)
    logits, probs, idx, gates = mom_kernels.mom_route(xd, wd, wu, k)
    act = torch.empty(B, T, R, device=dev)
    # recompute the forward's saved activation through the C ABI
    nbytes = lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, k)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    lg, pr, ti, tg = (torch.empty_like(t) for t in (logits, probs, idx, gates))
    st = _lib.stream_of(dev)
    assert lib.naylis_mom_router_fwd(xd.data_ptr(), 1, wd.data_ptr(), wu.data_ptr(), None, 0, 1.0, lg.data_ptr(),
                                     pr.data_ptr(), ti.data_ptr(), tg.data_ptr(), act.data_ptr(), None,
                                     ws.data_ptr(), nbytes, B, T, D, R, E, k, st) == 0
    prior = (torch.randn(B, T, D, generator=g) * 0.01).bfloat16().to(dev)
    outs = []
    for acc in (0, 1):
        dx = prior.clone() if acc else torch.empty_like(xd)
        dwd = torch.empty(R, D, device=dev)
        dwu = torch.empty(E, R, device=dev)
        rc = lib.naylis_mom_router_bwd(xd.data_ptr(), 1, wd.data_ptr(), wu.data_ptr(), act.data_ptr(), pr.data_ptr(),
                                       ti.data_ptr(), tg.data_ptr(), dg.data_ptr(), None, E, None, dx.data_ptr(), acc,
                                       dwd.data_ptr(), dwu.data_ptr(), ws.data_ptr(), nbytes, B, T, D, R, E, k, st)
        assert rc == 0, lib.naylis_mom_last_error()
        outs.append((dx, dwd, dwu))
    torch.cuda.synchronize()
    plain, accd = outs
    ref = plain[0].float() + prior.float()
    err = (accd[0].float() - ref).abs()
    # two bf16 roundings (of the plain gradient, and of the sum) at most
    bound = 2.0 ** -8 * (plain[0].float().abs() + prior.float().abs() + ref.abs()) + 1e-6
    assert bool((err <= bound).all()), f"max err {float(err.max())}"
    assert torch.equal(plain[1], accd[1]) and torch.equal(plain[2], accd[2])
    # fp32 x cannot accumulate: rejected before any device work
    xf = x.float().to(dev)
    rc = lib.naylis_mom_router_bwd(xf.data_ptr(), 0, wd.data_ptr(), wu.data_ptr(), act.data_ptr(), pr.data_ptr(),
                                   ti.data_ptr(), tg.data_ptr(), dg.data_ptr(), None, E, None, xf.data_ptr(), 1,
                                   dwd.data_ptr(), dwu.data_ptr(), ws.data_ptr(), nbytes, B, T, D, R, E, k, st)
    assert rc == _lib.NAYLIS_ERR_ARG


@pytest.mark.parametrize("B,T,D,R,E,k,with_noise", [
    (8, 2048, 1024, 32, 8, 2, False),   # config 2
    (4, 4096, 1536, 32, 32, 2, True),   # config 4 shape, additive logit noise
    (2, 512, 256, 16, 8, 2, True),      # rank 16, two sequences of 16 chunks
])
@pytest.mark.parametrize("spin", [None, 0, 1])
def test_router_one_launch_matches_two_launches(B, T, D, R, E, k, with_noise, spin, dev):
    """The forward in one launch (workgroups publish their chunks' fp64 sums
    to the later chunks' workgroups) against the two launches (projection,
    then head) that the same call makes under stream capture: logits, probs,
    top_idx, gates and act bitwise equal.  A launch on other data through the
    same workspace first leaves published sums of another epoch behind, which
    the checked launch must not take; the captured graph is replayed twice
    with eager launches between, every replay checked.  spin sets the one
    launch's poll bound from the host: 0 makes every workgroup project all
    earlier chunks itself (the fallback for sums still missing at the bound),
    1 mixes taken and re-projected blocks; None keeps the default bound."""
    from naylis_amd import _lib
    lib = _lib.load()
    if spin is not None:
        prev = lib.naylis_mom_spin_limit(spin)
        try:
            _one_launch_vs_two(lib, _lib, B, T, D, R, E, k, with_noise, dev)
        finally:
            assert lib.naylis_mom_spin_limit(prev) == spin
    else:
        _one_launch_vs_two(lib, _lib, B, T, D, R, E, k, with_noise, dev)


def _one_launch_vs_two(lib, _lib, B, T, D, R, E, k, with_noise, dev):
    x, w_down, w_up, noise = make(B, T, D, R, E, torch.bfloat16, seed=11, bias_blocks=(1, 3) if with_noise else None)
    x_other, _, _, _ = make(B, T, D, R, E, torch.bfloat16, seed=12)
    xd, xo, wd, wu = x.to(dev), x_other.to(dev), w_down.to(dev), w_up.to(dev)
    nz = noise.to(dev) if noise is not None else None
    nbytes = lib.naylis_mom_router_workspace_bytes(B, T, D, R, E, k)

    def outputs():
        return (torch.empty(B, T, E, device=dev), torch.empty(B, T, E, device=dev),
                torch.empty(B, T, k, dtype=torch.int32, device=dev), torch.empty(B, T, k, device=dev),
                torch.empty(B, T, R, device=dev))

    def call(xin, outs, ws):
        lg, pr, ti, tg, act = outs
        rc = lib.naylis_mom_router_fwd(xin.data_ptr(), 1, wd.data_ptr(), wu.data_ptr(),
                                       nz.data_ptr() if nz is not None else None, 0, 1.0, lg.data_ptr(),
                                       pr.data_ptr(), ti.data_ptr(), tg.data_ptr(), act.data_ptr(), None,
                                       ws.data_ptr(), nbytes, B, T, D, R, E, k, _lib.stream_of(dev))
        assert rc == 0, lib.naylis_mom_last_error()

    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    # small-integer words everywhere (consecutive 64-bit words differ in one low bit: their XOR is a
    # small number, which a plain launch counter used as the epoch could equal); then a launch on
    # other data, whose sums stay published in ws
    ws[:nbytes // 8 * 8].view(torch.int64)[:] = torch.arange(nbytes // 8, device=dev)
    ramp = outputs()
    call(xd, ramp, ws)               # one launch over the ramp
    call(xo, outputs(), ws)
    eager = outputs()
    call(xd, eager, ws)              # one launch
    for name, a, b in zip(("logits", "probs", "top_idx", "gates", "act"), eager, ramp):
        assert torch.equal(a, b), ("ramp", name)
    torch.cuda.synchronize()
    ws_cap = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    cap = outputs()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(xd, cap, ws_cap)        # under capture: the two launches
    for rep in range(2):
        for t in cap:
            t.zero_()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("logits", "probs", "top_idx", "gates", "act"), eager, cap):
            assert torch.equal(a, b), (rep, name)
        call(xo, outputs(), ws)      # eager work between the replays
        torch.cuda.synchronize()
