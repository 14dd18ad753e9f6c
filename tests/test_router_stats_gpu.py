"""Router statistics and the Gumbel path on the GPU (model.py:209-213,
476-517; the reference's RNG-order check is test_parity.py:292-306).

* ``mom_router_stats`` against the reference's formulas (oracle.aux_loss /
  oracle.router_stats on the same probs and top_idx), and its gradient
  against torch autograd through those formulas.
* The in-kernel Gumbel transform of the uniform draw against torch's own
  -log(-log(u + 1e-9) + 1e-9): same selection, gates to the last-bit
  rounding of the two separately compiled logs.
* The layer consumes exactly one uniform draw of (B, S, E) per forward, at
  the point the reference draws it, so a seeded run routes as the seeded
  draw says.
"""
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _routing(N, E, k, seed, dead=0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(N, E, generator=g) * 2.0
    if dead:
        logits[:, E - dead:] -= 100.0          # these blocks are never in the top-k
    probs = torch.softmax(logits, -1)
    idx = logits.topk(k, -1).indices.to(torch.int32)
    return probs, idx


@pytest.mark.parametrize("N,E,k,dead", [(16384, 8, 2, 0), (1000, 8, 2, 3), (77, 32, 3, 5), (300, 64, 8, 0),
                                        (5, 4, 1, 2)])
def test_router_stats_match_reference_formulas(N, E, k, dead, dev):
    from naylis_amd import mom_kernels
    probs, idx = _routing(N, E, k, seed=N + E, dead=dead)
    stats = mom_kernels.mom_router_stats(probs.to(dev), idx.to(dev)).cpu()
    # model.py:495-507 on the CPU in fp64 (the oracle's formulas)
    aux = oracle.aux_loss(probs.double(), idx.long(), E)
    ent, dead_frac = oracle.router_stats(probs.double(), idx.long(), E)
    sel = (idx.long().unsqueeze(2) == torch.arange(E).view(1, 1, -1)).any(1)
    frac = sel.double().mean(0)
    mean_prob = probs.double().mean(0)
    assert torch.equal(stats[E:2 * E], frac.float())                  # counts / N, one rounding
    assert torch.allclose(stats[:E].double(), mean_prob, rtol=1e-6, atol=1e-9)
    assert abs(float(stats[2 * E]) - float(aux)) <= 1e-6 * float(aux)
    assert abs(float(stats[2 * E + 1]) - float(ent)) <= 1e-5 * float(ent) + 1e-7
    assert float(stats[2 * E + 2]) == float(dead_frac) == dead / E


def test_router_stats_closed_forms(dev):
    """Entropy and dead fraction where the mathematics fixes them: log E for
    uniform probs, 0 for one-hot probs, the binary entropy for a two-point
    distribution; blocks no token selects are dead (aux = k at uniform
    routing, the closed form of METHODOLOGY.md:90)."""
    from test_oracle import router_stats_closed_forms

    from naylis_amd import mom_kernels
    for probs, idx, E, ent_want, dead_want in router_stats_closed_forms():
        stats = mom_kernels.mom_router_stats(probs.to(dev), idx.to(torch.int32).contiguous().to(dev)).cpu()
        assert abs(float(stats[2 * E + 1]) - ent_want) <= 1e-6 * max(ent_want, 1.0), (float(stats[2 * E + 1]), ent_want)
        assert float(stats[2 * E + 2]) == dead_want
    probs, idx, E = router_stats_closed_forms()[0][:3]
    stats = mom_kernels.mom_router_stats(probs.to(dev), idx.to(torch.int32).contiguous().to(dev)).cpu()
    assert abs(float(stats[2 * E]) - idx.shape[1]) <= 1e-6


def test_router_stats_deterministic(dev):
    from naylis_amd import mom_kernels
    probs, idx = _routing(20000, 8, 2, seed=1)
    a = mom_kernels.mom_router_stats(probs.to(dev), idx.to(dev))
    b = mom_kernels.mom_router_stats(probs.to(dev), idx.to(dev))
    assert torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_router_stats_gradient_reaches_the_router(dtype, dev):
    """loss = aux + <c, mean_prob> through mom_router_stats (one broadcast row
    into the router backward) against the same loss written with torch ops on
    the router's probs (a dense (B, T, E) gradient), same router call."""
    from naylis_amd import mom_kernels
    B, T, D, R, E, k = 2, 300, 256, 32, 8, 2
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, T, D, generator=g).to(dtype).to(dev)
    wd0 = (torch.randn(R, D, generator=g) * 0.05).to(dev)
    wu0 = (torch.randn(E, R, generator=g) * 0.5).to(dev)
    c = torch.randn(E, generator=g).to(dev)
    grads = []
    for fused in (True, False):
        wd = wd0.clone().requires_grad_(True)
        wu = wu0.clone().requires_grad_(True)
        xg = x.clone().requires_grad_(True)
        _, probs, idx, _ = mom_kernels.mom_route(xg, wd, wu, k)
        p2 = probs.reshape(-1, E)
        i2 = idx.reshape(-1, k)
        if fused:
            stats = mom_kernels.mom_router_stats(p2, i2)
            loss = stats[2 * E] + (stats[:E] * c).sum()
        else:
            loss = oracle.aux_loss(p2, i2.long(), E) + (p2.mean(0) * c).sum()
        loss.backward()
        grads.append((float(loss.detach()), wd.grad, wu.grad, xg.grad.float()))
    torch.cuda.synchronize()
    (l0, a0, b0, x0), (l1, a1, b1, x1) = grads
    assert abs(l0 - l1) <= 1e-5 * abs(l1)
    for got, want in ((a0, a1), (b0, b1), (x0, x1)):
        err = float((got - want).norm() / want.norm())
        assert err <= (1e-2 if dtype == torch.bfloat16 and got is x0 else 1e-4), err


def test_gumbel_transform_in_kernel_matches_torch(dev):
    from naylis_amd import mom_kernels
    B, T, D, R, E, k = 2, 512, 256, 32, 8, 2
    g = torch.Generator().manual_seed(21)
    x = torch.randn(B, T, D, generator=g).bfloat16().to(dev)
    wd = (torch.randn(R, D, generator=g) * 0.05).to(dev)
    wu = (torch.randn(E, R, generator=g) * 0.5).to(dev)
    u = torch.rand(B, T, E, generator=g).to(dev)
    u[0, :8] = torch.tensor([0.0, 1e-12, 0.5, 0.9999999, 1e-9, 0.25, 0.75, 1e-3], device=dev).view(-1, 1)
    gumbel = -torch.log(-torch.log(u + 1e-9) + 1e-9)          # model.py:210, on the GPU
    a = mom_kernels.mom_route(x, wd, wu, k, noise=u, noise_scale=0.7, noise_is_uniform=True)
    b = mom_kernels.mom_route(x, wd, wu, k, noise=gumbel, noise_scale=0.7)
    torch.cuda.synchronize()
    # torch's elementwise log and the kernel's logf may round the last bit of
    # g differently (they are separately compiled); the selection must agree
    # and the gates to that rounding
    assert torch.equal(a[2], b[2])
    assert torch.equal(a[1], b[1])          # probs do not see the noise
    diff = float((a[3] - b[3]).abs().max())
    print(f"gates max |diff| {diff:.3e}, differing {int((a[3] != b[3]).sum())} of {a[3].numel()}")
    assert torch.allclose(a[3], b[3], rtol=1e-5, atol=1e-7)


def test_layer_draws_one_uniform_per_forward(dev):
    """Reference RNG order (test_parity.py:292-306): one rand of the logits'
    shape per layer forward, before anything else draws; a seeded forward
    routes exactly as the router with that seeded draw."""
    from naylis_amd import mom_kernels
    from naylis_amd.layer import MoMLayer
    B, S, D, H, E, BS, K, R = 2, 256, 256, 4, 8, 64, 2, 32
    torch.manual_seed(0)
    layer = MoMLayer(D, H, E * BS, BS, K, R).to(dev)
    for lin in (layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
        lin.to(torch.bfloat16)
    layer.train()
    layer.noise_scale = 1.0
    x = torch.randn(B, S, D, device=dev).bfloat16()
    M = (torch.randn(E, BS * D, device=dev) * 0.5).bfloat16()
    torch.manual_seed(1234)
    with torch.no_grad():
        layer(x, M)
    state_after = torch.cuda.get_rng_state(dev)
    idx_layer = layer.last_top_idx.view(B, S, K).clone()
    torch.manual_seed(1234)
    u = torch.rand((B, S, E), device=dev, dtype=torch.float32)
    assert torch.equal(torch.cuda.get_rng_state(dev), state_after)
    _, _, idx, _ = mom_kernels.mom_route(x, layer.router_down.weight, layer.router_up.weight, K, noise=u,
                                         noise_scale=1.0, noise_is_uniform=True)
    assert torch.equal(idx, idx_layer)
    # a different seed changes the routing (the noise is live)
    torch.manual_seed(99)
    with torch.no_grad():
        layer(x, M)
    assert not torch.equal(layer.last_top_idx.view(B, S, K), idx_layer)
