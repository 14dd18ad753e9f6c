"""GPU parity of the bank K/V GEMM and of the whole MoMLayer (router + bank +
read + projections) against the CPU oracle layer (model.py:71-276,
mom_kernels/reference.py:64-95), forward and backward.

Layer checks mirror the reference's tests/test_parity.py §1 (layer ==
reference), §3a (causality, bitwise), §13 (gradient checkpointing recomputes
exactly) and probe.py C1-C3 (gradients finite, router and bank alive).
"""
import pytest
import torch

import oracle
from tests._tol import assert_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("L,D_in,D_out", [(1024, 1024, 1024), (64, 32, 32), (144, 48, 48), (4096, 1536, 1536)])
def test_bank_kv(L, D_in, D_out, dev):
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(1)
    M = (torch.randn(L, D_in, generator=g) * 0.5).bfloat16()
    wk = (torch.randn(D_out, D_in, generator=g) * 0.03).bfloat16()
    wv = (torch.randn(D_out, D_in, generator=g) * 0.03).bfloat16()
    dk = torch.randn(L, D_out, generator=g).bfloat16()
    dv = torch.randn(L, D_out, generator=g).bfloat16()
    Md, wkd, wvd = (t.to(dev).requires_grad_(True) for t in (M, wk, wv))
    k, v = mom_kernels.mom_bank_kv(Md, wkd, wvd, mem_slots=L)
    torch.autograd.backward([k, v], [dk.to(dev), dv.to(dev)])
    Mr, wkr, wvr = (t.float().requires_grad_(True) for t in (M, wk, wv))
    kr, vr = oracle.bank_kv(Mr, wkr, wvr)
    torch.autograd.backward([kr, vr], [dk.float(), dv.float()])
    assert_close(k, kr, "K")
    assert_close(v, vr, "V")
    assert_close(Md.grad, Mr.grad, "dM")
    assert_close(wkd.grad, wkr.grad, "dW_k")
    assert_close(wvd.grad, wvr.grad, "dW_v")


def build_pair(D, H, NB, BS, K, R, seed=7, bank_scale=0.5, mom_scale=0.5):
    from naylis_amd.layer import MoMLayer
    torch.manual_seed(seed)
    layer = MoMLayer(d_model=D, n_heads=H, mem_size=NB * BS, block_size=BS, top_blocks=K, router_rank=R)
    layer.mom_scale.data.fill_(mom_scale)
    for lin in (layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
        lin.weight.data = lin.weight.data.bfloat16().float()  # identical bf16 values on both sides
    ref = oracle.OracleMoMLayer(D, H, NB * BS, BS, K, R)
    ref.load_state_dict(layer.state_dict())
    g = torch.Generator().manual_seed(seed + 1)
    M = (torch.randn(NB, BS * D, generator=g) * bank_scale).bfloat16()
    return layer, ref, M


LAYER_CASES = [
    # B, S, D, H, NB, BS, K, R
    (2, 64, 32, 2, 4, 16, 2, 8),       # reference suite shapes
    (2, 256, 256, 4, 8, 128, 2, 32),   # config-2 geometry, small
    (1, 300, 512, 8, 4, 64, 2, 32),    # ragged S
]


@pytest.mark.parametrize("case", LAYER_CASES, ids=[f"B{c[0]}S{c[1]}D{c[2]}H{c[3]}E{c[4]}bs{c[5]}" for c in LAYER_CASES])
def test_layer_fwd_bwd_matches_oracle(case, dev):
    B, S, D, H, NB, BS, K, R = case
    layer, ref, M = build_pair(D, H, NB, BS, K, R)
    layer.eval()
    ref.eval()
    ref.noise_scale = 0.0
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, S, D, generator=g).bfloat16()
    dy = torch.randn(B, S, D, generator=g).bfloat16()

    ld = layer.to(dev)
    for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
        lin.to(torch.bfloat16)
    xd = x.to(dev).requires_grad_(True)
    Md = M.to(dev).requires_grad_(True)
    y = ld(xd, Md)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()

    xr = x.float().requires_grad_(True)
    Mr = M.float().requires_grad_(True)
    yr = ref(xr, Mr)
    yr.backward(dy.float())

    # mom_scale * out promotes like the reference (model.py:239)
    assert y.dtype == torch.promote_types(ld.mom_scale.dtype, torch.bfloat16)
    assert_close(y, yr, "y")
    assert_close(xd.grad, xr.grad, "dx")
    assert_close(Md.grad, Mr.grad, "dM_blocks")
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "router_down", "router_up"):
        got = getattr(ld, name).weight.grad
        exp = getattr(ref, name).weight.grad
        assert_close(got, exp, f"d{name}", atol=2e-3 * max(1.0, float(exp.abs().max())))
    assert_close(ld.mom_scale.grad, ref.mom_scale.grad, "dmom_scale", atol=2e-3 * max(1.0, float(ref.mom_scale.grad.abs().max())))


def test_layer_causality_bitwise(dev):
    B, S, D, H, NB, BS, K, R = 2, 256, 256, 4, 8, 128, 2, 32
    layer, _, M = build_pair(D, H, NB, BS, K, R, seed=21)
    ld = layer.to(dev)
    for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
        lin.to(torch.bfloat16)
    ld.eval()
    x = torch.randn(B, S, D).bfloat16().to(dev)
    cut = S // 2
    with torch.no_grad():
        a = ld(x, M.to(dev))
        x2 = x.clone()
        x2[:, cut + 1:] += 1.0
        b = ld(x2, M.to(dev))
    assert torch.equal(a[:, :cut + 1], b[:, :cut + 1])


def test_layer_grad_ckpt_exact_and_alive(dev):
    B, S, D, H, NB, BS, K, R = 2, 256, 256, 4, 8, 128, 2, 32
    outs = []
    for ck in (False, True):
        layer, _, M = build_pair(D, H, NB, BS, K, R, seed=5)
        layer.mom_grad_ckpt = ck
        ld = layer.to(dev)
        for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
            lin.to(torch.bfloat16)
        ld.train()
        ld.noise_scale = 0.0
        x = torch.randn(B, S, D, generator=torch.Generator().manual_seed(2)).bfloat16().to(dev)
        Md = M.to(dev).requires_grad_(True)
        y = ld(x, Md)
        y.float().pow(2).mean().backward()
        outs.append((y.detach(), Md.grad.clone(), {n: p.grad.clone() for n, p in ld.named_parameters()}))
    (y0, m0, g0), (y1, m1, g1) = outs
    assert torch.equal(y0, y1)
    assert torch.equal(m0, m1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
        assert torch.isfinite(g0[n]).all(), n
    assert float(g0["router_up.weight"].abs().sum()) > 0
    assert float(m0.float().abs().sum()) > 0


def test_layer_fused_node_matches_modular(dev, monkeypatch):
    """The single-node layer (hip_layer.MomLayerFunction) against the
    modular autograd graph on the same inputs: forward bitwise, parameter
    gradients bitwise (same kernels in the same order), and dx within one
    bf16 rounding (the fused backward adds the router's fp32 input gradient
    before rounding; autograd adds two bf16 tensors)."""
    import naylis_amd.layer as layer_mod
    B, S, D, H, NB, BS, K, R = 2, 256, 256, 4, 8, 128, 2, 32
    res = []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(layer_mod, "fused_layer_supported", lambda *a, **k: False)
        layer, _, M = build_pair(D, H, NB, BS, K, R, seed=13)
        ld = layer.to(dev)
        for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
            lin.to(torch.bfloat16)
        ld.train()
        ld.noise_scale = 0.0
        g = torch.Generator().manual_seed(4)
        x = torch.randn(B, S, D, generator=g).bfloat16().to(dev).requires_grad_(True)
        dy = torch.randn(B, S, D, generator=g).to(dev)
        Md = M.to(dev).requires_grad_(True)
        y = ld(x, Md)
        # the load-balance aux loss reaches the router through the probs
        aux = layer_mod.mom_aux_loss([ld])
        (y * dy).sum().add(aux).backward()
        res.append((y.detach(), x.grad.clone(), Md.grad.clone(), {n: p.grad.clone() for n, p in ld.named_parameters()}))
    (y0, x0, m0, g0), (y1, x1, m1, g1) = res
    assert torch.equal(y0, y1)
    assert torch.equal(m0, m1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
    # dx is the sum of the q projection's and the router's parts; where they
    # cancel, the modular path's two separate bf16 roundings dominate, so the
    # difference is bounded by bf16 rounding at the gradient's scale
    err = (x0.float() - x1.float()).abs()
    scale = float(x1.float().abs().max())
    assert float(err.max()) <= 2.0 ** -7 * scale, (float(err.max()), scale)


EXT_CASES = [
    # B, S, D, H, NB, BS, K, R, bank dtype, external bank, router noise
    (2, 256, 256, 4, 8, 128, 2, 32, torch.bfloat16, False, False),  # pair-tiled read, bf16 bank
    (2, 256, 256, 4, 8, 128, 2, 32, torch.float32, False, True),    # fp32 bank gradient, uniform noise (Gumbel)
    (2, 256, 256, 4, 8, 128, 2, 32, torch.bfloat16, True, False),   # bank K/V from the caller
    (1, 131, 256, 2, 4, 64, 2, 16, torch.bfloat16, False, False),   # 131 tokens: the unsplit weight gradients
]


@pytest.mark.parametrize("case", EXT_CASES, ids=[f"case{i}" for i in range(len(EXT_CASES))])
def test_layer_torch_ext_matches_python_node(case, dev, monkeypatch):
    """The fused node's host side in C++ (csrc/torch_layer.cpp): the node as a
    C++ autograd function, and the Python node calling the extension once per
    direction, each against the Python statement (the same library and torch
    calls through ctypes): output, probs, routing and every gradient bitwise
    equal, with the aux loss reaching the router through the probs."""
    import naylis_amd.layer as layer_mod
    from naylis_amd import mom_kernels
    from naylis_amd.mom_kernels import hip_layer
    B, S, D, H, NB, BS, K, R, m_dtype, external, noise = case
    res = []
    for use_ext, cpp_node in ((True, True), (True, False), (False, False)):
        monkeypatch.setattr(hip_layer, "USE_TORCH_EXT", use_ext)
        monkeypatch.setattr(hip_layer, "USE_CPP_NODE", cpp_node)
        layer, _, M = build_pair(D, H, NB, BS, K, R, seed=31)
        ld = layer.to(dev)
        for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
            lin.to(torch.bfloat16)
        ld.train()
        ld.noise_scale = 1.0 if noise else 0.0
        g = torch.Generator().manual_seed(6)
        x = torch.randn(B, S, D, generator=g).bfloat16().to(dev).requires_grad_(True)
        dy = torch.randn(B, S, D, generator=g).to(dev)
        Md = M.to(m_dtype).to(dev).requires_grad_(True)
        torch.manual_seed(77)  # the router's noise draw
        torch.cuda.manual_seed(77)
        if external:
            kv = mom_kernels.mom_bank_kv_grouped(Md, [ld.k_proj.weight], [ld.v_proj.weight], mem_slots=NB * BS)[0]
            y = ld(x, Md, kv)
        else:
            y = ld(x, Md)
        idx = ld.last_top_idx.clone()  # (the aux loss consumes the layer's routing record)
        aux = layer_mod.mom_aux_loss([ld])
        (y * dy).sum().add(aux).backward()
        res.append((y.detach(), idx, x.grad.clone(), Md.grad.clone(),
                    {n: p.grad.clone() for n, p in ld.named_parameters() if p.grad is not None}))
    y1, i1, x1, m1, g1 = res[-1]  # the Python statement
    for mode, (y0, i0, x0, m0, g0) in zip(("C++ node", "extension calls"), res[:2]):
        assert torch.equal(i0, i1), mode
        assert torch.equal(y0, y1), mode
        assert torch.equal(x0, x1), mode
        assert torch.equal(m0, m1), mode
        assert g0.keys() == g1.keys(), mode
        for n in g0:
            assert torch.equal(g0[n], g1[n]), (mode, n)


@pytest.mark.parametrize("n,L,D", [(3, 1024, 1024), (20, 1024, 1024), (25, 512, 256)])
def test_bank_kv_grouped_matches_per_layer(n, L, D, dev):
    """The grouped projection of n layers that read one bank (the decoder's
    layers share model.M_blocks, model.py:409-416): every K_i, V_i, dW_k,i and
    dW_v,i bitwise equal to the per-layer call, and the bank gradient equal to
    the per-layer fp32 bank gradients added in layer order (25 layers run as
    two groups of at most 24, whose two sums autograd adds)."""
    from naylis_amd import mom_kernels
    g = torch.Generator().manual_seed(n)
    M = torch.randn(L, D, generator=g) * 0.5  # fp32 bank: its gradient stays fp32
    wk = [(torch.randn(D, D, generator=g) * 0.03).bfloat16() for _ in range(n)]
    wv = [(torch.randn(D, D, generator=g) * 0.03).bfloat16() for _ in range(n)]
    dk = [torch.randn(L, D, generator=g).bfloat16() for _ in range(n)]
    dv = [torch.randn(L, D, generator=g).bfloat16() for _ in range(n)]
    Md = M.to(dev).requires_grad_(True)
    wkd = [w.to(dev).requires_grad_(True) for w in wk]
    wvd = [w.to(dev).requires_grad_(True) for w in wv]
    kv = mom_kernels.mom_bank_kv_grouped(Md, wkd, wvd, mem_slots=L)
    assert len(kv) == n
    torch.autograd.backward([t for pair in kv for t in pair],
                            [t.to(dev) for i in range(n) for t in (dk[i], dv[i])])
    ref_dm = None
    for i in range(n):
        Mi = M.to(dev).requires_grad_(True)
        wki, wvi = wk[i].to(dev).requires_grad_(True), wv[i].to(dev).requires_grad_(True)
        k, v = mom_kernels.mom_bank_kv(Mi, wki, wvi, mem_slots=L)
        torch.autograd.backward([k, v], [dk[i].to(dev), dv[i].to(dev)])
        assert torch.equal(kv[i][0], k) and torch.equal(kv[i][1], v), i
        assert torch.equal(wkd[i].grad, wki.grad) and torch.equal(wvd[i].grad, wvi.grad), i
        ref_dm = Mi.grad if ref_dm is None else ref_dm + Mi.grad
    assert Md.grad.dtype == torch.float32
    assert torch.equal(Md.grad, ref_dm)


@pytest.mark.parametrize("fused", [True, False])
def test_layer_external_bank_matches_own_projection(fused, dev, monkeypatch):
    """MoMLayer given its bank K/V from the grouped projection (as the decoder
    does) against the layer projecting M_blocks itself: output and every
    gradient (bank, projections, router, x) bitwise equal, on the fused node
    and on the modular path."""
    import naylis_amd.layer as layer_mod
    from naylis_amd import mom_kernels
    if not fused:
        monkeypatch.setattr(layer_mod, "fused_layer_supported", lambda *a, **k: False)
    B, S, D, H, NB, BS, K, R = 2, 256, 256, 4, 8, 128, 2, 32
    res = []
    for external in (False, True):
        layer, _, M = build_pair(D, H, NB, BS, K, R, seed=21)
        ld = layer.to(dev)
        for lin in (ld.q_proj, ld.k_proj, ld.v_proj, ld.o_proj):
            lin.to(torch.bfloat16)
        ld.train()
        ld.noise_scale = 0.0
        g = torch.Generator().manual_seed(5)
        x = torch.randn(B, S, D, generator=g).bfloat16().to(dev).requires_grad_(True)
        dy = torch.randn(B, S, D, generator=g).to(dev)
        Md = M.to(dev).requires_grad_(True)
        if external:
            kv = mom_kernels.mom_bank_kv_grouped(Md, [ld.k_proj.weight], [ld.v_proj.weight], mem_slots=NB * BS)[0]
            y = ld(x, Md, kv)
        else:
            y = ld(x, Md)
        (y * dy).sum().backward()
        res.append((y.detach(), x.grad.clone(), Md.grad.clone(),
                    {n: p.grad.clone() for n, p in ld.named_parameters()}))
    (y0, x0, m0, g0), (y1, x1, m1, g1) = res
    assert torch.equal(y0, y1)
    assert torch.equal(x0, x1)
    assert torch.equal(m0, m1)
    for n in g0:
        assert torch.equal(g0[n], g1[n]), n
