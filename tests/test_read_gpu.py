"""GPU parity of the HIP gated flash read (forward + backward) against the
CPU fp32 oracle on identical bf16 inputs.

Mirrors the reference's checks tests/test_parity.py:460-490 (§20a/§20b:
flash read vs eager reference, then dq/dk/dv/d gates vs eager autograd) at
the suite shapes (B=2, S=64, H=2, hd=16, 4 blocks x 16 slots, top-2 with
duplicate ids allowed, test_parity.py:74-77,144) and at wider geometries:
block-aligned fast paths (block_size 32/64/128), ragged S, head_dim
16..128, top_k 1..3, 32 blocks.  Every case calls through the C ABI.
"""
import pytest
import torch
import torch.nn.functional as F

import oracle
from tests._tol import assert_close, scaled_max

pytestmark = pytest.mark.gpu

CASES = [
    # B, S, H, HD, NB, BS, topk, routing
    (2, 64, 2, 16, 4, 16, 2, "random"),      # reference suite shapes (unaligned path)
    (2, 64, 2, 16, 2, 64, 2, "random"),      # test_parity §5b geometry
    (2, 100, 4, 32, 4, 32, 2, "random"),     # ragged S, SG=32 aligned
    (1, 300, 2, 64, 8, 128, 2, "distinct"),  # config-2 geometry, ragged
    (2, 256, 4, 64, 8, 128, 2, "smooth"),    # router-like smooth routing
    (2, 130, 2, 128, 4, 64, 2, "distinct"),  # head_dim 128
    (1, 128, 2, 64, 4, 64, 1, "random"),     # top-1
    (1, 192, 2, 64, 8, 32, 3, "distinct"),   # top-3
    (1, 256, 2, 64, 32, 128, 2, "distinct"), # 32 blocks (config-4 geometry)
    (1, 96, 2, 32, 3, 48, 2, "random"),      # block_size 48: not a multiple of 32
    # the pair-tiled path (head_dim 64, 128-slot blocks, top-2, at most 8 blocks)
    (2, 200, 2, 64, 4, 128, 2, "random"),    # duplicate ids: one-block pairs, ragged tiles
    (1, 2048, 4, 64, 8, 128, 2, "distinct"), # many ranges per head, ranges crossing pairs
]


def make_inputs(B, S, H, HD, NB, BS, topk, routing, seed=8):
    g = torch.Generator().manual_seed(seed)
    L, D = NB * BS, H * HD
    q = (torch.randn(B, S, H, HD, generator=g) * 0.7).bfloat16()
    k = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    v = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    gates = F.softmax(torch.randn(B, S, topk, generator=g), -1)
    if routing == "random":
        top = torch.randint(0, NB, (B, S, topk), generator=g)          # duplicates allowed
    elif routing == "distinct":
        top = torch.argsort(torch.rand(B, S, NB, generator=g), -1)[..., :topk]
    else:  # smooth: slowly varying logits over the sequence, like the prefix-mean router
        base = torch.randn(B, 1, NB, generator=g) * 2.0
        drift = torch.cumsum(torch.randn(B, S, NB, generator=g) * 0.05, 1)
        top = (base + drift).topk(topk, -1).indices
    dout = torch.randn(B, S, H, HD, generator=g).bfloat16()
    return q, k, v, top, gates, dout


def oracle_read(q, k, v, top, gates, dout, NB, BS):
    qf = q.float().requires_grad_(True)
    kf = k.float().requires_grad_(True)
    vf = v.float().requires_grad_(True)
    gf = gates.clone().requires_grad_(True)
    out = oracle.mom_read(qf, kf, vf, top, gf, num_blocks=NB, block_size=BS)
    out.backward(dout.float())
    return out.detach(), qf.grad, kf.grad, vf.grad, gf.grad


@pytest.mark.parametrize("case", CASES, ids=[f"B{c[0]}S{c[1]}H{c[2]}hd{c[3]}E{c[4]}bs{c[5]}k{c[6]}{c[7]}" for c in CASES])
def test_read_fwd_bwd_matches_oracle(case, dev):
    from naylis_amd import mom_kernels
    B, S, H, HD, NB, BS, topk, routing = case
    q, k, v, top, gates, dout = make_inputs(*case)
    ref = oracle_read(q, k, v, top, gates, dout, NB, BS)

    qd = q.to(dev).requires_grad_(True)
    kd = k.to(dev).requires_grad_(True)
    vd = v.to(dev).requires_grad_(True)
    gd = gates.to(dev).requires_grad_(True)
    out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16 and out.shape == (B, S, H, HD)
    assert_close(out, ref[0], "out")
    assert_close(qd.grad, ref[1], "dq")
    assert_close(kd.grad, ref[2], "dk")
    assert_close(vd.grad, ref[3], "dv")
    assert_close(gd.grad, ref[4], "d_gates")
    # the reference's own metric (test_parity.py:488-490); a gradient that is
    # identically zero in exact arithmetic (the gates of a top-1 read) has no
    # scale to measure against and is covered by the elementwise bound above
    worst = max(scaled_max(a, b) for a, b in zip((qd.grad, kd.grad, vd.grad, gd.grad), ref[1:])
                if float(b.abs().max()) > 1e-4)
    assert worst < 2e-2, worst


@pytest.mark.parametrize("big_block,BS", [(1, 64), (0, 64), (1, 128), (0, 128)])
def test_read_score_jump_moves_the_reference(big_block, BS, dev):
    """Every token selects blocks 0 and 1; the scores of one block sit about
    2^138 above the other's in p.  With the large block second, the forward's
    reference (set from a score of the token's first selected chunk) is far
    below it: without moving the reference p would be inf.  With the large
    block first, the second block's p underflow towards zero.  Forward and
    backward against the fp32 oracle.  All the weight lands on one block, so
    the gates' true gradient is ~0: the backward must normalise its recomputed
    weights by their sum (the forward's lse carries the rounding of its bf16
    row sum) for the gate gradient to come out ~0 too.  128-slot blocks take
    the pair-tiled kernels, whose delta comes from o and its bf16 remainder."""
    from naylis_amd import mom_kernels
    B, S, H, HD, NB = 1, 128, 2, 64, 4
    g = torch.Generator().manual_seed(21)
    L, D = NB * BS, H * HD
    q = (1.0 + 0.1 * torch.randn(B, S, H, HD, generator=g)).bfloat16()
    k = 0.3 * torch.randn(L, D, generator=g)
    k[big_block * BS:(big_block + 1) * BS] += 12.0   # scores ~ 64 * 12 / 8 = 96 (log2: 138)
    k = k.bfloat16()
    v = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    gates = F.softmax(torch.randn(B, S, 2, generator=g), -1)
    top = torch.tensor([0, 1]).expand(B, S, 2).clone()
    top[:, ::3] = torch.tensor([1, 0])                # both selection orders
    dout = torch.randn(B, S, H, HD, generator=g).bfloat16()
    ref = oracle_read(q, k, v, top, gates, dout, NB, BS)
    qd, kd, vd, gd = (t.to(dev).requires_grad_(True) for t in (q, k, v, gates))
    out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    assert_close(out, ref[0], "out")
    # every k of the large block carries the same offset (12 in each feature),
    # so an error in sum_n dS_n (the bf16 rounding of dS; the delta taken from
    # the forward's bf16 output) reaches dq as one shift of all its features,
    # 12/8 times larger: compare dq with its feature mean removed
    dq = qd.grad.float().cpu()
    assert_close(dq - dq.mean(-1, keepdim=True), ref[1] - ref[1].mean(-1, keepdim=True), "dq")
    for got, want, name in zip((kd.grad, vd.grad, gd.grad), ref[2:], ("dk", "dv", "d_gates")):
        assert_close(got, want, name)


def test_read_deterministic(dev):
    from naylis_amd import mom_kernels
    case = (2, 256, 4, 64, 8, 128, 2, "smooth")
    q, k, v, top, gates, dout = make_inputs(*case)
    res = []
    for _ in range(2):
        qd = q.to(dev).requires_grad_(True)
        kd = k.to(dev).requires_grad_(True)
        vd = v.to(dev).requires_grad_(True)
        gd = gates.to(dev).requires_grad_(True)
        out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=8, block_size=128, mode="hip")
        out.backward(dout.to(dev))
        res.append([t.detach().clone() for t in (out, qd.grad, kd.grad, vd.grad, gd.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("case", [(2, 256, 4, 64, 8, 128, 2, "distinct"),   # pair-tiled backward
                                  (2, 100, 4, 32, 4, 32, 2, "random")])    # two-pass backward
def test_read_tiny_gradients_keep_their_precision(case, dev):
    """An upstream gradient of 2^-20 (a layer loss's mean over many
    elements gives such scales) scales every gradient by 2^-20 and keeps
    the relative bar: no product may flush it (fp16 operands would, below
    2^-14).  The bound is the parity bar with atol scaled alike."""
    from naylis_amd import mom_kernels
    B, S, H, HD, NB, BS, topk, routing = case
    q, k, v, top, gates, dout = make_inputs(*case)
    dout = (dout.float() * 2.0 ** -20).bfloat16()
    ref = oracle_read(q, k, v, top, gates, dout, NB, BS)
    qd = q.to(dev).requires_grad_(True)
    kd = k.to(dev).requires_grad_(True)
    vd = v.to(dev).requires_grad_(True)
    gd = gates.to(dev).requires_grad_(True)
    out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
    out.backward(dout.to(dev))
    torch.cuda.synchronize()
    atol = 2e-3 * 2.0 ** -20
    for name, got, want in (("dq", qd.grad, ref[1]), ("dk", kd.grad, ref[2]), ("dv", vd.grad, ref[3]),
                            ("d_gates", gd.grad, ref[4])):
        assert float(want.abs().max()) > 0, name
        assert_close(got, want, name, atol=atol)


def test_read_empty_sequence(dev):
    from naylis_amd import mom_kernels
    q = torch.zeros(2, 0, 2, 16, dtype=torch.bfloat16, device=dev, requires_grad=True)
    k = torch.randn(64, 32, device=dev).bfloat16().requires_grad_(True)
    v = torch.randn(64, 32, device=dev).bfloat16().requires_grad_(True)
    top = torch.zeros(2, 0, 2, dtype=torch.long, device=dev)
    g = torch.zeros(2, 0, 2, device=dev, requires_grad=True)
    out = mom_kernels.mom_read(q, k, v, top, g, num_blocks=4, block_size=16, mode="hip")
    assert out.shape == (2, 0, 2, 16)
    out.sum().backward()
    torch.cuda.synchronize()
    assert float(k.grad.float().abs().sum()) == 0.0 and float(v.grad.float().abs().sum()) == 0.0


def test_read_single_block_gate_independence(dev):
    """A token whose k selections all name one block attends to that block
    alone, whatever the gate values (the bias is constant over the block).
    The gate enters the exp2 argument through two fp32 roundings, and P enters
    the P.V product in bf16, so a gate change can move one p across a bf16
    rounding boundary (2^-8 of p): the outputs agree to one bf16 ulp plus
    2^-8 of the largest |o| of the (token, head) row, not bitwise (an output
    that cancels, |o| << sum_n p_n |v_n|, shows that 2^-8 as several ulps)."""
    from naylis_amd import mom_kernels
    B, S, H, HD, NB, BS = 1, 128, 2, 64, 4, 64
    q, k, v, _, gates, _ = make_inputs(B, S, H, HD, NB, BS, 2, "random")
    top = torch.full((B, S, 2), 2, dtype=torch.long)
    g2 = F.softmax(torch.randn(B, S, 2, generator=torch.Generator().manual_seed(142)) * 3, -1)
    o1 = mom_kernels.mom_read(q.to(dev), k.to(dev), v.to(dev), top.to(dev), gates.to(dev),
                              num_blocks=NB, block_size=BS, mode="hip")
    o2 = mom_kernels.mom_read(q.to(dev), k.to(dev), v.to(dev), top.to(dev), g2.to(dev),
                              num_blocks=NB, block_size=BS, mode="hip")
    # one bf16 ulp of the larger of the two values (an ulp is at most 2^-7 of
    # the value; measuring against the smaller one fails spuriously when the
    # two round to neighbours on either side of a power of two), plus the
    # bf16 rounding of one P entry at the row's scale
    a, b = o1.float(), o2.float()
    row = torch.maximum(a.abs(), b.abs()).amax(-1, keepdim=True)
    assert bool(((a - b).abs() <= 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 2.0 ** -8 * row + 1e-6).all())


def test_read_full_config2_vs_torch_fp32(dev):
    """Config-2 shape (B=8, T=2048, H=16x64, bank 8x128, top-2) against a
    torch fp32 reference on the GPU (dense masked softmax), forward and
    backward."""
    from naylis_amd import mom_kernels
    B, S, H, HD, NB, BS, topk = 8, 2048, 16, 64, 8, 128, 2
    q, k, v, top, gates, dout = make_inputs(B, S, H, HD, NB, BS, topk, "smooth", seed=3)
    qd, kd, vd, gd = (t.to(dev).requires_grad_(True) for t in (q, k, v, gates))
    out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
    out.backward(dout.to(dev))
    qf, kf, vf, gf = (t.to(dev).float().requires_grad_(True) for t in (q, k, v, gates))
    ref = oracle.mom_read(qf, kf, vf, top.to(dev), gf, num_blocks=NB, block_size=BS)
    ref.backward(dout.to(dev).float())
    assert_close(out, ref, "out")
    assert_close(qd.grad, qf.grad, "dq")
    assert_close(kd.grad, kf.grad, "dk")
    assert_close(vd.grad, vf.grad, "dv")
    assert_close(gd.grad, gf.grad, "d_gates")


def test_read_dkdv_work_split_edges(dev):
    """The dK/dV pass cuts each head's (slot group, active tile) items into
    equal ranges that cross group boundaries.  Two heads give many short
    ranges; the routing leaves blocks 0-3 unselected (empty groups, zero
    dK/dV), gives block 4 to one token (a group inside one range), and
    spreads the rest unevenly (heavy groups over many ranges).  Against the
    fp32 oracle, and bitwise the same on a second run."""
    from naylis_amd import mom_kernels
    B, S, H, HD, NB, BS, topk = 2, 1536, 2, 64, 32, 128, 2
    g = torch.Generator().manual_seed(77)
    L, D = NB * BS, H * HD
    q = (torch.randn(B, S, H, HD, generator=g) * 0.7).bfloat16()
    k = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    v = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    gates = F.softmax(torch.randn(B, S, topk, generator=g), -1)
    w = torch.linspace(1.0, 8.0, NB - 5)                     # blocks 5..31, uneven popularity
    first = 5 + torch.multinomial(w, B * S * topk, replacement=True, generator=g).view(B, S, topk)
    top = first.clone()
    top[..., 1] = torch.where(top[..., 1] == top[..., 0], 5 + (top[..., 0] - 5 + 1) % (NB - 5), top[..., 1])
    top[1, 700, 1] = 4                                       # block 4: one token
    dout = torch.randn(B, S, H, HD, generator=g).bfloat16()
    res = []
    for _ in range(2):
        qd, kd, vd, gd = (t.to(dev).requires_grad_(True) for t in (q, k, v, gates))
        out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
        out.backward(dout.to(dev))
        res.append([t.detach().clone() for t in (out, qd.grad, kd.grad, vd.grad, gd.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)
    out, dq, dk, dv, dg = res[0]
    assert float(dk[:4 * BS].float().abs().max()) == 0.0 and float(dv[:4 * BS].float().abs().max()) == 0.0
    assert float(dv[4 * BS:5 * BS].float().abs().max()) > 0.0
    qf, kf, vf, gf = (t.to(dev).float().requires_grad_(True) for t in (q, k, v, gates))
    ref = oracle.mom_read(qf, kf, vf, top.to(dev), gf, num_blocks=NB, block_size=BS)
    ref.backward(dout.to(dev).float())
    assert_close(out, ref, "out")
    assert_close(dq, qf.grad, "dq")
    assert_close(dk, kf.grad, "dk")
    assert_close(dv, vf.grad, "dv")
    assert_close(dg, gf.grad, "d_gates")


def test_read_pair_path_edges(dev):
    """The pair-tiled kernels (head_dim 64, 128-slot blocks, top-2): two heads
    give many short backward ranges, each crossing several pairs (their
    dK / dV go out as (range, pair) partials); blocks 0 and 1 are never
    selected (zero dK / dV rows), block 2 by one token (a pair of one tile),
    the rest unevenly, with a few duplicate selections (one-block pairs).
    The library must take the pair path (its launches are timed under their
    own names), match the fp32 oracle and repeat bitwise."""
    from naylis_amd import _lib, mom_kernels
    B, S, H, HD, NB, BS, topk = 2, 1000, 2, 64, 8, 128, 2
    g = torch.Generator().manual_seed(91)
    L, D = NB * BS, H * HD
    q = (torch.randn(B, S, H, HD, generator=g) * 0.7).bfloat16()
    k = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    v = (torch.randn(L, D, generator=g) * 0.4).bfloat16()
    gates = F.softmax(torch.randn(B, S, topk, generator=g), -1)
    w = torch.tensor([1.0, 2.0, 3.0, 5.0, 8.0])             # blocks 3..7, uneven popularity
    top = 3 + torch.multinomial(w, B * S * topk, replacement=True, generator=g).view(B, S, topk)
    top[0, 17, 1] = 2                                        # block 2: one token
    dout = torch.randn(B, S, H, HD, generator=g).bfloat16()
    res = []
    for rep in range(2):
        qd, kd, vd, gd = (t.to(dev).requires_grad_(True) for t in (q, k, v, gates))
        with _lib.KernelTimer():
            out = mom_kernels.mom_read(qd, kd, vd, top.to(dev), gd, num_blocks=NB, block_size=BS, mode="hip")
            out.backward(dout.to(dev))
            torch.cuda.synchronize()
        names = _lib.KernelTimer.results()
        assert "read_bwd_pair" in names and "read_bwd_dq" not in names, sorted(names)
        res.append([t.detach().clone() for t in (out, qd.grad, kd.grad, vd.grad, gd.grad)])
    for a, b in zip(*res):
        assert torch.equal(a, b)
    out, dq, dk, dv, dg = res[0]
    assert float(dk[:2 * BS].float().abs().max()) == 0.0 and float(dv[:2 * BS].float().abs().max()) == 0.0
    assert float(dv[2 * BS:3 * BS].float().abs().max()) > 0.0
    qf, kf, vf, gf = (t.to(dev).float().requires_grad_(True) for t in (q, k, v, gates))
    ref = oracle.mom_read(qf, kf, vf, top.to(dev), gf, num_blocks=NB, block_size=BS)
    ref.backward(dout.to(dev).float())
    assert_close(out, ref, "out")
    assert_close(dq, qf.grad, "dq")
    assert_close(dk, kf.grad, "dk")
    assert_close(dv, vf.grad, "dv")
    assert_close(dg, gf.grad, "d_gates")
