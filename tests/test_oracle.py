"""CPU pins of the oracle (oracle/mom_oracle.py) — no GPU needed.

Each oracle function is checked against something other than its own
formula: the reference's golden vectors (tests/golden/golden_mom.npz,
written from mom_kernels/reference.py), a C restatement (oracle/prefix_mean.c),
brute-force loops, fp64 evaluation, finite differences, closed forms and
invariants — chosen so that a dropped term, a wrong sign or index, or a
transposed operand fails one of them.
"""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden", "golden_mom.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN)  # allow_pickle defaults to False


@pytest.fixture(scope="module")
def c_oracle():
    lib = os.path.join(ROOT, "oracle", "_build", "liboracle.so")
    if not os.path.exists(lib):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    dll = ctypes.CDLL(lib)
    dll.naylis_oracle_prefix_mean_f32.argtypes = [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_long] * 3
    return dll


# ------------------------------------------------------------ golden vectors
def test_golden_gate_bias(gold):
    top = torch.from_numpy(gold["bias_top_idx"])
    g = torch.from_numpy(gold["bias_gates"])
    assert torch.equal(oracle.build_gate_bias(top, g, 4, 16, torch.float32), torch.from_numpy(gold["bias_fp32"]))
    assert torch.equal(oracle.build_gate_bias(top, g, 4, 16, torch.bfloat16), torch.from_numpy(gold["bias_bf16mask"]))


def test_golden_prefix_mean(gold):
    assert torch.equal(oracle.prefix_mean(torch.from_numpy(gold["pm_x"])), torch.from_numpy(gold["pm_h"]))
    xb = torch.from_numpy(gold["pm_xb_as_f32"]).bfloat16()
    assert torch.equal(oracle.prefix_mean(xb), torch.from_numpy(gold["pm_hb"]))


def test_golden_attention(gold):
    q, k, v = (torch.from_numpy(gold[n]) for n in ("att_q", "att_k", "att_v"))
    bias = torch.from_numpy(gold["bias_fp32"])
    ref = torch.from_numpy(gold["att_out"])
    # explicit-matmul restatement vs the reference's SDPA: fp32 rounding only
    torch.testing.assert_close(oracle.mom_attention(q, k, v, bias), ref, rtol=1e-5, atol=1e-6)
    kb = k.unsqueeze(0).expand(2, -1, -1).contiguous()
    vb = v.unsqueeze(0).expand(2, -1, -1).contiguous()
    torch.testing.assert_close(oracle.mom_attention(q, kb, vb, bias), torch.from_numpy(gold["att_out_batched"]),
                               rtol=1e-5, atol=1e-6)


def test_golden_full_layer(gold):
    layer = oracle.OracleMoMLayer(32, 2, 64, 16, 2, 8)
    sd = {k[len("layer."):]: torch.from_numpy(gold[k]) for k in gold.files if k.startswith("layer.")}
    layer.load_state_dict(sd)
    layer.eval()
    layer.noise_scale = 0.0
    x, M = torch.from_numpy(gold["layer_x"]), torch.from_numpy(gold["layer_M"])
    with torch.no_grad():
        y, probs, idx, gates = oracle.layer_forward(x, layer, M)
    assert torch.equal(idx.reshape(-1, 2), torch.from_numpy(gold["layer_top_idx"]).reshape(-1, 2))
    assert torch.equal(probs.reshape(-1, 4), torch.from_numpy(gold["layer_probs"]).reshape(-1, 4))
    assert torch.equal(gates.reshape(-1, 2), torch.from_numpy(gold["layer_top_gates"]).reshape(-1, 2))
    torch.testing.assert_close(y, torch.from_numpy(gold["layer_y"]), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------ prefix mean
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefix_mean_matches_c_restatement(c_oracle, dtype):
    torch.manual_seed(0)
    x = torch.randn(3, 700, 96).to(dtype)
    xf = x.float().contiguous()
    h_c = torch.empty_like(xf)
    c_oracle.naylis_oracle_prefix_mean_f32(xf.data_ptr(), h_c.data_ptr(), 3, 700, 96)
    assert torch.equal(oracle.prefix_mean(x), h_c)


def test_prefix_mean_closed_form_and_causality():
    torch.manual_seed(1)
    x = torch.randn(2, 257, 33)
    h = oracle.prefix_mean(x)
    assert torch.equal(h[:, 0], x[:, 0])                                   # test_parity §2a
    exact = np.cumsum(x.numpy().astype(np.float64), axis=1).astype(np.float32)
    exact = exact / np.arange(1, 258, dtype=np.float32).reshape(1, -1, 1)
    assert np.array_equal(h.numpy(), exact)
    manual = torch.stack([x[:, :t + 1].double().mean(1) for t in range(257)], 1)
    torch.testing.assert_close(h.double(), manual, rtol=0, atol=1e-5)      # test_parity §2b
    x2 = x.clone()
    x2[:, 100:] += 3.0
    assert torch.equal(oracle.prefix_mean(x2)[:, :100], h[:, :100])       # causality


# ------------------------------------------------------------ gate bias
def test_gate_bias_brute_force_with_duplicates():
    g = torch.Generator().manual_seed(3)
    B, S, K, NB, BS = 2, 9, 3, 5, 4
    top = torch.randint(0, NB, (B, S, K), generator=g)
    top[0, 0] = torch.tensor([2, 2, 4])                                      # a duplicate id
    gates = torch.softmax(torch.randn(B, S, K, generator=g), -1)
    gates[1, 1, 0] = 1e-12                                                   # below the clamp
    bias = oracle.build_gate_bias(top, gates, NB, BS, torch.float32)
    lo = float(torch.finfo(torch.float32).min)
    for b in range(B):
        for s in range(S):
            for n in range(NB * BS):
                blk = n // BS
                hits = [t for t in range(K) if int(top[b, s, t]) == blk]
                want = sum(math.log(max(float(gates[b, s, t]), 1e-9)) for t in hits) if hits else lo
                assert abs(float(bias[b, s, n]) - want) <= 1e-6 * max(1.0, abs(want)), (b, s, n)


# ------------------------------------------------------------ attention
def _gather_read_fp64(q, k, v, top, gates, NB, BS):
    """Brute force: softmax over only the token's selected slots, fp64, with
    the log-gates rounded to fp32 and summed in fp32 as the reference builds
    them (reference.py:23-27)."""
    B, S, H, hd = q.shape
    out = torch.zeros(B, S, H, hd, dtype=torch.float64)
    for b in range(B):
        for s in range(S):
            bias = {}
            for t in range(top.shape[-1]):
                e = int(top[b, s, t])
                lg = np.float32(math.log(max(float(gates[b, s, t]), 1e-9)))
                bias[e] = np.float32(bias.get(e, np.float32(0.0)) + lg)
            slots = [n for e in sorted(bias) for n in range(e * BS, (e + 1) * BS)]
            for h in range(H):
                qv = q[b, s, h].double()
                ks = k[slots, h * hd:(h + 1) * hd].double()
                vs = v[slots, h * hd:(h + 1) * hd].double()
                sc = ks @ qv / math.sqrt(hd) + torch.tensor([float(bias[n // BS]) for n in slots], dtype=torch.float64)
                out[b, s, h] = torch.softmax(sc, 0) @ vs
    return out


def test_read_equals_gather_over_active_slots():
    g = torch.Generator().manual_seed(4)
    B, S, H, hd, NB, BS = 2, 6, 2, 8, 4, 5
    q = torch.randn(B, S, H, hd, generator=g)
    k = torch.randn(NB * BS, H * hd, generator=g)
    v = torch.randn(NB * BS, H * hd, generator=g)
    top = torch.randint(0, NB, (B, S, 2), generator=g)
    gates = torch.softmax(torch.randn(B, S, 2, generator=g), -1)
    got = oracle.mom_read(q.double(), k.double(), v.double(), top, gates.double(), num_blocks=NB, block_size=BS)
    torch.testing.assert_close(got, _gather_read_fp64(q, k, v, top, gates, NB, BS), rtol=1e-12, atol=1e-12)
    got32 = oracle.mom_read(q, k, v, top, gates, num_blocks=NB, block_size=BS)
    torch.testing.assert_close(got32.double(), _gather_read_fp64(q, k, v, top, gates, NB, BS), rtol=1e-5, atol=1e-5)


def test_read_invariants_convex_hull_and_gate_independence():
    g = torch.Generator().manual_seed(6)
    B, S, H, hd, NB, BS = 1, 16, 2, 8, 4, 8
    q = torch.randn(B, S, H, hd, generator=g, dtype=torch.float64)
    k = torch.randn(NB * BS, H * hd, generator=g, dtype=torch.float64)
    v = torch.randn(NB * BS, H * hd, generator=g, dtype=torch.float64)
    top = torch.randint(0, NB, (B, S, 2), generator=g)
    gates = torch.softmax(torch.randn(B, S, 2, generator=g, dtype=torch.float64), -1)
    o = oracle.mom_read(q, k, v, top, gates, num_blocks=NB, block_size=BS)
    for s in range(S):
        sel = sorted({int(e) for e in top[0, s]})
        rows = torch.cat([v[e * BS:(e + 1) * BS] for e in sel])
        for h in range(H):
            vv = rows[:, h * hd:(h + 1) * hd]
            assert bool((o[0, s, h] <= vv.max(0).values + 1e-12).all())
            assert bool((o[0, s, h] >= vv.min(0).values - 1e-12).all())
    one = torch.full((B, S, 2), 1, dtype=torch.long)                         # both picks name block 1
    o1 = oracle.mom_read(q, k, v, one, gates, num_blocks=NB, block_size=BS)
    o2 = oracle.mom_read(q, k, v, one, torch.softmax(torch.randn(B, S, 2, generator=g, dtype=torch.float64), -1),
                         num_blocks=NB, block_size=BS)
    torch.testing.assert_close(o1, o2, rtol=1e-12, atol=1e-12)


def test_read_backward_finite_differences_and_gate_sum():
    g = torch.Generator().manual_seed(8)
    B, S, H, hd, NB, BS = 1, 5, 2, 4, 3, 4
    q = torch.randn(B, S, H, hd, generator=g, dtype=torch.float64, requires_grad=True)
    k = torch.randn(NB * BS, H * hd, generator=g, dtype=torch.float64, requires_grad=True)
    v = torch.randn(NB * BS, H * hd, generator=g, dtype=torch.float64, requires_grad=True)
    top = torch.argsort(torch.rand(B, S, NB, generator=g), -1)[..., :2]    # distinct blocks
    gates = torch.softmax(torch.randn(B, S, 2, generator=g, dtype=torch.float64), -1).requires_grad_(True)

    def f(q, k, v, gates):
        return oracle.mom_read(q, k, v, top, gates, num_blocks=NB, block_size=BS)

    # q, k, v: fp64 finite differences
    assert torch.autograd.gradcheck(lambda q, k, v: f(q, k, v, gates.detach()), (q, k, v), eps=1e-6, atol=1e-7)
    # gates: the reference rounds log(gate) to fp32 (reference.py:23), so use
    # central differences with a step large enough to dwarf that rounding
    w = torch.randn(B, S, H, hd, generator=g, dtype=torch.float64)
    (ga,) = torch.autograd.grad((f(q, k, v, gates) * w).sum(), gates)
    with torch.no_grad():
        for idx in [(0, 0, 0), (0, 2, 1), (0, 4, 0)]:
            eps = 1e-3 * float(gates[idx])
            gp, gm = gates.clone(), gates.clone()
            gp[idx] += eps
            gm[idx] -= eps
            fd = ((f(q, k, v, gp) * w).sum() - (f(q, k, v, gm) * w).sum()) / (2 * eps)
            assert abs(float(fd) - float(ga[idx])) <= 1e-3 * max(1.0, abs(float(fd))), (idx, float(fd), float(ga[idx]))
    # softmax shift invariance: sum_t dlog_t = sum_t g_t dL/dg_t = 0 per token
    y = f(q, k, v, gates)
    (gq,) = torch.autograd.grad((y * torch.randn_like(y)).sum(), gates)
    # (the bias path is fp32 in the reference, reference.py:23-27, so the sum
    # vanishes to fp32 rounding of the per-selection terms)
    scale = float((gq * gates).detach().abs().max())
    torch.testing.assert_close((gq * gates).sum(-1), torch.zeros(B, S, dtype=torch.float64), rtol=0,
                               atol=1e-6 * max(scale, 1e-3))
    assert scale > 1e-3  # the individual terms are not trivially zero


# ------------------------------------------------------------ router
def test_router_identities_and_fp64_decider():
    torch.manual_seed(2)
    B, T, D, R, E, K = 2, 300, 64, 8, 8, 2
    x = torch.randn(B, T, D)
    wd = torch.randn(R, D) * 0.3
    wu = torch.randn(E, R) * 0.3
    logits, probs, idx, gates, h = oracle.router(x, wd, wu, K)
    torch.testing.assert_close(probs.sum(-1), torch.ones(B, T))
    torch.testing.assert_close(gates.sum(-1), torch.ones(B, T))
    assert bool((gates[..., 0] >= gates[..., 1]).all())                      # topk sorted descending
    assert torch.equal(logits.gather(-1, idx).argsort(-1, descending=True)[..., 0], torch.zeros(B, T, dtype=torch.long))
    l64 = F.linear(torch.tanh(F.linear(oracle.prefix_mean(x).double(), wd.double())), wu.double())
    srt = l64.sort(-1, descending=True)
    clear = (srt.values[..., K - 1] - srt.values[..., K]) > 1e-5 * float(l64.abs().max())
    assert torch.equal(idx[clear].sort(-1).values, srt.indices[..., :K][clear].sort(-1).values)
    torch.testing.assert_close(logits.double(), l64, rtol=1e-5, atol=1e-6)


def test_router_noise_only_reranks():
    torch.manual_seed(3)
    x = torch.randn(1, 50, 16)
    wd, wu = torch.randn(4, 16), torch.randn(6, 4)
    noise = torch.zeros(1, 50, 6)
    noise[..., 5] = 100.0
    l0, p0, i0, g0, _ = oracle.router(x, wd, wu, 2)
    l1, p1, i1, g1, _ = oracle.router(x, wd, wu, 2, noise=noise, noise_scale=1.0)
    assert torch.equal(l0, l1) and torch.equal(p0, p1)                      # probs stay clean
    assert bool((i1[..., 0] == 5).all())                                     # noise decides top-1


# ------------------------------------------------------------ bank K/V and aux
def test_bank_kv_fp64():
    torch.manual_seed(4)
    M = torch.randn(4, 3 * 16)
    wk, wv = torch.randn(8, 16), torch.randn(8, 16)
    k, v = oracle.bank_kv(M, wk, wv)
    slots = M.view(12, 16).double()
    torch.testing.assert_close(k.double(), slots @ wk.double().T, rtol=1e-6, atol=1e-5)
    torch.testing.assert_close(v.double(), slots @ wv.double().T, rtol=1e-6, atol=1e-5)


def test_aux_loss_closed_form_and_scatter():
    E, K, N = 8, 2, 64
    # exactly uniform routing: every block selected by a fraction K/E of tokens,
    # uniform probs -> E * sum_e (K/E)(1/E) = K   (METHODOLOGY.md:90: 2.0 at top-2)
    idx = torch.stack([torch.arange(N) % E, (torch.arange(N) + 1) % E], -1)
    probs = torch.full((N, E), 1.0 / E)
    assert abs(float(oracle.aux_loss(probs, idx, E)) - K) < 1e-6
    torch.manual_seed(42)                                                    # test_parity.py §14
    probs = torch.softmax(torch.randn(128, E), -1)
    idx = torch.randint(0, E, (128, K))
    sel = torch.zeros_like(probs).scatter_(1, idx, 1.0)
    torch.testing.assert_close(oracle.aux_loss(probs, idx, E), E * (sel.mean(0) * probs.mean(0)).sum(),
                               rtol=0, atol=1e-6)


def router_stats_closed_forms():
    """(probs, top_idx, E, entropy, dead fraction) cases whose statistics are
    fixed by the mathematics, not by the formula under test: uniform probs
    have entropy log E, one-hot probs 0 (0 * log(1e-9) = 0), a two-point
    distribution (a, 1-a, 0, ...) the binary entropy; a block no token
    selects is dead."""
    E = 8
    cases = []
    N = 40
    idx = torch.stack([torch.arange(N) % E, (torch.arange(N) + 3) % E], -1)
    cases.append((torch.full((N, E), 1.0 / E), idx, E, math.log(E), 0.0))
    onehot = torch.zeros(N, E)
    onehot[torch.arange(N), torch.arange(N) % 5] = 1.0
    idx1 = torch.stack([torch.arange(N) % 5, (torch.arange(N) % 5 + 1) % 5], -1)  # blocks 5..7 never selected
    cases.append((onehot, idx1, E, 0.0, 3.0 / E))
    a = 0.25  # exact in fp32
    two = torch.zeros(N, E)
    two[:, 0], two[:, 1] = a, 1.0 - a
    cases.append((two, torch.tensor([[0, 1]]).expand(N, 2), E, -(a * math.log(a) + (1 - a) * math.log(1 - a)),
                  6.0 / E))
    return cases


def test_router_stats_closed_forms():
    for probs, idx, E, ent_want, dead_want in router_stats_closed_forms():
        ent, dead = oracle.router_stats(probs.double(), idx, E)
        assert abs(float(ent) - ent_want) <= 1e-6 * max(1.0, ent_want)  # fp32 arithmetic, as model.py:505
        assert float(dead) == dead_want


def test_active_tile_blocks_brute_force():
    g = torch.Generator().manual_seed(9)
    top = torch.randint(0, 6, (3, 300, 2), generator=g)
    want = 0
    for b in range(3):
        for t0 in range(0, 300, 128):
            want += len({int(e) for e in top[b, t0:t0 + 128].flatten()})
    assert oracle.active_tile_blocks(top, 6, 128) == want


def test_decode_step_equals_full_sequence_rows():
    """Stepping the running prefix-sum state token by token gives, at every
    position, the router decision and read output of the full-sequence
    oracle (model.py:172-173 vs the O(1) decode form)."""
    g = torch.Generator().manual_seed(13)
    B, S, H, HD, NB, BS, K, R = 2, 24, 2, 16, 4, 16, 2, 8
    D = H * HD
    x = torch.randn(B, S, D, generator=g)
    wd, wu = torch.randn(R, D, generator=g) * 0.3, torch.randn(NB, R, generator=g)
    q = torch.randn(B, S, H, HD, generator=g)
    k, v = torch.randn(NB * BS, D, generator=g), torch.randn(NB * BS, D, generator=g)
    _, _, idx_full, gates_full, _ = oracle.router(x, wd, wu, K)
    out_full = oracle.mom_read(q, k, v, idx_full, gates_full, num_blocks=NB, block_size=BS)
    state = torch.zeros(B, D, dtype=torch.float64)
    for t in range(S):
        tp = torch.full((B,), t, dtype=torch.int64)
        out, state, idx, gates = oracle.decode_step(state, tp, x[:, t], wd, wu, K, q[:, t], k, v, NB, BS)
        assert torch.equal(idx, idx_full[:, t])
        torch.testing.assert_close(gates, gates_full[:, t], rtol=0, atol=0)
        torch.testing.assert_close(out, out_full[:, t].float(), rtol=1e-5, atol=1e-6)


def test_router_forced_selection_equals_free_selection():
    """router(force_idx=its own top-k) reproduces every output bitwise, and a
    forced different selection changes only top_idx / gates."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(2, 40, 32, generator=g)
    wd = torch.randn(8, 32, generator=g) * 0.2
    wu = torch.randn(6, 8, generator=g) * 0.5
    free = oracle.router(x, wd, wu, 2)
    forced = oracle.router(x, wd, wu, 2, force_idx=free[2])
    for a, b in zip(free, forced):
        assert torch.equal(a, b)
    other = torch.stack([free[2][..., 1], free[2][..., 0]], -1)     # same pair, swapped
    sw = oracle.router(x, wd, wu, 2, force_idx=other)
    assert torch.equal(sw[3], free[3].flip(-1)) and torch.equal(sw[1], free[1])
