#!/usr/bin/env python3
"""MoM layer forward+backward throughput on one MI355X.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--workload config2|config3|config4|config5]

Workload ("config2"): one Naylis MoM layer in bf16,
forward + backward at the training shape B=8, T=2048, d=1024, 16 heads x 64,
bank 8 blocks x 128 slots x 1024 rescaled to Frobenius norm 63, router
d -> 32 -> 8 with top-2, ReZero scale 1.0, Gumbel noise off.  x is RMS-normed
N(0,1) in bf16, dy ~ N(0,1) in fp32 (the dtype of y); router weights, prefix mean and routing in fp32.
Random-init weights, synthetic data.  A step is y = layer(x, M); y.backward(dy)
with all parameter gradients.

Prints ONE JSON line: tokens/s (value) and per-step time over K uninstrumented
steps; then, over K further steps with every library launch bracketed by HIP
events on its launch stream, each kernel's average duration and the roofline
of the read (its forward and backward kernels summed, priced on the
tile-active basis against the bf16 MFMA peak); and a CPU baseline (the eager
fp32 oracle on the host).

config5 is the inference decode step instead: B=64
sequences, one new token each, running prefix-sum state of prior length
1..4096, d=1024, 16 x 64 heads, router rank 32, bank 8 x 128 quantised to fp8
e4m3 with per-slot scales, top-2.  A step is one naylis_mom_decode_step for
the 64 sequences (state ping-pong between two buffers); the K timed steps are
one captured HIP graph of K steps, replayed once, so host launch cost stays
out of the figure.  value = decoded tokens/s (B per step).

config3 is the full decoder: 20 Llama layers (d=1024,
16 heads, SwiGLU 2816, RoPE, vocab 32768, tied head), each with a MoM read of
the one shared 8 x 128 bank, bf16 with fp32 routing, random init, B=8, T=2048,
token ids uniform; a step is next-token CE + 0.01 aux loss, forward and
backward.  value = tokens/s; "model" gives the step's model FLOP rate and
"read" the MoM reads' MFMA fraction summed over the layers.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "MoM layer fwd+bwd tokens/s at d=1024, 8x128 slots; % bf16 MFMA peak"

WORKLOADS = {
    # B, T, d, heads, blocks, block_size, top_k, rank
    # config1 (the reference's CPU case): x ~ N(0, 1), bank N(0, 0.02) as drawn
    "config1": dict(B=2, T=512, D=1024, H=16, E=8, BS=128, K=2, R=32, bank_fro=None, tile_bias=None,
                    x_rmsnorm=False),
    "config2": dict(B=8, T=2048, D=1024, H=16, E=8, BS=128, K=2, R=32, bank_fro=63.0, tile_bias=None),
    "config4": dict(B=4, T=4096, D=1536, H=24, E=32, BS=128, K=2, R=32, bank_fro=None, tile_bias=(3, 6)),
    "config5": dict(B=64, D=1024, H=16, E=8, BS=128, K=2, R=32, bank_fro=63.0, max_prior=4096),
    "config3": dict(B=8, T=2048, D=1024, H=16, E=8, BS=128, K=2, R=32, layers=20, ffn=2816, vocab=32768),
}
DECODE_METRIC = "MoM decode step tokens/s at B=64, d=1024, fp8 8x128 bank"
DECODER_METRIC = "Naylis decoder (20 layers, d=1024, shared 8x128 bank) fwd+bwd tokens/s"


def build(cfg, device):
    import torch

    from naylis_amd.layer import MoMLayer
    B, T, D, H, E, BS, K, R = (cfg[k] for k in ("B", "T", "D", "H", "E", "BS", "K", "R"))
    gw = torch.Generator().manual_seed(0)
    layer = MoMLayer(d_model=D, n_heads=H, mem_size=E * BS, block_size=BS, top_blocks=K, router_rank=R)
    with torch.no_grad():
        for lin in (layer.router_down, layer.router_up, layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=gw) * 0.02)
        layer.mom_scale.fill_(1.0)
    layer = layer.to(device)
    for lin in (layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
        lin.to(torch.bfloat16)
    layer.train()
    layer.noise_scale = 0.0
    gb = torch.Generator().manual_seed(3)
    M = torch.randn(E, BS * D, generator=gb) * 0.02
    if cfg["bank_fro"]:
        M = M * (cfg["bank_fro"] / float(M.norm()))
    M = M.bfloat16().to(device).requires_grad_(True)
    gx = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, D, generator=gx)
    if cfg.get("x_rmsnorm", True):
        x = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)
    x = x.bfloat16().to(device).requires_grad_(True)
    gd = torch.Generator().manual_seed(2)
    dy = torch.randn(B, T, D, generator=gd).to(device)  # fp32: the dtype of y (ReZero promotes to fp32)
    if cfg["tile_bias"]:
        lo, hi = cfg["tile_bias"]
        bias = torch.zeros(B, T, E)
        for b in range(B):
            for t0 in range(0, T, 128):
                n = int(torch.randint(lo, hi + 1, (1,), generator=gb))
                bias[b, t0:t0 + 128, torch.randperm(E, generator=gb)[:n]] = 1.0
        # the additive logit hook of the router: +10 x logit std on the favoured blocks
        layer._bench_bias = (bias * 10.0 * 0.02).to(device)
    return layer, M, x, dy


def layer_step(layer, M, x, dy):
    bias = getattr(layer, "_bench_bias", None)
    if bias is None:
        y = layer(x, M)
    else:
        y = _forward_with_bias(layer, x, M, bias)
    y.backward(dy)
    # the gradient reset (the step's end): the parameter list is taken once
    params = layer.__dict__.get("_bench_params")
    if params is None:
        params = layer.__dict__["_bench_params"] = list(layer.parameters())
    for p in params:
        p.grad = None
    M.grad = None
    x.grad = None


def _forward_with_bias(layer, x, M, bias):
    """Layer forward with an additive router-logit bias (config 4's sparsity),
    through the layer's fused node when it applies."""
    from naylis_amd import mom_kernels
    from naylis_amd.mom_kernels.hip_layer import fused_layer_supported, mom_layer
    if layer._kernel_mode is None:
        layer._kernel_mode = layer._resolve_kernel(x)
    ws = (layer.router_down.weight, layer.router_up.weight, layer.q_proj.weight, layer.k_proj.weight,
          layer.v_proj.weight, layer.o_proj.weight, layer.mom_scale)
    if fused_layer_supported(x, M, *ws):
        y, _, _ = mom_layer(x, M, *ws, n_heads=layer.n_heads, num_blocks=layer.num_blocks,
                            block_size=layer.block_size, top_k=layer.top_blocks, noise=bias, noise_scale=1.0)
        return y
    _, probs, idx, gates = mom_kernels.mom_route(x, layer.router_down.weight, layer.router_up.weight,
                                                 layer.top_blocks, noise=bias, noise_scale=1.0)
    return mom_kernels.mom_rezero(layer._read(x, idx, gates, M), layer.mom_scale)


def torch_projection_gemms(layer, x, steps):
    """The layer's q / o projection GEMMs that run on torch (hipBLASLt): the
    q projection forward (model.py:251), the o projection forward with the
    ReZero gate folded into the weight and an fp32 result (model.py:276) and
    the two input gradients, each called as the layer calls it, on the layer's
    own shapes and weights, timed standalone with events on the current
    stream (the library's KernelTimer does not see torch's launches).  2 N d^2
    FLOP each."""
    import torch
    import torch.nn.functional as F
    B, T, D = x.shape
    N = B * T
    x2 = x.detach().reshape(N, D).to(torch.bfloat16).contiguous()
    w_q = layer.q_proj.weight.detach()
    w_os = (layer.o_proj.weight.detach().float() * float(layer.mom_scale.detach())).to(w_q.dtype)
    g = torch.Generator(device=x.device).manual_seed(1)
    a2 = torch.randn((N, D), generator=g, device=x.device).to(torch.bfloat16)
    calls = {"q_proj_fwd": lambda: F.linear(x2, w_q),
             "o_proj_fwd": lambda: torch.mm(a2, w_os.t(), out_dtype=torch.float32),
             "o_proj_dgrad": lambda: torch.mm(a2, w_os),
             "q_proj_dgrad": lambda: torch.mm(a2, w_q)}
    out = {}
    flop = 2.0 * N * D * D
    for name, fn in calls.items():
        for _ in range(3):
            fn()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / steps
        tf = flop / (us * 1e-6) / 1e12
        out["hipblaslt_" + name] = {"us": round(us, 2), "tflops": round(tf, 1),
                                    "mfma_frac": round(tf / PEAK_BF16_TFLOPS, 4),
                                    "timing": "standalone, back to back, events on the current stream"}
    return out


def routing(layer, M, x):
    import torch

    from naylis_amd import mom_kernels
    with torch.no_grad():
        bias = getattr(layer, "_bench_bias", None)
        _, _, idx, _ = mom_kernels.mom_route(x, layer.router_down.weight, layer.router_up.weight,
                                             layer.top_blocks, noise=bias, noise_scale=1.0)
    return idx


def active_tiles(idx, E, tile=128):
    import torch
    B, T, K = idx.shape
    n_tiles = (T + tile - 1) // tile
    oh = torch.zeros(B, n_tiles * tile, E, dtype=torch.bool, device=idx.device)
    oh[:, :T].scatter_(2, idx.long(), True)
    return int(oh.view(B, n_tiles, tile, E).any(2).sum())


def executed_tiles(idx, E, tile=128):
    """(tile, block) pairs over the flattened tokens in the order the read
    kernels walk them (the library's token order for this routing)."""
    import torch
    from naylis_amd.mom_kernels.hip_read import read_order
    B, T, K = idx.shape
    N = B * T
    order = read_order(idx.to(torch.int32).contiguous(), E)
    flat = idx.reshape(N, K).long()
    if int(order[0]) == 1:
        flat = flat[order[1:1 + N].long()]
    n_tiles = (N + tile - 1) // tile
    oh = torch.zeros(n_tiles * tile, E, dtype=torch.bool, device=idx.device)
    oh[:N].scatter_(1, flat, True)
    return int(oh.view(n_tiles, tile, E).any(1).sum()), ("grouped" if int(order[0]) == 1 else "sequence")


# Every launch of the read path (the north star's kernels): the token order (local histogram
# and scatter launches), the two-pass path's tile lists, the forward, the backward kernels and
# the backward's reduction.  Each is bracketed by its own HIP events (KernelTimer).
READ_LAUNCHES = ("read_order", "read_tile_lists", "read_fwd", "read_bwd_pair", "read_bwd_dq", "read_bwd_dkdv",
                 "read_bwd_reduce")


def pair_executed_tiles(idx, E):
    """(128-token tile, block) units the pair-tiled kernels execute: every
    token of a 32-token tile of pair (a, b) runs against both blocks (one
    for a == b), the pair's runs padded to whole tiles."""
    import torch
    K = idx.shape[-1]
    flat = idx.reshape(-1, K).long().clamp(0, E - 1)
    lo, hi = flat.min(1).values, flat.max(1).values
    key = lo * E + hi
    counts = torch.bincount(key, minlength=E * E)
    tiles = (counts + 31) // 32
    nblk = torch.where(torch.arange(E * E, device=idx.device) % (E + 1) == 0, 1, 2)
    return float((tiles * 32 * nblk).sum()) / 128.0


def cpu_model():
    """The host CPU's model name as `lscpu` reports it (its "Model name"
    line), else /proc/cpuinfo's "model name"."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, sample_b):
    """Eager fp32 oracle layer on every core of the process's affinity set,
    as planned for the CPU baseline: config 2 fwd+bwd on `sample_b` of the B
    sequences at the full T (all of them by default), the bank rescaled to
    the workload's Frobenius norm, and config 1 forward (B=2, T=512), each 2
    warmup runs then the median of 5."""
    import torch

    import oracle
    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def make(B, T, D, H, E, BS, K, R, bank_fro=None):
        torch.manual_seed(0)
        layer = oracle.OracleMoMLayer(D, H, E * BS, BS, K, R)
        with torch.no_grad():
            for lin in (layer.router_down, layer.router_up, layer.q_proj, layer.k_proj, layer.v_proj, layer.o_proj):
                lin.weight.normal_(0, 0.02)
            layer.mom_scale.fill_(1.0)
        layer.noise_scale = 0.0
        M = torch.randn(E, BS * D) * 0.02
        if bank_fro:
            M = M * (bank_fro / float(M.norm()))
        M.requires_grad_(True)
        x = torch.randn(B, T, D)
        x = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)).requires_grad_(True)
        return layer, M, x, torch.randn(B, T, D)

    def median_time(fn):
        times = []
        for _ in range(2 + 5):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return statistics.median(times[2:])

    B, T, D, H, E, BS, K, R = (cfg[k] for k in ("B", "T", "D", "H", "E", "BS", "K", "R"))
    b = min(sample_b, B)
    layer, M, x, dy = make(b, T, D, H, E, BS, K, R, cfg.get("bank_fro"))

    def fwd_bwd():
        y = layer(x, M)
        y.backward(dy)
        layer.zero_grad(set_to_none=True)
        M.grad = None
        x.grad = None

    med = median_time(fwd_bwd)
    del layer, M, x, dy
    c1 = WORKLOADS["config1"]
    l1, M1, x1, _ = make(*(c1[k] for k in ("B", "T", "D", "H", "E", "BS", "K", "R")))
    with torch.no_grad():
        med1 = median_time(lambda: l1(x1, M1))
    return {"value": round(b * T / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle.OracleMoMLayer fp32 fwd+bwd, {b} of {B} sequences x T={T}, bank "
                      f"Frobenius {cfg.get('bank_fro') or 'as drawn'} (2 warmup, median of 5 runs: {med:.3f} s), "
                      f"torch {torch.__version__}, {threads} threads (the affinity set)",
            "cpu_model": cpu_model(),
            "config1_forward": {"value": round(c1["B"] * c1["T"] / med1, 1), "unit": "tokens/s",
                                "ms": round(med1 * 1e3, 2),
                                "sample": f"oracle.OracleMoMLayer fp32 forward, B={c1['B']} T={c1['T']} "
                                          f"d={c1['D']} (2 warmup, median of 5)"}}


def build_decode(cfg, device):
    """Config-5 inputs: bank K / V from a random bank (Frobenius 63) and random
    N(0, 1/d) projections, quantised once to fp8; states of random prior
    lengths; new tokens and queries N(0, 1) in bf16."""
    import math

    import torch

    from naylis_amd.mom_kernels.hip_decode import quantize_bank_fp8
    B, D, H, E, BS, R = (cfg[k] for k in ("B", "D", "H", "E", "BS", "R"))
    g = torch.Generator().manual_seed(0)
    M = torch.randn(E * BS, D, generator=g)
    M = M * (cfg["bank_fro"] / float(M.norm()))
    wk = torch.randn(D, D, generator=g) / math.sqrt(D)
    wv = torch.randn(D, D, generator=g) / math.sqrt(D)
    k = (M @ wk.t()).bfloat16().to(device)
    v = (M @ wv.t()).bfloat16().to(device)
    bank = quantize_bank_fp8(k, v)
    t_prev = torch.randint(1, cfg["max_prior"] + 1, (B,), generator=g)
    state = torch.randn(B, D, generator=g, dtype=torch.float64) * t_prev.double().sqrt()[:, None]
    x = torch.randn(B, D, generator=g).bfloat16()
    q = torch.randn(B, H, D // H, generator=g).bfloat16()
    w_down = torch.randn(R, D, generator=g) * 0.02
    w_up = torch.randn(E, R, generator=g) * 0.02
    to = lambda t: t.to(device)
    return bank, (k, v), to(state), to(t_prev.int()), to(x), to(q), to(w_down), to(w_up)


def decode_alg_bytes(cfg, idx):
    """Unique bytes one decode launch must move: state in + out (fp64), token,
    query and output (bf16), router weights (fp32), and the K / V rows (fp8)
    and scales of every block some sequence selected (all heads)."""
    B, D, E, BS, R = (cfg[k] for k in ("B", "D", "E", "BS", "R"))
    blocks = len(set(int(i) for i in idx.flatten().tolist()))
    return (B * D * 8 * 2 + B * D * 2 * 3 + (R * D + E * R) * 4
            + blocks * BS * (2 * D + 2 * 4) + B * cfg["K"] * 8)


def decode_cpu_baseline(cfg, bank_bf16, state, t_prev, x, q, w_down, w_up, reps=20):
    """oracle.decode_step (fp32 router, dense read over the bf16 bank) on the
    host cores for the whole B=64 batch, median of `reps` steps."""
    import torch

    import oracle
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    k, v = (t.float().cpu() for t in bank_bf16)
    args = (state.cpu(), t_prev.cpu(), x.cpu(), w_down.cpu(), w_up.cpu(), cfg["K"], q.cpu(), k, v, cfg["E"],
            cfg["BS"])
    oracle.decode_step(*args)
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle.decode_step(*args)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(cfg["B"] / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle.decode_step fp32 over the bf16 bank, the full B={cfg['B']} batch, "
                      f"median of {reps} steps ({med * 1e3:.3f} ms/step), torch {torch.__version__}"}


def decode_bench(args, cfg, dev):
    import torch

    from naylis_amd import _lib
    from naylis_amd.mom_kernels.hip_decode import decode_step
    B, D, H, E, BS, K = (cfg[k] for k in ("B", "D", "H", "E", "BS", "K"))
    bank, kv_bf16, state, t_prev, x, q, w_down, w_up = build_decode(cfg, dev)
    st = [state.clone(), torch.empty_like(state)]

    def run(n, j0=0):
        for j in range(j0, j0 + n):
            o, _, idx, _ = decode_step(st[j % 2], t_prev, x, w_down, w_up, K, q, bank, E, BS,
                                       out_state=st[(j + 1) % 2])
        return idx

    idx = run(max(args.warmup, 1))
    torch.cuda.synchronize()
    # (1) K steps captured in one graph (an even count keeps the ping-pong aligned), replayed once
    n = args.steps + (args.steps & 1)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        run(2)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            run(n)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    # HIP events on the stream the graph (and so every decode launch) runs on
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / n
    # the step is one decode_step launch, so the events' average per launch is the kernel's duration
    # (back to back, inter-launch gaps included)
    dom_ms = e0.elapsed_time(e1) / n
    # (2) per-launch durations of eager launches, each bracketed by HIP events (adds the events' cost)
    with _lib.KernelTimer():
        run(args.steps)
        torch.cuda.synchronize()
    kernels = _lib.KernelTimer.results()
    per = {k: (v[0] / v[1], v[1]) for k, v in kernels.items() if v[1]}
    alg = decode_alg_bytes(cfg, idx)
    ach = alg / (dom_ms * 1e-3) / 1e9
    roof = {"kernel": "decode_step", "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None, "avg_us": round(dom_ms * 1e3, 2),
            "alg_bytes_per_launch": alg}
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            roof["traffic"] = json.load(f).get("config5:decode_step")
    line = {
        "metric": DECODE_METRIC,
        "value": round(B / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": n,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8-e4m3 bank, bf16 q, fp32 router, fp64 state",
        "data": "synthetic (random bank / weights, random prior lengths 1..4096)",
        "config": {"workload": f"config5: MoM decode step B={B} d={D} heads={H}x{D // H} bank {E}x{BS} fp8 "
                               f"top-{K} rank {cfg['R']}",
                   "global_batch": B, "seq_len": 1, "parallelism": "single-gpu"},
        "roofline": roof,
        "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in sorted(per.items())},
        "kernels_timing": f"roofline avg_us: HIP events around the graph of {n} launches; kernels_us: events "
                          f"around each of {args.steps} eager launches",
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = decode_cpu_baseline(cfg, kv_bf16, state, t_prev, x, q, w_down, w_up)
    print(json.dumps(line), flush=True)
    return 0


def decoder_flops(cfg, params_dense):
    """Model FLOP of one fwd+bwd step for the per-token weights and the trunk's
    attention: 6 per weight per token (trunk, MoM q/o projections and router,
    LM head) plus causal attention (QK^T and PV over half the square, x3 for
    fwd+bwd)."""
    B, T, D, L = cfg["B"], cfg["T"], cfg["D"], cfg["layers"]
    return 6.0 * B * T * params_dense + 3.0 * L * 2 * 2 * B * T * T * D / 2


def decoder_cpu_baseline(cfg, state):
    """The fp32 CPU oracle decoder (all layers, full width, eager MoM read) fwd+bwd
    on one sequence of 256 tokens, 1 warmup + median of 2."""
    import torch

    import oracle
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    ref = oracle.OracleDecoder(cfg["vocab"], cfg["D"], cfg["layers"], cfg["H"], cfg["ffn"], cfg["E"] * cfg["BS"],
                               cfg["BS"], cfg["K"], cfg["R"])
    ref.load_state_dict(state, strict=True)
    ref.train()
    T = 256
    ids = torch.randint(0, cfg["vocab"], (1, T), generator=torch.Generator().manual_seed(4))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        loss, _, _ = ref(ids, labels=ids)
        loss.backward()
        times.append(time.perf_counter() - t0)
        ref.zero_grad(set_to_none=True)
    med = statistics.median(times[1:])
    return {"value": round(T / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle.OracleDecoder fp32 fwd+bwd (CE + aux), 1 sequence x T={T} of the config-3 model "
                      f"(1 warmup, median of 2 runs: {med:.3f} s), torch {torch.__version__}"}


def decoder_bench(args, cfg, dev):
    """Config 3: the full decoder, bf16 (router weights and ReZero scales fp32),
    random init, token ids uniform over the vocabulary, next-token CE + 0.01 aux.
    A step is loss = model(ids, labels=ids).loss; loss.backward(); grads dropped."""
    import torch

    from naylis_amd import _lib
    from naylis_amd.decoder import NaylisLlamaForCausalLM, cast_for_training, naylis_config
    from naylis_amd.layer import MoMLayer
    B, T, D, H, E, BS = (cfg[k] for k in ("B", "T", "D", "H", "E", "BS"))
    torch.manual_seed(0)
    mcfg = naylis_config(vocab_size=cfg["vocab"], d_model=D, n_layers=cfg["layers"], n_heads=H,
                         intermediate_size=cfg["ffn"], seq_len=T, mem_size=E * BS, mom_block_size=BS,
                         mom_top_blocks=cfg["K"], mom_router_rank=cfg["R"])
    model = NaylisLlamaForCausalLM(mcfg)
    state_fp32 = None if args.no_cpu_baseline else {k: v.detach().clone() for k, v in model.state_dict().items()}
    model = cast_for_training(model).to(dev).train()
    # router noise on, as the reference trains until its noise cutoff (pretrain.py:515-535): each MoM
    # layer draws its (B, T, E) uniform and the router kernel applies the Gumbel transform
    model.set_noise_scale(1.0)
    ids = torch.randint(0, cfg["vocab"], (B, T), generator=torch.Generator().manual_seed(1)).to(dev)

    def step():
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
        model.zero_grad(set_to_none=True)
        return out.loss

    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / args.steps
    with _lib.KernelTimer():
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    kernels = _lib.KernelTimer.results()
    per = {k: (v[0] / v[1], v[1] / args.steps) for k, v in kernels.items() if v[1]}

    # routing of every MoM layer for one forward (without labels the layers keep it)
    with torch.no_grad():
        model(input_ids=ids)
    A_total, A_exec = 0, 0.0
    for m in (x for x in model.modules() if isinstance(x, MoMLayer)):
        # the routing this forward drew (with its Gumbel noise): the timed steps draw their own,
        # of the same distribution
        idx_l = m.last_top_idx.view(B, T, -1)
        A_total += active_tiles(idx_l, E)
        A_exec += pair_executed_tiles(idx_l, E) if "read_bwd_pair" in kernels else float(executed_tiles(idx_l, E)[0])
    read_ms = sum(kernels[k][0] for k in READ_LAUNCHES if k in kernels) / args.steps
    read_flop = 14.0 * D * BS * 128 * A_total
    read_tf = read_flop / (read_ms * 1e-3) / 1e12
    # the read's launches over all layers, priced on the work the kernels execute (the pair tiles:
    # Gumbel-noised routing selects every block in nearly every 128-token tile, so the reference's
    # active-pair basis A would credit work the grouped order never runs); that basis is reported
    # beside it as an effective rate.  Both take one forward's routing: the timed steps draw their
    # own, of the same distribution.
    exec_flop = 14.0 * D * BS * 128 * A_exec
    exec_tf = exec_flop / (read_ms * 1e-3) / 1e12
    roof = {"kernel": "read (all layers): " + " + ".join(k for k in READ_LAUNCHES if k in kernels),
            "bound": "mfma", "achieved": round(exec_tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(exec_tf / PEAK_BF16_TFLOPS, 4), "traffic": None, "avg_us": round(read_ms * 1e3, 2),
            "alg_flop_per_launch": exec_flop,
            "basis": "executed tile-block units over %d layers: %.1f (pair tiles of one forward's Gumbel-noised "
                     "routing)" % (cfg["layers"], A_exec),
            "effective_tflops_reference_basis": round(read_tf, 2),
            "effective_frac_reference_basis": round(read_tf / PEAK_BF16_TFLOPS, 4),
            "note": "the reference basis counts A = %d active (128-token tile, block) pairs over %d layers in "
                    "sequence order, which the grouped order does not execute: an effective rate, not a "
                    "utilisation; trunk GEMMs and attention are torch's" % (A_total, cfg["layers"])}
    # per-token weights: every matrix but the bank and its K/V projections (the tied
    # embedding counts once, as the LM head); the bank projections run over the L slots
    params_dense = sum(p.numel() for n, p in model.named_parameters()
                       if p.dim() == 2 and n != "model.M_blocks" and ".mom.k_proj" not in n
                       and ".mom.v_proj" not in n)
    bank_flop = cfg["layers"] * 2 * 6.0 * E * BS * D * D
    model_flop = decoder_flops(cfg, params_dense) + bank_flop + read_flop
    model_tf = model_flop / (ms_per_step * 1e-3) / 1e12
    line = {
        "metric": DECODER_METRIC,
        "value": round(B * T / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, token ids uniform over the vocabulary)",
        "config": {"workload": f"config3: Naylis decoder fwd+bwd, {cfg['layers']} layers d={D} heads={H}x{D // H} "
                               f"SwiGLU {cfg['ffn']} vocab {cfg['vocab']}, shared bank {E}x{BS} top-{cfg['K']} "
                               f"rank {cfg['R']}, CE + 0.01 aux, router Gumbel noise scale 1.0",
                   "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        "roofline": roof,
        "model": {"flop_per_step": model_flop, "tflops": round(model_tf, 1),
                  "mfma_frac": round(model_tf / PEAK_BF16_TFLOPS, 4), "loss": round(float(loss.detach()), 4)},
        "read": {"active_tile_blocks_all_layers": A_total, "executed_tile_blocks_all_layers": round(A_exec, 1),
                 "alg_flop": read_flop, "ms": round(read_ms, 4), "effective_tflops": round(read_tf, 2),
                 "executed_tflops": round(exec_tf, 2)},
        "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in sorted(per.items())},
        "kernels_per_step": {k: round(v[1], 2) for k, v in sorted(per.items())},
    }
    if state_fp32 is not None:
        del model
        torch.cuda.empty_cache()
        line["cpu_baseline"] = decoder_cpu_baseline(cfg, state_fp32)
    print(json.dumps(line), flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="config2", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=8)
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the timed region, run 3 plain device copies of this many MiB (a known-size "
                         "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; multi-GPU runs are not part of it "
              "(the sharding design is in DESIGN.md).", file=sys.stderr)
        return 2

    import torch

    from naylis_amd import _lib
    dev = torch.device("cuda:0")
    cfg = WORKLOADS[args.workload]
    if args.workload == "config5":
        return decode_bench(args, cfg, dev)
    if args.workload == "config3":
        return decoder_bench(args, cfg, dev)
    layer, M, x, dy = build(cfg, dev)
    B, T, D, H, E, BS = (cfg[k] for k in ("B", "T", "D", "H", "E", "BS"))
    ntok = B * T

    for _ in range(args.warmup):
        layer_step(layer, M, x, dy)
    torch.cuda.synchronize()
    # (1) throughput: K steps with no instrumentation
    t0 = time.perf_counter()
    for _ in range(args.steps):
        layer_step(layer, M, x, dy)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / args.steps
    # (2) per-kernel durations: K more steps with every library launch bracketed
    # by HIP events on its stream (the events add host and GPU time, so this
    # region is timed separately from the throughput above)
    with _lib.KernelTimer():
        t2 = time.perf_counter()
        for _ in range(args.steps):
            layer_step(layer, M, x, dy)
        torch.cuda.synchronize()
        t3 = time.perf_counter()
    kernels = _lib.KernelTimer.results()
    ms_per_step_events = (t3 - t2) * 1e3 / args.steps

    # algorithmic work on the tile-active basis (128-token tiles, the
    # reference's BLOCK_M): per (b, tile, active block) d*bs*128 MACs per GEMM
    idx = routing(layer, M, x)
    A = active_tiles(idx, E)
    A_exec, order_mode = executed_tiles(idx, E)
    unit = 2.0 * D * BS * 128 * A          # FLOP of one GEMM-shaped product
    L = E * BS
    alg = {"read_fwd": 2 * unit, "read_bwd_dq": 3 * unit, "read_bwd_dkdv": 4 * unit,
           # GEMMs: 2 flop per multiply-add; bank K/V (two products), d_slots, dW_k/dW_v; q/o weight grads
           "bank_kv_fwd": 2 * 2.0 * L * D * D, "bank_kv_bwd_dslots": 2.0 * L * 2 * D * D,
           "bank_kv_bwd_dw": 2 * 2.0 * D * D * L, "linear_wgrad": 2.0 * ntok * D * D}
    per = {k: (v[0] / v[1], v[1] / args.steps) for k, v in kernels.items() if v[1]}  # avg ms, launches/step

    # the roofline is the read itself (the north-star path): all of its launches per step (the
    # token order, the forward, the backward and its reduction), priced on the reference's work,
    # the 14-unit basis (forward 2 products, backward 5, 2 flop per multiply-add) over its active
    # (128-token tile, block) pairs A, and beside it on the basis of the tile-blocks the path
    # executed
    read_launched = [k for k in READ_LAUNCHES if k in kernels]
    read_ms = sum(kernels[k][0] for k in read_launched) / args.steps
    read_flop = 14.0 * D * BS * 128 * A
    read_tf = read_flop / (read_ms * 1e-3) / 1e12
    if "read_bwd_pair" in kernels:
        A_run, run_basis = pair_executed_tiles(idx, E), "pair tiles: 32 tokens x both blocks of their pair"
    else:
        A_run, run_basis = float(A_exec), f"{order_mode}-order 128-token tiles"
    exec_tf = 14.0 * D * BS * 128 * A_run / (read_ms * 1e-3) / 1e12
    roof = {"kernel": "read: " + " + ".join(read_launched), "bound": "mfma",
            "achieved": round(read_tf, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(read_tf / PEAK_BF16_TFLOPS, 4), "traffic": None, "avg_us": round(read_ms * 1e3, 2),
            "alg_flop_per_launch": read_flop, "basis": f"active (128-token tile, block) pairs A = {A}",
            "frac_exec": round(exec_tf / PEAK_BF16_TFLOPS, 4),
            "exec_basis": f"{run_basis}: {A_run:.1f} tile-block units"}
    traffic_file = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            tr = json.load(f)
        parts = [tr.get(f"{args.workload}:{k}") for k in read_launched]
        if parts and all(t is not None for t in parts):
            roof["traffic"] = int(sum(parts))
            roof["traffic_source"] = "profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE per launch, " \
                                     "scaled by a copy kernel's readings)"
    counters_file = os.path.join(ROOT, "profiles", "read_counters.json")
    if os.path.exists(counters_file):
        with open(counters_file) as f:
            rc = json.load(f).get(args.workload, {})
        if rc:
            roof["mfma_busy_counters"] = rc.get("mfma_busy")
            roof["mfma_busy_source"] = "profiles/read_counters.json (SQ_VALU_MFMA_BUSY_CYCLES over the read's " \
                                       "launches, per SIMD, over their GRBM_GUI_ACTIVE cycles)"
    # library GEMMs on the MFMA (bank K/V and its gradients, q/o weight gradients)
    gemms = {k: {"us": round(per[k][0] * 1e3, 2), "tflops": round(alg[k] / (per[k][0] * 1e-3) / 1e12, 1),
                 "mfma_frac": round(alg[k] / (per[k][0] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}
             for k in ("bank_kv_fwd", "bank_kv_bwd_dslots", "bank_kv_bwd_dw", "linear_wgrad") if k in per}
    gemms.update(torch_projection_gemms(layer, x, args.steps))
    # the prefix-mean router against HBM: forward reads x once and writes logits / probs / top-k /
    # gates / activations (plus the (N, R) projection written and read back when it runs as two
    # launches; the one-launch kernel `router_fwd` keeps it on chip); the backward reads x,
    # the incoming dx and writes dx (the accumulating input gradient), plus the (N, R) and (N, E)
    # per-token terms
    R_, E_, K_ = cfg["R"], E, cfg["K"]
    f_bytes = ntok * D * 2 + ntok * (2 * E_ + 2 * K_ + R_ + 2 * R_) * 4
    b_bytes = 3 * ntok * D * 2 + ntok * (3 * R_ + 2 * E_ + 3 * K_) * 4
    f_us = sum(per[k][0] * per[k][1] for k in ("router_fwd", "router_proj", "router_head") if k in per) * 1e3
    b_us = sum(per[k][0] * per[k][1] for k in ("router_bwd_token", "router_bwd_scan", "router_bwd_dx",
                                               "router_reduce") if k in per) * 1e3
    router = {"fwd_alg_bytes": f_bytes, "fwd_us": round(f_us, 2), "bwd_alg_bytes": b_bytes, "bwd_us": round(b_us, 2)}
    if f_us > 0:
        router["fwd_gbs"] = round(f_bytes / (f_us * 1e-6) / 1e9, 1)
        router["fwd_hbm_frac"] = round(router["fwd_gbs"] / PEAK_HBM_GBS, 4)
    if b_us > 0:
        router["bwd_gbs"] = round(b_bytes / (b_us * 1e-6) / 1e9, 1)
        router["bwd_hbm_frac"] = round(router["bwd_gbs"] / PEAK_HBM_GBS, 4)
    line = {
        "metric": METRIC,
        "value": round(ntok / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init weights, RMS-normed N(0,1) x in bf16, N(0,1) dy in fp32)",
        "config": {"workload": f"{args.workload}: MoM layer fwd+bwd B={B} T={T} d={D} heads={H}x{D // H} "
                               f"bank {E}x{BS} top-{cfg['K']} rank {cfg['R']}",
                   "global_batch": B, "seq_len": T, "parallelism": "single-gpu"},
        "roofline": roof,
        "read": {"active_tile_blocks": A, "active_per_tile": round(A / (B * ((T + 127) // 128)), 3),
                 "token_order": order_mode, "executed_tile_blocks": A_exec,
                 "alg_flop": read_flop, "ms": round(read_ms, 4), "tflops": round(read_tf, 2),
                 "mfma_frac": round(read_tf / PEAK_BF16_TFLOPS, 4)},
        "gemms": gemms,
        "router": router,
        "kernels_us": {k: round(v[0] * 1e3, 2) for k, v in sorted(per.items())},
        "kernels_timing": f"HIP events per launch over a second region of {args.steps} steps "
                          f"({ms_per_step_events:.4f} ms/step with the events)",
    }
    if args.copy_probe_mib > 0:
        src = torch.ones(args.copy_probe_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        line["copy_probe_bytes"] = src.numel()
        del src, dst
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.cpu_sample_batch)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
