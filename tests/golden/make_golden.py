#!/usr/bin/env python3
"""Write golden vectors for the MoM oracle from the reference's own code.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py [/root/reference]

It imports mom_kernels/reference.py of the reference tree by file path (a
torch-only module) and evaluates, at the reference test-suite shapes
(tests/test_parity.py:74-96: B=2, S=64, H=2, hd=16, 4 blocks x 16 slots,
top-2, router rank 8, bank ~ N(0,1), mom_scale 0.5):

  * build_gate_bias            (reference.py:14-29), duplicate ids included
  * prefix_mean_reference      (reference.py:32-36)
  * mom_attention_reference    (reference.py:39-61), shared and batched K/V
  * mom_full_reference         (reference.py:64-95), the full layer forward

with inputs drawn here from fixed seeds.  mom_full_reference is driven with a
stand-in layer that carries the parameters and attributes the function reads
(the oracle's OracleMoMLayer), so model.py and transformers are not needed.
Inputs and outputs are stored as float32 / int64 arrays in golden_mom.npz.
"""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)


def load_reference(ref_root):
    path = os.path.join(ref_root, "mom_kernels", "reference.py")
    spec = importlib.util.spec_from_file_location("naylis_reference_math", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(ref_root="/root/reference"):
    ref = load_reference(ref_root)
    import oracle

    B, S, H, HD = 2, 64, 2, 16
    D = H * HD
    NB, BS, T, R = 4, 16, 2, 8
    L = NB * BS
    out = {}

    # --- gate bias, duplicate block ids allowed (test_parity.py:144)
    g = torch.Generator().manual_seed(5)
    gates = torch.softmax(torch.randn(B, S, T, generator=g), -1)
    top = torch.randint(0, NB, (B, S, T), generator=g)
    out["bias_top_idx"] = top.numpy()
    out["bias_gates"] = gates.numpy()
    out["bias_fp32"] = ref.build_gate_bias(top, gates, NB, BS, torch.float32).numpy()
    out["bias_bf16mask"] = ref.build_gate_bias(top, gates, NB, BS, torch.bfloat16).numpy()

    # --- prefix mean, fp32 and bf16 inputs
    x = torch.randn(B, S, D, generator=g)
    out["pm_x"] = x.numpy()
    out["pm_h"] = ref.prefix_mean_reference(x).numpy()
    xb = x.bfloat16()
    out["pm_xb_as_f32"] = xb.float().numpy()
    out["pm_hb"] = ref.prefix_mean_reference(xb).numpy()

    # --- attention with the per-token bias, shared and batched K/V
    q = torch.randn(B, S, H, HD, generator=g) * 0.7
    k = torch.randn(L, D, generator=g) * 0.4
    v = torch.randn(L, D, generator=g) * 0.4
    bias = ref.build_gate_bias(top, gates, NB, BS, torch.float32)
    out["att_q"], out["att_k"], out["att_v"] = q.numpy(), k.numpy(), v.numpy()
    out["att_out"] = ref.mom_attention_reference(q, k, v, bias).numpy()
    kb = k.unsqueeze(0).expand(B, -1, -1).contiguous()
    vb = v.unsqueeze(0).expand(B, -1, -1).contiguous()
    out["att_out_batched"] = ref.mom_attention_reference(q, kb, vb, bias).numpy()

    # --- full layer forward at the suite shapes (test_parity.py:80-110)
    torch.manual_seed(7)
    layer = oracle.OracleMoMLayer(D, H, NB * BS, BS, T, R)
    layer.mom_scale.data.fill_(0.5)
    layer.eval()
    layer.noise_scale = 0.0
    torch.manual_seed(11)
    M = torch.randn(NB, BS * D)
    xl = torch.randn(B, S, D, generator=g)
    with torch.no_grad():
        y, probs, idx, gts = ref.mom_full_reference(xl, layer, M)
    for name, p in layer.state_dict().items():
        out["layer." + name] = p.numpy()
    out["layer_x"], out["layer_M"] = xl.numpy(), M.numpy()
    out["layer_y"], out["layer_probs"] = y.numpy(), probs.numpy()
    out["layer_top_idx"], out["layer_top_gates"] = idx.numpy(), gts.numpy()

    dst = os.path.join(HERE, "golden_mom.npz")
    np.savez_compressed(dst, **out)
    print(f"wrote {dst} ({os.path.getsize(dst)} bytes, {len(out)} arrays) with torch {torch.__version__}")


if __name__ == "__main__":
    main(*sys.argv[1:])
