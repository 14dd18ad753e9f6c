"""Checkpoint layout: legacy key remap, geometry from the weights, strict
per-layer loads (evaluate.py:198-289; the reference's own check is
test_parity.py:343-392, section 15)."""
import os
import tempfile
from types import SimpleNamespace

import pytest
import torch

import oracle
from naylis_amd import checkpoint as ck
from naylis_amd.layer import MoMLayer

D, H, NB, BS, K, R = 64, 4, 4, 16, 2, 8


def _model_state_dict(n_layers=3, mom_layers=(0, 2), seed=0):
    """A state dict in the reference's NaylisLlamaModel layout (model.py:305-306,
    374-381): the bank once, a mom / mom_norm pair in each MoM layer, trunk keys
    around them."""
    g = torch.Generator().manual_seed(seed)
    sd = {"model.embed_tokens.weight": torch.randn(32, D, generator=g),
          "model.M_blocks": torch.randn(NB, BS * D, generator=g) * 0.02}
    for i in range(n_layers):
        p = f"model.layers.{i}."
        sd[p + "self_attn.q_proj.weight"] = torch.randn(D, D, generator=g)
        sd[p + "input_layernorm.weight"] = torch.ones(D)
        if i in mom_layers:
            layer = oracle.OracleMoMLayer(D, H, NB * BS, BS, K, R)
            with torch.no_grad():
                for prm in layer.parameters():
                    prm.copy_(torch.randn(prm.shape, generator=g))
            for k, v in layer.state_dict().items():
                sd[p + "mom." + k] = v
            sd[p + "mom_norm.weight"] = torch.rand(D, generator=g)
    sd["model.norm.weight"] = torch.ones(D)
    return sd


def _to_legacy(sd):
    """The inverse rename the reference's test uses (test_parity.py:346-350)."""
    out = {}
    for k, v in sd.items():
        k2 = k.replace(".mom.", ".graph_mem.").replace(".mom_norm.", ".graph_norm.")
        k2 = k2.replace(".graph_mem.mom_scale", ".graph_mem.graph_scale")
        out[k2] = v
    return out


def test_remap_round_trip_restores_every_key():
    sd = _model_state_dict()
    legacy = _to_legacy(sd)
    n_renamed = sum(a != b for a, b in zip(sd, legacy))
    assert n_renamed == 2 * (7 + 1)
    back = ck.remap_legacy_keys(legacy)
    assert list(back) == list(sd)
    for k in sd:
        assert back[k] is sd[k]


def test_remap_rules_one_by_one():
    t = torch.zeros(1)
    legacy = {
        "model.layers.0.graph_mem.graph_scale": t,
        "model.layers.0.graph_mem.router_up.weight": t,
        "model.layers.0.graph_norm.weight": t,
        # graph_scale outside a MoM submodule, and names without the dots around them, stay
        "model.layers.0.other.graph_scale": t,
        "graph_mem.q_proj.weight": t,
        "model.layers.0.graph_memory.weight": t,
        "model.layers.0.graph_scale": t,
    }
    got = ck.remap_legacy_keys(legacy)
    assert list(got) == [
        "model.layers.0.mom.mom_scale",
        "model.layers.0.mom.router_up.weight",
        "model.layers.0.mom_norm.weight",
        "model.layers.0.other.graph_scale",
        "graph_mem.q_proj.weight",
        "model.layers.0.graph_memory.weight",
        "model.layers.0.graph_scale",
    ]


def test_remap_leaves_current_layout_alone():
    sd = _model_state_dict()
    got = ck.remap_legacy_keys(sd)
    assert list(got) == list(sd) and all(got[k] is sd[k] for k in sd)


def test_geometry_from_weights():
    sd = _model_state_dict()
    kw = ck.mom_kwargs_from_state_dict(sd, hidden_size=D)
    assert kw == {"mem_size": NB * BS, "mom_block_size": BS, "mom_top_blocks": 2, "mom_router_rank": R,
                  "mom_aux_weight": 0.01}
    # the row length divided by the hidden size, not the row count, is block_size
    bank = torch.zeros(8, 128 * 32)
    sd2 = {"model.M_blocks": bank, "model.layers.0.mom.router_down.weight": torch.zeros(24, 32)}
    assert ck.mom_kwargs_from_state_dict(sd2, hidden_size=32)["mom_block_size"] == 128
    assert ck.mom_kwargs_from_state_dict(sd2, hidden_size=32)["mem_size"] == 1024
    assert ck.mom_kwargs_from_state_dict(sd2, hidden_size=64)["mom_block_size"] == 64
    assert ck.mom_kwargs_from_state_dict(sd2, hidden_size=32)["mom_router_rank"] == 24


def test_geometry_from_config_wins():
    sd = _model_state_dict()
    cfg = SimpleNamespace(mem_size=4096, mom_block_size=256, mom_top_blocks=3, mom_router_rank=16,
                          mom_aux_weight=0.05)
    assert ck.mom_kwargs_from_state_dict(sd, D, cfg) == {
        "mem_size": 4096, "mom_block_size": 256, "mom_top_blocks": 3, "mom_router_rank": 16,
        "mom_aux_weight": 0.05}
    # a config without mem_size (a bare LlamaConfig) falls through to the weights
    assert ck.mom_kwargs_from_state_dict(sd, D, SimpleNamespace())["mem_size"] == NB * BS


def test_geometry_errors_and_vanilla():
    sd = _model_state_dict()
    assert ck.mom_kwargs_from_state_dict({k: v for k, v in sd.items() if ".mom." not in k}, D) is None
    with pytest.raises(RuntimeError, match="M_blocks"):
        ck.mom_kwargs_from_state_dict({k: v for k, v in sd.items() if k != "model.M_blocks"}, D)
    with pytest.raises(RuntimeError, match="router_down"):
        ck.mom_kwargs_from_state_dict({k: v for k, v in sd.items() if "router_down" not in k}, D)
    with pytest.raises(RuntimeError, match="M_blocks"):
        ck.mom_kwargs_from_state_dict(sd, hidden_size=D + 1)


def test_layers_load_strict_from_a_legacy_safetensors_folder():
    from safetensors.torch import load_file, save_file
    sd = _model_state_dict()
    with tempfile.TemporaryDirectory() as tmp:
        path = os.path.join(tmp, "model.safetensors")
        save_file({k: v.contiguous() for k, v in _to_legacy(sd).items()}, path)
        loaded = load_file(path)
    bank, layers = ck.mom_layers_from_state_dict(loaded, hidden_size=D, n_heads=H)
    assert sorted(layers) == [0, 2]
    assert torch.equal(bank, sd["model.M_blocks"])
    for i, layer in layers.items():
        assert isinstance(layer, MoMLayer)
        assert (layer.num_blocks, layer.block_size, layer.top_blocks) == (NB, BS, 2)
        for k, v in layer.state_dict().items():
            assert torch.equal(v, sd[f"model.layers.{i}.mom.{k}"]), k


def test_layer_strict_load_rejects_missing_and_unexpected():
    sd = _model_state_dict()
    with pytest.raises(RuntimeError, match="Missing"):
        ck.mom_layers_from_state_dict({k: v for k, v in sd.items() if not k.endswith("mom.mom_scale")}, D, H)
    extra = dict(sd)
    extra["model.layers.0.mom.gate_bias"] = torch.zeros(NB)
    with pytest.raises(RuntimeError, match="Unexpected"):
        ck.mom_layers_from_state_dict(extra, D, H)


def test_state_dict_moves_between_oracle_and_hip_layer():
    ref = oracle.OracleMoMLayer(D, H, NB * BS, BS, K, R)
    hip = MoMLayer(D, H, NB * BS, BS, K, R)
    assert list(ref.state_dict()) == list(hip.state_dict())
    hip.load_state_dict(ref.state_dict(), strict=True)
    ref2 = oracle.OracleMoMLayer(D, H, NB * BS, BS, K, R)
    ref2.load_state_dict(hip.state_dict(), strict=True)
    for k, v in ref.state_dict().items():
        assert torch.equal(v, ref2.state_dict()[k])


@pytest.mark.gpu
def test_legacy_loaded_layer_output_bitwise(dev):
    """Section 15a of the reference's test on the HIP layer: a layer loaded
    from the legacy layout with dtype=bf16 (no manual casts) gives the bitwise
    output of the original."""
    from naylis_amd.layer import cast_mom_layer
    torch.manual_seed(3)
    Dg, Hg = 256, 4
    orig = cast_mom_layer(MoMLayer(Dg, Hg, 4 * 64, 64, 2, 16).to(dev), torch.bfloat16)
    with torch.no_grad():
        orig.mom_scale.fill_(0.5)
    bank = (torch.randn(4, 64 * Dg, device=dev) * 0.5).bfloat16()
    sd = {"model.M_blocks": bank.cpu()}
    for k, v in orig.state_dict().items():
        sd["model.layers.5.mom." + k] = v.cpu()
    bank2, layers = ck.mom_layers_from_state_dict(_to_legacy(sd), Dg, Hg, device=dev, dtype=torch.bfloat16)
    assert bank2.dtype == torch.bfloat16 and layers[5].q_proj.weight.dtype == torch.bfloat16
    assert layers[5].router_down.weight.dtype == torch.float32 and layers[5].mom_scale.dtype == torch.float32
    x = torch.randn(2, 128, Dg, device=dev, dtype=torch.bfloat16)
    orig.eval()
    layers[5].eval()
    with torch.no_grad():
        a = orig(x, bank)
        b = layers[5](x, bank2)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_legacy_checkpoint_file_hip_layer_matches_oracle(dev):
    """A legacy-layout fp32 checkpoint file (safetensors, the reference's
    graph_mem / graph_scale names, evaluate.py:198-289) loaded into the HIP
    layer with dtype=bf16 and into the fp32 oracle layer: forward and
    backward through the fused node agree at the north-star tolerance,
    parameter gradients by the reference's scaled_max metric
    (the oracle sees the bf16-rounded projections and bank the HIP layer
    holds)."""
    from safetensors.torch import load_file, save_file

    from naylis_amd.mom_kernels.hip_layer import fused_layer_supported
    from tests._tol import assert_close, scaled_max
    Dg, Hg, NBg, BSg, Kg, Rg = 256, 4, 8, 64, 2, 32
    g = torch.Generator().manual_seed(11)
    src = oracle.OracleMoMLayer(Dg, Hg, NBg * BSg, BSg, Kg, Rg)
    with torch.no_grad():
        for p_ in src.parameters():
            p_.copy_(torch.randn(p_.shape, generator=g) * 0.05)
        src.mom_scale.fill_(0.7)
    sd = {"model.M_blocks": torch.randn(NBg, BSg * Dg, generator=g) * 0.5}
    for k, v in src.state_dict().items():
        sd["model.layers.3.mom." + k] = v
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.safetensors")
        save_file(_to_legacy(sd), path)
        loaded = load_file(path)
    bank, layers = ck.mom_layers_from_state_dict(loaded, Dg, Hg, device=dev, dtype=torch.bfloat16)
    hip = layers[3].train()
    hip.noise_scale = 0.0
    assert fused_layer_supported(torch.empty(1, 1, Dg, device=dev, dtype=torch.bfloat16), bank,
                                 hip.router_down.weight, hip.router_up.weight, hip.q_proj.weight, hip.k_proj.weight,
                                 hip.v_proj.weight, hip.o_proj.weight, hip.mom_scale)
    ref = oracle.OracleMoMLayer(Dg, Hg, NBg * BSg, BSg, Kg, Rg)
    ref.load_state_dict({k: v.detach().float().cpu() for k, v in hip.state_dict().items()}, strict=True)
    ref.noise_scale = 0.0
    x = torch.randn(2, 200, Dg, generator=g).bfloat16()
    dy = torch.randn(2, 200, Dg, generator=g)
    xd = x.to(dev).requires_grad_(True)
    bank = bank.detach().requires_grad_(True)
    y = hip(xd, bank)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    xr = x.float().requires_grad_(True)
    Mr = bank.detach().float().cpu().requires_grad_(True)
    yr = ref(xr, Mr)
    yr.backward(dy)
    assert_close(y, yr, "y")
    assert_close(xd.grad, xr.grad, "dx")
    assert_close(bank.grad, Mr.grad, "dM_blocks")
    # parameter gradients (sums over all tokens) by the reference's gradient metric, scaled_max =
    # max|a - b| / max|b| (test_parity.py:64-67, bar 2e-2 at :488-490), at half that bar, and a
    # relative Frobenius error of at most 1e-2
    for name in ("q_proj", "k_proj", "v_proj", "o_proj", "router_down", "router_up"):
        got = getattr(hip, name).weight.grad.double().cpu()
        exp = getattr(ref, name).weight.grad.double()
        sm = scaled_max(got, exp)
        fro = float((got - exp).norm() / exp.norm().clamp_min(1e-30))
        assert sm <= 1e-2 and fro <= 1e-2, f"d{name}: scaled_max {sm:.3e}, relative Frobenius {fro:.3e}"
