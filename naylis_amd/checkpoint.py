"""Checkpoint layout of the MoM read: legacy key names, bank geometry from the
weights, and per-layer state dicts (evaluate.py:198-289, model.py:305-306,374).

A Naylis checkpoint stores the shared bank once as ``model.M_blocks``
(num_blocks, block_size * hidden) and each decoder layer's read under
``model.layers.<i>.mom.`` (router_down, router_up, q_proj, k_proj, v_proj,
o_proj, mom_scale) with its pre-norm under ``model.layers.<i>.mom_norm.``.
``naylis_amd.layer.MoMLayer`` uses the same parameter names, so a layer's
slice of the checkpoint loads into it with ``strict=True``.

Checkpoints written by the standalone training scripts name the submodules
graph_mem / graph_norm / graph_scale and carry no MoM keys in their config;
``remap_legacy_keys`` renames them and ``mom_kwargs_from_state_dict`` derives
the geometry from the tensor shapes, as evaluate.py does.
"""
from __future__ import annotations

import logging
import re

import torch

from .layer import MoMLayer, cast_mom_layer

__all__ = ["LEGACY_TOP_BLOCKS", "LEGACY_AUX_WEIGHT", "remap_legacy_keys", "mom_kwargs_from_state_dict",
           "mom_layer_indices", "mom_layer_state_dict", "mom_layers_from_state_dict"]

# Not recoverable from the weights: every legacy run routed top-2 and used
# aux weight 0.01 (evaluate.py:232-233).
LEGACY_TOP_BLOCKS = 2
LEGACY_AUX_WEIGHT = 0.01

_log = logging.getLogger(__name__)
_LAYER_MOM = re.compile(r"^(.*\.)?layers\.(\d+)\.mom\.")


def remap_legacy_keys(state_dict):
    """Rename legacy keys to the current layout (evaluate.py:198-229).

    ``.graph_mem.`` -> ``.mom.``, ``.graph_norm.`` -> ``.mom_norm.``, and a
    key that then ends in ``.mom.graph_scale`` -> ``.mom.mom_scale``.  Tensors
    are passed through (same objects); a dict with no legacy key comes back
    with the same keys in the same order.  As in the reference, a later key
    that lands on an earlier one's new name replaces its value.
    """
    out = {}
    renamed = 0
    for key, value in state_dict.items():
        new = key.replace(".graph_mem.", ".mom.").replace(".graph_norm.", ".mom_norm.")
        if new.endswith(".mom.graph_scale"):
            new = new[: -len("graph_scale")] + "mom_scale"
        if new != key:
            renamed += 1
        out[new] = value
    if renamed:
        _log.info("legacy checkpoint layout: %d keys renamed (graph_mem/graph_norm/graph_scale -> "
                  "mom/mom_norm/mom_scale)", renamed)
    return out


def mom_kwargs_from_state_dict(state_dict, hidden_size, config=None):
    """MoM constructor kwargs for a checkpoint (evaluate.py:236-289).

    Returns None when no key contains ``.mom.``.  If ``config`` carries
    ``mem_size`` its mom_* fields are returned as they are; otherwise the
    geometry comes from the weights: num_blocks and block_size from
    ``model.M_blocks`` (num_blocks, block_size * hidden_size), router_rank from
    the first ``*.mom.router_down.weight`` (router_rank, hidden_size), and
    top_blocks / aux_weight take the legacy protocol values.  Raises
    RuntimeError when the bank or the router is missing.
    """
    if not any(".mom." in k for k in state_dict):
        return None
    mem_size = getattr(config, "mem_size", None) if config is not None else None
    if mem_size is not None:
        return {
            "mem_size": mem_size,
            "mom_block_size": config.mom_block_size,
            "mom_top_blocks": config.mom_top_blocks,
            "mom_router_rank": config.mom_router_rank,
            "mom_aux_weight": config.mom_aux_weight,
        }
    bank = state_dict.get("model.M_blocks")
    if bank is None:
        raise RuntimeError("MoM checkpoint without model.M_blocks: the bank geometry cannot be derived")
    router_down = next((v for k, v in state_dict.items() if k.endswith(".mom.router_down.weight")), None)
    if router_down is None:
        raise RuntimeError("MoM checkpoint without a router_down weight: router_rank cannot be derived")
    if bank.dim() != 2 or bank.shape[1] % hidden_size != 0:
        raise RuntimeError(f"model.M_blocks of shape {tuple(bank.shape)} is not (num_blocks, "
                           f"block_size * {hidden_size})")
    num_blocks = int(bank.shape[0])
    block_size = int(bank.shape[1]) // hidden_size
    return {
        "mem_size": num_blocks * block_size,
        "mom_block_size": block_size,
        "mom_top_blocks": LEGACY_TOP_BLOCKS,
        "mom_router_rank": int(router_down.shape[0]),
        "mom_aux_weight": LEGACY_AUX_WEIGHT,
    }


def mom_layer_indices(state_dict):
    """Sorted decoder-layer indices that hold a MoM read."""
    found = set()
    for k in state_dict:
        m = _LAYER_MOM.match(k)
        if m:
            found.add(int(m.group(2)))
    return sorted(found)


def mom_layer_state_dict(state_dict, layer, prefix="model.layers."):
    """One layer's MoM parameters with the ``<prefix><layer>.mom.`` prefix
    stripped — the keys ``MoMLayer.state_dict()`` has."""
    head = f"{prefix}{layer}.mom."
    return {k[len(head):]: v for k, v in state_dict.items() if k.startswith(head)}


def mom_layers_from_state_dict(state_dict, hidden_size, n_heads, config=None, prefix="model.layers.",
                               device=None, dtype=None):
    """Build one ``MoMLayer`` per MoM decoder layer of a checkpoint and load it
    strictly; returns (M_blocks, {layer index: MoMLayer}).

    Legacy keys are remapped first.  ``strict=True`` raises on any missing or
    unexpected key of a layer, which is the reference's strict check
    (evaluate.py:187-195) restricted to the MoM read.  ``dtype`` applies to
    the q/k/v/o projections and the bank only; the router weights and the
    ReZero scale stay fp32 (cast_mom_layer), so a layer loaded with
    dtype=torch.bfloat16 runs the fused HIP node directly.
    """
    state_dict = remap_legacy_keys(state_dict)
    kw = mom_kwargs_from_state_dict(state_dict, hidden_size, config)
    if kw is None:
        raise RuntimeError("checkpoint holds no MoM layer")
    bank = state_dict.get("model.M_blocks")
    if bank is None:
        raise RuntimeError("MoM checkpoint without model.M_blocks")
    layers = {}
    for i in mom_layer_indices(state_dict):
        layer = MoMLayer(hidden_size, n_heads, kw["mem_size"], kw["mom_block_size"], kw["mom_top_blocks"],
                         kw["mom_router_rank"])
        layer.load_state_dict(mom_layer_state_dict(state_dict, i, prefix), strict=True)
        if device is not None:
            layer = layer.to(device=device)
        if dtype is not None:
            cast_mom_layer(layer, dtype)
        layers[i] = layer
    bank = bank.detach().clone()
    if device is not None or dtype is not None:
        bank = bank.to(device=device, dtype=dtype)
    return torch.nn.Parameter(bank), layers
