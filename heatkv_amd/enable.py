"""Enabling the fused segmented path on a model's attention layers.

Mirrors ``enable_real_pruning_scale_specific_fused_segmented`` /
``enable_real_pruning_scale_specific_fast`` (enable_real_pruning_fast.py:
2279-2402): find the attention layers, number them, compute the HeatKV
removal policy for the budget (:mod:`heatkv_amd.policy`), build each layer's
static slab schedule (:func:`heatkv_amd.slab_schedule.build_static_slot_schedule`)
and give each layer its segmented KV cache
(:class:`heatkv_amd.segmented_cache.SegmentedLayerCache`).

Layers with Infinity's ``SelfAttention`` attributes (``mat_qkv`` ...) also
get their ``forward`` and ``kv_caching`` replaced, as the reference does
(:2381-2388), by :mod:`heatkv_amd.attention_forward` (QKV projection, the
fused HIP producer, the segmented cache step, output projection).  Other
modules only get the cache: their forward calls
``layer.heatkv_cache.step(q, k, v, scale_ind, softmax_scale)`` with its
post-RoPE ``q, k, v`` ``[B, H, L, D]`` where the reference's patched forward
runs its cache logic (:2040-2254), and gets the ``[B, L, H * D]`` attention
output to project.
"""

from __future__ import annotations

import types
from typing import Callable, List, Optional, Sequence

from .attention_forward import real_scale_fused_segmented_forward, real_scale_fused_segmented_kv_caching
from .policy import controller_for_budget
from .segmented_cache import SegmentedLayerCache
from .slab_schedule import SIDES_1M, build_static_slot_schedule

METHOD_NAME = "real_scale_fused_segmented"
METHOD_ALIASES = ("fused-segmented", "fused_segmented")


def canonical_method(name: str) -> str:
    """Harness method name with its aliases folded (profile_cache_methods.py:40-45, 144-154)."""
    key = str(name).strip()
    if key == METHOD_NAME or key in METHOD_ALIASES:
        return METHOD_NAME
    raise ValueError(f"unknown cache method {name!r}; this package provides {METHOD_NAME!r}")


def _default_filter(module) -> bool:
    return type(module).__name__ == "SelfAttention" and hasattr(module, "num_heads")


def attention_layers(model, module_filter: Optional[Callable] = None) -> List:
    """The model's attention layers in module order (the reference's
    ``isinstance(module, SelfAttention)`` scan)."""
    keep = module_filter or _default_filter
    return [m for m in model.modules() if keep(m)]


def enable_real_pruning_scale_specific_fused_segmented(
    model,
    budget,
    scale_specific_removal_orders,
    *,
    protected_prefix_scales: int = 4,
    source_scale_start: Optional[int] = None,
    skip_last_scale: bool = True,
    merge_mode: str = "exact",
    requested_generation_batch_size: Optional[int] = None,
    module_filter: Optional[Callable] = None,
    sides: Sequence[int] = SIDES_1M,
    patch_forward: bool = True,
):
    """Attach the policy, slab schedule and segmented cache to every attention
    layer of ``model`` (same arguments and checks as the reference entry;
    ``module_filter`` selects the layers, by default modules of a class named
    ``SelfAttention`` with a ``num_heads`` attribute) and, with
    ``patch_forward``, replace the forward of layers that have a ``mat_qkv``
    projection.  Returns ``model``."""
    if merge_mode != "exact":
        raise ValueError("real pruning fast v1 only supports merge_mode='exact'")
    layers = attention_layers(model, module_filter)
    if not layers:
        return model
    for idx, layer in enumerate(layers):
        layer.layer_idx = idx
    num_heads = layers[0].num_heads
    if any(layer.num_heads != num_heads for layer in layers):
        raise ValueError("real pruning fast requires all SelfAttention modules to use the same num_heads")
    ctrl = controller_for_budget(budget, scale_specific_removal_orders, num_layers=len(layers),
                                 num_heads=num_heads, protected_prefix_scales=protected_prefix_scales,
                                 source_scale_start=source_scale_start, skip_last_scale=skip_last_scale,
                                 sides=sides)
    for layer in layers:
        sched = build_static_slot_schedule(ctrl, layer_idx=layer.layer_idx, num_heads=num_heads)
        lid = layer.layer_idx
        layer.heatkv_controller = ctrl
        layer.heatkv_schedule = sched
        layer.heatkv_budget = float(budget)
        layer.heatkv_requested_generation_batch_size = (
            None if requested_generation_batch_size is None else int(requested_generation_batch_size))
        layer.heatkv_cache = SegmentedLayerCache(
            sched, lambda t, lid=lid: ctrl.removed_heads_by_source_for(lid, t), num_heads=num_heads,
            num_scales=len(sides))
        if patch_forward and hasattr(layer, "mat_qkv"):
            if not hasattr(layer, "_pre_heatkv_forward"):
                layer._pre_heatkv_forward = layer.forward
            layer.forward = types.MethodType(real_scale_fused_segmented_forward, layer)
            if not hasattr(layer, "_pre_heatkv_kv_caching"):
                layer._pre_heatkv_kv_caching = layer.kv_caching
            layer.kv_caching = types.MethodType(real_scale_fused_segmented_kv_caching, layer)
    return model


def enable_real_pruning_scale_specific_fast(
    model,
    budget,
    scale_specific_removal_orders,
    *,
    protected_prefix_scales: int = 4,
    source_scale_start: Optional[int] = None,
    skip_last_scale: bool = True,
    merge_mode: str = "exact",
    attention_impl: str = "fused_segmented",
    requested_generation_batch_size: Optional[int] = None,
    module_filter: Optional[Callable] = None,
    sides: Sequence[int] = SIDES_1M,
    patch_forward: bool = True,
):
    """The reference's general entry (enable_real_pruning_fast.py:2279-2378):
    ``attention_impl`` must be ``"fused_segmented"`` (the only implementation
    the reference has too); then as
    :func:`enable_real_pruning_scale_specific_fused_segmented`."""
    if merge_mode != "exact":
        raise ValueError("real pruning fast v1 only supports merge_mode='exact'")
    if attention_impl != "fused_segmented":
        raise ValueError(f"unsupported real pruning fast attention_impl: {attention_impl!r}")
    return enable_real_pruning_scale_specific_fused_segmented(
        model, budget, scale_specific_removal_orders, protected_prefix_scales=protected_prefix_scales,
        source_scale_start=source_scale_start, skip_last_scale=skip_last_scale, merge_mode=merge_mode,
        requested_generation_batch_size=requested_generation_batch_size, module_filter=module_filter,
        sides=sides, patch_forward=patch_forward)
