"""Host logic of heatkv_amd/harness.py that needs no GPU: method names, the
seeded removal orders (valid orders for the policy), the result fields."""

from __future__ import annotations

import pytest
import torch

from heatkv_amd import harness as Hn
from heatkv_amd import policy as P


def test_method_names_follow_the_reference():
    assert Hn.normalize_method("baseline") == "baseline"
    for name in ("real_scale_fused_segmented", "fused-segmented", "fused_segmented"):
        assert Hn.normalize_method(name) == "real_scale_fused_segmented"
    with pytest.raises(ValueError, match="unsupported method"):
        Hn.normalize_method("dense")


def test_seeded_orders_are_valid_policy_input():
    orders = Hn.seeded_orders(32, 16, 9, seed=4)
    assert orders == Hn.seeded_orders(32, 16, 9, seed=4)
    norm = P.normalize_orders(orders, num_layers=32, num_heads=16, source_scale_start=3)
    assert len(norm) == 9 and all(len(o) == 512 for o in norm)
    ctrl = P.controller_for_budget(0.1, orders, num_layers=32, num_heads=16, protected_prefix_scales=3)
    assert sum(len(ctrl.removed_heads_for(l, 12, 5)) for l in range(32)) > 0


def test_layers_for_each_method():
    base = Hn.build_layers("baseline", num_layers=2, num_heads=4, budget=0.1, initial_scales=3, orders=None)
    assert all(not any(l.removed(t) for t in range(13)) for l in base)
    orders = Hn.seeded_orders(2, 4, 9, seed=1)
    fused = Hn.build_layers("real_scale_fused_segmented", num_layers=2, num_heads=4, budget=0.1,
                            initial_scales=3, orders=orders)
    assert any(l.schedule.capacity < l.schedule.capacity_bound or l.removed(12) for l in fused)


def test_synthetic_layers_get_the_patched_forward():
    from heatkv_amd.attention_forward import real_scale_fused_segmented_forward

    orders = Hn.seeded_orders(2, 4, 9, seed=1)
    model = Hn.build_model("real_scale_fused_segmented", device="cpu", num_layers=2, num_heads=4, embed_dim=512,
                          budget=0.2, initial_scales=3, orders=orders)
    for i, layer in enumerate(model):
        assert layer.layer_idx == i and layer.forward.__func__ is real_scale_fused_segmented_forward
        assert layer.mat_qkv.weight.dtype == torch.bfloat16
        layer.kv_caching(True)
        assert layer.caching and layer.heatkv_cache.logical_len == 0
    base = Hn.build_model("baseline", device="cpu", num_layers=2, num_heads=4, embed_dim=512, budget=0.2,
                         initial_scales=3, orders=orders)
    ctrl = base[0].heatkv_controller
    assert all(not any(ctrl.removed_heads_by_source_for(l, t).values()) for l in range(2) for t in range(13))


def test_forward_parameter_caches_follow_parameter_updates():
    from heatkv_amd import attention_forward as AF

    layer = Hn.SyntheticSelfAttention(256, 2, seed=3)
    x = torch.zeros((1, 4, 256))
    b1 = AF._qkv_bias(layer, x)
    assert AF._qkv_bias(layer, x) is b1
    assert torch.equal(b1, torch.cat((layer.q_bias, layer.zero_k_bias, layer.v_bias)))
    s1 = AF._scale_mul(layer)
    assert AF._scale_mul(layer) is s1
    with torch.no_grad():
        layer.q_bias.add_(1.0)
        layer.scale_mul_1H11.fill_(10.0)  # clamped at log(100)
    b2 = AF._qkv_bias(layer, x)
    assert b2 is not b1 and torch.equal(b2, torch.cat((layer.q_bias, layer.zero_k_bias, layer.v_bias)))
    s2 = AF._scale_mul(layer)
    assert s2 is not s1 and torch.allclose(s2, torch.full((2,), 100.0))
