"""Python surface: argument validation mirrors the reference's (CPU tensors).

The reference checks shapes/devices first and raises ValueError, then raises
RuntimeError for non-GPU tensors (real_pruning_fused_attention.py:385-396,
465-525).  This library has no CPU path, so CPU tensors raise RuntimeError
even with ``allow_cpu_fallback=True``.
"""

from __future__ import annotations

import pytest
import torch

from heatkv_amd import fused_real_pruning_flat_segmented_attention as attn
from heatkv_amd import pack_flat_segments_kv as pack
from heatkv_amd.real_pruning_fused_attention import _fused_qk_dot_mode_id, _fused_value_dot_mode_id, \
    _positive_int_env


def _args(B=1, H=2, L=3, D=128, cap=10, S=2):
    return dict(q=torch.zeros(B, H, L, D), persisted_k=torch.zeros(B, cap, D),
                persisted_v=torch.zeros(B, cap, D), segment_starts=torch.zeros(H, S, dtype=torch.int32),
                segment_ends=torch.zeros(H, S, dtype=torch.int32),
                segment_counts=torch.zeros(H, dtype=torch.int32), current_k=torch.zeros(B, H, L, D),
                current_v=torch.zeros(B, H, L, D), softmax_scale=0.1)


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(q=torch.zeros(1, 2, 3)), "must have shape \\[B, H, L, D\\]"),
    (lambda a: a.update(current_k=torch.zeros(1, 2, 4, 128)), "identical \\[B, H, L, D\\]"),
    (lambda a: a.update(persisted_k=torch.zeros(1, 10)), "persisted_k and persisted_v must have shape"),
    (lambda a: a.update(persisted_v=torch.zeros(1, 11, 128)), "identical shapes"),
    (lambda a: a.update(persisted_k=torch.zeros(2, 10, 128), persisted_v=torch.zeros(2, 10, 128)),
     "batch dimension"),
    (lambda a: a.update(persisted_k=torch.zeros(1, 10, 64), persisted_v=torch.zeros(1, 10, 64)), "head_dim must match"),
    (lambda a: a.update(persisted_k=torch.zeros(1, 10, 128, dtype=torch.float16)), "identical shapes|dtype"),
    (lambda a: a.update(segment_ends=torch.zeros(2, 3, dtype=torch.int32)), "identical shapes"),
    (lambda a: a.update(segment_starts=torch.zeros(3, 2, dtype=torch.int32),
                        segment_ends=torch.zeros(3, 2, dtype=torch.int32)), "shape \\[H, S\\]"),
    (lambda a: a.update(segment_counts=torch.zeros(3, dtype=torch.int32)), "shape \\[H\\]"),
    (lambda a: a.update(softmax_mode="exp10"), "unsupported softmax_mode"),
])
def test_attention_value_errors(mutate, msg):
    a = _args()
    mutate(a)
    with pytest.raises(ValueError, match=msg):
        attn(**a)


def test_attention_persisted_dtype_mismatch():
    a = _args()
    a["persisted_k"] = a["persisted_k"].half()
    a["persisted_v"] = a["persisted_v"].half()
    with pytest.raises(ValueError, match="persisted_k dtype must match current_k"):
        attn(**a)


@pytest.mark.parametrize("fallback", [False, True])
def test_attention_cpu_tensors_raise(fallback):
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        attn(**_args(), allow_cpu_fallback=fallback)


def test_attention_none_persisted_accepted_until_device_check():
    a = _args()
    a["persisted_k"] = a["persisted_v"] = None
    a["segment_starts"] = a["segment_ends"] = torch.zeros(2, 0, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        attn(**a)


def _pack_args(B=1, S=20, C=30, D=128, n=2):
    return dict(dst_k=torch.zeros(B, C, D), dst_v=torch.zeros(B, C, D), src_k=torch.zeros(B, S, D),
                src_v=torch.zeros(B, S, D), dst_starts=torch.zeros(n, dtype=torch.int64),
                src_starts=torch.zeros(n, dtype=torch.int64), lengths=torch.ones(n, dtype=torch.int64))


@pytest.mark.parametrize("mutate,msg", [
    (lambda a: a.update(dst_k=torch.zeros(1, 30)), "expects dst_k shaped"),
    (lambda a: a.update(dst_v=torch.zeros(1, 31, 128)), "matching K/V destination shapes"),
    (lambda a: a.update(src_v=torch.zeros(1, 21, 128)), "matching K/V source shapes"),
    (lambda a: a.update(src_k=torch.zeros(2, 20, 128), src_v=torch.zeros(2, 20, 128)), "matching batch and head_dim"),
])
def test_pack_value_errors(mutate, msg):
    a = _pack_args()
    mutate(a)
    with pytest.raises(ValueError, match=msg):
        pack(**a)


def test_pack_cpu_tensors_raise():
    with pytest.raises(RuntimeError, match="requires CUDA tensors"):
        pack(**_pack_args())


def test_env_knobs(monkeypatch):
    monkeypatch.setenv("REAL_PRUNING_FUSED_BLOCK_M", "abc")
    assert _positive_int_env("REAL_PRUNING_FUSED_BLOCK_M", 64) == 64
    monkeypatch.setenv("REAL_PRUNING_FUSED_BLOCK_M", "-3")
    assert _positive_int_env("REAL_PRUNING_FUSED_BLOCK_M", 64) == 64
    monkeypatch.setenv("REAL_PRUNING_FUSED_BLOCK_M", "128")
    assert _positive_int_env("REAL_PRUNING_FUSED_BLOCK_M", 64) == 128
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "TF32")
    assert _fused_qk_dot_mode_id() == 1
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "int8")
    with pytest.raises(ValueError):
        _fused_qk_dot_mode_id()
    monkeypatch.setenv("REAL_PRUNING_FUSED_VALUE_DOT_MODE", "mixed")
    assert _fused_value_dot_mode_id() == 2
    monkeypatch.setenv("REAL_PRUNING_FUSED_VALUE_DOT_MODE", "tf32")
    with pytest.raises(ValueError):
        _fused_value_dot_mode_id()


def test_qkv_produce_rejects_cpu_and_non_bf16():
    from heatkv_amd.produce import qkv_produce

    with pytest.raises(RuntimeError, match="GPU only"):
        qkv_produce(torch.zeros((1, 4, 3 * 2 * 128), dtype=torch.bfloat16), 2)


def test_mixed_qk_promotion_rules():
    """q and k of different dtypes: refused in the default QK mode, the 16-bit
    side widened to fp32 (exactly) in the fp32-class modes, and a widened k
    refuses the in-launch append (it would write a copy)."""
    from heatkv_amd.real_pruning_fused_attention import _promote_mixed_qk

    q = torch.randn(1, 2, 8, 128)
    k = torch.randn(1, 2, 8, 128).to(torch.bfloat16)
    sk = torch.randn(1, 16, 128).to(torch.bfloat16)
    with pytest.raises(RuntimeError, match="one dtype"):
        _promote_mixed_qk(q, sk, k, 0, None)
    q2, sk2, k2 = _promote_mixed_qk(q, sk, k, 1, None)
    assert q2 is q and sk2.dtype == torch.float32 and k2.dtype == torch.float32
    assert torch.equal(k2, k.float()) and torch.equal(sk2, sk.float())
    with pytest.raises(ValueError, match="append after the call"):
        _promote_mixed_qk(q, sk, k, 2, torch.zeros(2, dtype=torch.int32))
    qb = q.to(torch.bfloat16)
    q3, sk3, k3 = _promote_mixed_qk(qb, sk.float(), k.float(), 2, torch.zeros(2, dtype=torch.int32))
    assert q3.dtype == torch.float32 and torch.equal(q3, qb.float()) and k3.dtype == torch.float32


def test_item_shape_helpers_follow_promotion(monkeypatch):
    """attention_queries_per_item and attention_fuses_append answer for the
    kernel the operator runs after widening mixed q/k to fp32: under tf32,
    bf16 q with fp32 k and 16-bit v is the split-row kernel's call (256-query
    items, no fused append), and fp32 q with 16-bit k widens k, which refuses
    the append."""
    from heatkv_amd.real_pruning_fused_attention import attention_fuses_append, attention_queries_per_item

    f32, bf16 = torch.float32, torch.bfloat16
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "tf32")
    assert attention_queries_per_item(f32, f32, bf16) == 256
    assert attention_queries_per_item(bf16, f32, bf16) == 256
    assert attention_queries_per_item(f32, bf16, bf16) == 256
    assert attention_queries_per_item(bf16, bf16, bf16) == 128
    assert not attention_fuses_append(bf16, f32, bf16)
    assert not attention_fuses_append(f32, bf16, bf16)
    assert attention_fuses_append(bf16, bf16, bf16)
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "fp32")
    # staged fp32 kernel: 128-query items; fp32 k takes the append, widened bf16 k does not
    assert attention_queries_per_item(bf16, f32, bf16) == 128
    assert attention_fuses_append(bf16, f32, bf16)
    assert not attention_fuses_append(f32, bf16, bf16)
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "bf16")
    # the default mode refuses mixed q/k; the helpers answer for the dtypes as given
    assert attention_queries_per_item(bf16, f32, bf16) == 128


def test_env_get_matches_os_environ(monkeypatch):
    """The knob reader sees what os.environ.get sees: unset, set, changed,
    empty and deleted values, and the default."""
    import os

    from heatkv_amd._lib import env_get

    name = "HKV_TEST_ENV_GET_KNOB"
    monkeypatch.delenv(name, raising=False)
    assert env_get(name) is None and env_get(name, "d") == "d"
    for value in ("1", "0", "", "fp32", "é"):
        monkeypatch.setenv(name, value)
        assert env_get(name) == os.environ.get(name) == value
        assert env_get(name, "d") == value
    monkeypatch.delenv(name)
    assert env_get(name, "d") == "d" == os.environ.get(name, "d")
