"""Attention-layer forward of the fused segmented path (the patched ``forward``).

``real_scale_fused_segmented_forward`` replaces a cosine-attention layer's
forward like ``_real_pruning_scale_specific_fast_forward``
(enable_real_pruning_fast.py:1951-2254) does, with the same signature and
checks:

1. QKV projection ``F.linear`` with the ``(q_bias, zero_k_bias, v_bias)``
   bias (:2040-2044; a library GEMM, bf16 under autocast);
2. one HIP kernel (:func:`heatkv_amd.produce.qkv_produce`): cosine-attention
   normalize and ``scale_mul`` (:2052-2060), 2-D RoPE (:2062-2072,
   infinity/models/basic.py:97-117), the ``[B, H, L, D]`` permute, and the
   append of the kept heads' rows into the slab where this scale's attention
   does not read them;
3. the layer's segmented cache step (HIP segmented attention, remaining
   appends / packs; :2074-2254);
4. output projection (:2172).

The layer needs the attributes of Infinity's ``SelfAttention``
(infinity/models/basic.py:196-241): ``mat_qkv``, ``q_bias``, ``zero_k_bias``,
``v_bias``, ``scale_mul_1H11``, ``max_scale_mul``, ``cos_attn``, ``scale``,
``num_heads``, ``head_dim``, ``proj``, ``proj_drop``, ``caching``; and the
``heatkv_cache`` that :func:`heatkv_amd.enable.enable_real_pruning_scale_specific_fused_segmented`
attaches.

Precision: the reference runs its dense-prefix scales through the model's own
flash attention with q and k cast to bf16 (basic.py:296-302) and its
segmented scales with fp32 q and k (a TF32 product); here every scale attends
with the fp32 q and k of the producer (split-bf16 products, about 16
significand bits); the producer writes that K as split rows (bf16 high and
low parts, the split-row kernel's K format), so the cache keeps K in that
form and no attention call splits it again.  With
``REAL_PRUNING_FUSED_QK_DOT_MODE=tf32`` (the
reference's knob for TF32 q/k products) a cosine-attention layer's producer
writes q and k as fp16 instead: the same 11-bit significand as TF32, exact
range for cosine attention (|k| = 1, |q| <= exp(max_scale_mul)), half the K
cache, and the 16-bit attention kernel (one product per MFMA step instead of
three).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .produce import qkv_produce, rope_start, rope_table_for, scale_mul_of
from .real_pruning_fused_attention import _fused_qk_dot_mode_id, split_rows_k_format

_QK_DOT_TF32 = 1


def _versions(*tensors):
    return tuple((t.data_ptr(), t._version, t.dtype, t.device) for t in tensors)


def _autocast_dtype(x):
    if x.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return None


def _qkv_bias(layer, x):
    """``cat(q_bias, zero_k_bias, v_bias)`` as the projection takes it (cast to
    the autocast dtype, as autocast casts it), remade only when a bias tensor
    changes (its storage or version): parameters do not change between the
    steps of a generation, and each remake costs the chain two small kernels."""
    dtype = _autocast_dtype(x)
    key = (_versions(layer.q_bias, layer.zero_k_bias, layer.v_bias), dtype)
    hit = getattr(layer, "_heatkv_qkv_bias", None)
    if hit is None or hit[0] != key:
        bias = torch.cat((layer.q_bias, layer.zero_k_bias, layer.v_bias))
        hit = (key, bias if dtype is None else bias.to(dtype))
        layer._heatkv_qkv_bias = hit
    return hit[1]


def _scale_mul(layer):
    """:func:`scale_mul_of` of the layer, remade only when ``scale_mul_1H11`` changes."""
    key = (_versions(layer.scale_mul_1H11), float(layer.max_scale_mul))
    hit = getattr(layer, "_heatkv_scale_mul", None)
    if hit is None or hit[0] != key:
        hit = (key, scale_mul_of(layer))
        layer._heatkv_scale_mul = hit
    return hit[1]


def real_scale_fused_segmented_forward(self, x, attn_bias_or_two_vector=None, attn_fn=None,
                                       scale_schedule=None, rope2d_freqs_grid=None, scale_ind=0):
    if not self.caching:
        raise NotImplementedError("real pruning fused segmented only supports kv-cached inference")
    if attn_bias_or_two_vector is not None:
        raise NotImplementedError("real pruning fused segmented does not support training attention masks")
    if attn_fn is not None:
        raise NotImplementedError("real pruning fused segmented does not support custom attention functions")

    batch_size, seq_len, _ = x.shape
    qkv = F.linear(input=x, weight=self.mat_qkv.weight, bias=_qkv_bias(self, x))
    table = None
    start = 0
    if rope2d_freqs_grid is not None:
        if scale_schedule is None:
            raise ValueError("scale_schedule is required when rope2d_freqs_grid is provided")
        table = rope_table_for(rope2d_freqs_grid, scale_schedule, qkv.device)
        start = rope_start(scale_schedule, scale_ind)
    cos_attn = bool(self.cos_attn)
    # q and k are fp32 wherever the reference promotes them (cosine attention
    # or RoPE); otherwise they keep the projection's dtype as in the
    # reference (bf16 under its bf16 autocast).  TF32 dot mode
    # on a cosine-attention layer: fp16 (TF32's significand, values in range).
    qk_dtype = torch.float32 if (cos_attn or table is not None) else qkv.dtype
    if cos_attn and _fused_qk_dot_mode_id() == _QK_DOT_TF32:
        qk_dtype = torch.float16
    # fp32 K that the attention reads as split rows is written in that form
    # by the producer (and kept so in the cache), so no call splits it again
    k_split = split_rows_k_format(qk_dtype, qk_dtype, qkv.dtype)
    cache = self.heatkv_cache
    append = cache.producer_append(int(scale_ind), qk_dtype, qkv.device)
    q, k, v = qkv_produce(
        qkv.view(batch_size, seq_len, 3 * self.num_heads * self.head_dim), self.num_heads,
        scale_mul=_scale_mul(self) if cos_attn else None, rope_table=table, rope_start_row=start,
        normalize=cos_attn, qk_dtype=qk_dtype, append=append, k_split_rows=k_split)
    del qkv
    # under autocast the projection takes the attention output in the autocast
    # dtype: the kernel writes it rounded once, as autocast's cast would
    output = cache.step(q, k, v, int(scale_ind), float(self.scale), appended=append is not None,
                        out_dtype=_autocast_dtype(x), k_split_rows=k_split)
    return self.proj_drop(self.proj(output))


def real_scale_fused_segmented_kv_caching(self, enable: bool):
    """kv_caching patch (enable_real_pruning_fast.py:2257-2276): the layer's own
    switch, then an empty segmented cache."""
    self._pre_heatkv_kv_caching(enable)
    self.heatkv_cache.reset()
