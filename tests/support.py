"""Shared helpers for the tests (imported by test modules; not collected)."""

from __future__ import annotations

import math

import numpy as np
import torch

# Tolerances of the attention contract (fp32-accumulated reference result).
OUT_MAX_ABS = 2e-2
OUT_MEAN_ABS = 2e-3
LSE_MAX_ABS = 1e-3


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy()


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw element bits (int16/int32 view) for bit-exact comparisons."""
    t = t.detach().cpu().contiguous()
    view = {2: torch.int16, 4: torch.int32}[t.element_size()]
    return t.view(view).numpy()


def assert_attention_close(out, lse, ref_out, ref_lse, *, max_abs=OUT_MAX_ABS,
                           mean_abs=OUT_MEAN_ABS, lse_abs=LSE_MAX_ABS, what=""):
    out = np.asarray(out, dtype=np.float64)
    ref_out = np.asarray(ref_out, dtype=np.float64)
    assert np.isfinite(out).all(), f"{what}: non-finite output"
    err = np.abs(out - ref_out)
    assert err.max() <= max_abs, f"{what}: out max-abs {err.max():.3e} > {max_abs}"
    assert err.mean() <= mean_abs, f"{what}: out mean-abs {err.mean():.3e} > {mean_abs}"
    if lse is not None:
        lerr = np.abs(np.asarray(lse, np.float64) - np.asarray(ref_lse, np.float64))
        assert lerr.max() <= lse_abs, f"{what}: lse max-abs {lerr.max():.3e} > {lse_abs}"
    return float(err.max()), float(err.mean())


def torch_qkv_prologue(qkv: torch.Tensor, scale_mul: torch.Tensor, table: torch.Tensor, start: int):
    """The reference layer prologue as torch ops in fp32 on the CPU: ``qkv``
    ``[B, L, 3, H, D]`` (bf16 values) -> q, k ``[B, H, L, D]`` fp32 and v.

    enable_real_pruning_fast.py:2040-2072 under bf16 autocast (``norm`` runs in
    fp32 there, so normalize gives fp32) and apply_rotary_emb
    (infinity/models/basic.py:97-117) with ``table`` ``[2, T, D // 2]``."""
    import torch.nn.functional as F

    B, L, _, H, D = qkv.shape
    q, k, v = qkv.float().unbind(dim=2)
    q = q.permute(0, 2, 1, 3).contiguous()
    k = k.permute(0, 2, 1, 3).contiguous()
    v = v.permute(0, 2, 1, 3).contiguous()
    q = F.normalize(q, dim=-1, eps=1e-12).mul(scale_mul.float().reshape(1, H, 1, 1))
    k = F.normalize(k, dim=-1, eps=1e-12)
    rc = table[:, start:start + L]
    qk = torch.stack((q, k), dim=0).reshape(2, B, H, L, D // 2, 2)
    qk = torch.stack([rc[0] * qk[..., 0] - rc[1] * qk[..., 1],
                      rc[1] * qk[..., 0] + rc[0] * qk[..., 1]], dim=-1)
    q, k = qk.reshape(2, B, H, L, D).unbind(dim=0)
    return q, k, v


class SelfAttention(torch.nn.Module):
    """A cosine-attention layer with the attributes of Infinity's SelfAttention
    (infinity/models/basic.py:196-246) that the fused segmented forward reads;
    random weights, learned-scale values on both sides of the clamp.  Its own
    forward is never run (the patched forward replaces it)."""

    def __init__(self, embed_dim: int, num_heads: int):
        super().__init__()
        self.num_heads, self.head_dim = num_heads, embed_dim // num_heads
        self.cos_attn, self.scale = True, 1
        self.scale_mul_1H11 = torch.nn.Parameter(
            torch.linspace(math.log(4.0), math.log(150.0), num_heads).reshape(1, num_heads, 1, 1))
        self.max_scale_mul = math.log(100)
        self.mat_qkv = torch.nn.Linear(embed_dim, 3 * embed_dim, bias=False)
        self.q_bias = torch.nn.Parameter(torch.randn(embed_dim) * 0.1)
        self.v_bias = torch.nn.Parameter(torch.randn(embed_dim) * 0.1)
        self.register_buffer("zero_k_bias", torch.zeros(embed_dim))
        self.proj = torch.nn.Linear(embed_dim, embed_dim)
        self.proj_drop = torch.nn.Identity()
        self.caching = False
        self.cached_k = self.cached_v = None

    def kv_caching(self, enable: bool):
        self.caching = enable
        self.cached_k = self.cached_v = None

    def forward(self, *args, **kwargs):  # pragma: no cover - replaced when enabled
        raise NotImplementedError("unpatched test layer")


def kept_keys_reference(inputs, kept_scales, t: int, scale: float, *, workers: int = 16):
    """fp32 oracle attention of generation step ``t`` over exactly the keys a
    policy keeps: head h attends to the rows of the prior scales
    ``kept_scales(h)`` (in that order), then to its own current rows.
    ``inputs[s]`` = ``(q, k, v)`` ``[B, H, n_s, D]`` of scale s.  Every (b, h)
    is computed (the oracle's thread pool over the pairs); returns
    ``(out [B, L, H*D], lse [B, H, L])``."""
    from oracle import segmented_attention as oattn

    q, k, v = inputs[t]
    B, H, _, D = q.shape
    pieces_k, pieces_v, starts, ends = [], [], [], []
    off = 0
    for h in range(H):
        n = 0
        for s in kept_scales(h):
            pieces_k.append(inputs[s][1][:, h])
            pieces_v.append(inputs[s][2][:, h])
            n += int(inputs[s][1].shape[2])
        starts.append(off)
        ends.append(off + n)
        off += n
    slab_k = torch.cat(pieces_k, dim=1) if pieces_k else torch.zeros((B, 0, D), dtype=k.dtype)
    slab_v = torch.cat(pieces_v, dim=1) if pieces_v else torch.zeros((B, 0, D), dtype=v.dtype)
    st = np.asarray(starts, np.int32).reshape(H, 1)
    en = np.asarray(ends, np.int32).reshape(H, 1)
    ct = np.ones(H, np.int32)
    return oattn.flat_segmented_attention(to_np(q), to_np(slab_k), to_np(slab_v), st, en, ct, to_np(k), to_np(v),
                                          scale, workers=workers)
