"""numpy restatement of the attention layer's QKV prologue (test infrastructure only).

Follows the reference layer forward under bf16 autocast
(enable_real_pruning_fast.py:2040-2072) and ``apply_rotary_emb``
(infinity/models/basic.py:97-117):

* ``qkv`` is the bf16 projection ``[B, L, 3, H, D]`` (given here as its fp32
  values); an optional fp32 bias is added to q and v;
* q and k are L2-normalized in fp32: ``x / max(||x||, eps)`` with the norm
  computed in float64 and rounded to fp32 (torch sums in fp32 in its own
  order; the product sums in yet another, so both sit within a few fp32 ulp
  of this one), then q is multiplied by ``scale_mul[h]``;
* every pair ``(x[2i], x[2i+1])`` of q and k is rotated with the table row of
  its token: ``(c*x0 - s*x1, s*x0 + c*x1)``, each product and sum rounded to
  fp32 separately (elementwise tensor ops, basic.py:110-113);
* outputs are ``[B, H, L, D]``; v is the bf16 value (plus bias, rounded to
  bf16 to nearest even); for an fp16 or fp32 projection (fp16 autocast, no
  autocast) the same in that type.

``rope_table`` restates ``precompute_rope2d_freqs_grid`` (basic.py:39-94) for
one schedule, with the angles in float64.

Pinning (tests/test_oracle_produce.py): normalized rows have unit norm times
``scale_mul``; the rotation preserves pair norms and equals multiplication of
the complex numbers ``x0 + i x1`` and ``c + i s``; position 0 of the table is
the identity; a basis vector at a known grid position comes out as the closed
form ``(cos, sin)`` of its row/column angle; inner products of rotated q and k
depend on the position difference only (mode 0); the mode-2 index rounding
matches values worked out by hand; inverse rotation recovers the input.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 (ties to even), returned as float32."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out)


def grid_angles(dim: int, max_height: int = 128, max_width: int = 128, base: float = 10000.0,
                scaling_factor: float = 1.0) -> np.ndarray:
    """Angles ``[max_height, max_width, dim // 2]`` (float64) of the 2-D grid
    (basic.py:41-52): the first ``dim // 4`` entries are row * inv_freq, the
    rest column * inv_freq, inv_freq[j] = base^(-2j / (dim // 2))."""
    half = dim // 2
    inv = 1.0 / base ** (np.arange(0, half, 2, dtype=np.float64) / half)
    rows = np.arange(max_height, dtype=np.float64) / scaling_factor
    cols = np.arange(max_width, dtype=np.float64) / scaling_factor
    ang = np.empty((max_height, max_width, half), dtype=np.float64)
    ang[:, :, : half // 2] = (rows[:, None] * inv[None, :])[:, None, :]
    ang[:, :, half // 2:] = (cols[:, None] * inv[None, :])[None, :, :]
    return ang


def star_indices(side: int, full: int) -> np.ndarray:
    """Grid rows (or columns) of a ``side``-long axis under
    rope2d_normalized_by_hw=2: ``round(i * full / side)`` (basic.py:73-76)."""
    return np.rint(np.arange(side, dtype=np.float32) * np.float32(full / side)).astype(np.int64)


def _bilinear_axis(n_out: int, n_in: int):
    """Source index pairs and weights of an align_corners=True linear resize."""
    if n_out == 1:
        pos = np.zeros(1)
    else:
        pos = np.arange(n_out) * (n_in - 1) / (n_out - 1)
    lo = np.floor(pos).astype(np.int64)
    hi = np.minimum(lo + 1, n_in - 1)
    return lo, hi, pos - lo


def rope_table(dim: int, scale_schedule, mode: int = 2, pad_to_multiplier: int = 1) -> np.ndarray:
    """``[2, T, dim // 2]`` float64 cos/sin table of one schedule.

    Mode 0 takes grid rows/columns ``[0, ph) x [0, pw)``; mode 2 the rows and
    columns of :func:`star_indices`; mode 1 resizes the cos/sin grid of the
    ``(uph, upw)`` corner (the final scale's aspect on the 128-edge grid)
    bilinearly to ``ph x pw`` with corners aligned (basic.py:59-84)."""
    ang = grid_angles(dim)
    cs = np.stack([np.cos(ang), np.sin(ang)], axis=0)
    edge = ang.shape[0]
    _, fh, fw = scale_schedule[-1]
    up = (edge, int(edge / fh * fw)) if fh >= fw else (int(edge / fw * fh), edge)
    parts = []
    for _, ph, pw in scale_schedule:
        if mode == 0:
            t = cs[:, :ph, :pw, :]
        elif mode == 2:
            t = cs[:, star_indices(ph, fh)][:, :, star_indices(pw, fw)]
        elif mode == 1:
            src = cs[:, :up[0], :up[1], :]
            r0, r1, wr = _bilinear_axis(ph, up[0])
            c0, c1, wc = _bilinear_axis(pw, up[1])
            rows = src[:, r0] * (1 - wr)[None, :, None, None] + src[:, r1] * wr[None, :, None, None]
            t = rows[:, :, c0] * (1 - wc)[None, None, :, None] + rows[:, :, c1] * wc[None, None, :, None]
        else:
            raise ValueError(f"unknown mode {mode}")
        parts.append(t.reshape(2, ph * pw, -1))
    table = np.concatenate(parts, axis=1)
    pad = table.shape[1] % max(1, pad_to_multiplier)
    if pad:
        table = np.concatenate([table, np.zeros((2, pad_to_multiplier - pad, dim // 2))], axis=1)
    return table


def normalize_rows(x: np.ndarray, eps: float = 1e-12) -> np.ndarray:
    n = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)).astype(np.float32)
    n = np.where(n < np.float32(eps), np.float32(eps), n)
    return (x / n).astype(np.float32)


def rotate_pairs(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate pairs of ``x`` ``[..., L, D]`` with ``cos``/``sin`` ``[L, D // 2]`` (fp32 ops)."""
    x0 = x[..., 0::2]
    x1 = x[..., 1::2]
    c = cos.astype(np.float32)
    s = sin.astype(np.float32)
    out = np.empty_like(x)
    out[..., 0::2] = (c * x0).astype(np.float32) - (s * x1).astype(np.float32)
    out[..., 1::2] = (s * x0).astype(np.float32) + (c * x1).astype(np.float32)
    return out


def fp16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest float16 (ties to even), returned as float32."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def produce(qkv: np.ndarray, *, scale_mul=None, table=None, start: int = 0, q_bias=None, v_bias=None,
            normalize: bool = True, eps: float = 1e-12, v_type: str = "bf16"):
    """``(q, k, v)`` ``[B, H, L, D]`` (q, k float32; v float32 holding values
    of the projection's type ``v_type``: "bf16", "fp16" or "fp32") from
    ``qkv`` ``[B, L, 3, H, D]`` float32 (values of that type); v plus
    ``v_bias`` is rounded once to that type."""
    v_round = {"bf16": bf16_round, "fp16": fp16_round, "fp32": lambda a: np.asarray(a, np.float32)}[v_type]
    qkv = np.asarray(qkv, dtype=np.float32)
    B, L, _, H, D = qkv.shape
    q = qkv[:, :, 0].copy()
    k = qkv[:, :, 1].copy()
    v = qkv[:, :, 2].copy()
    if q_bias is not None:
        q = (q + np.asarray(q_bias, np.float32).reshape(H, D)).astype(np.float32)
    if v_bias is not None:
        v = v_round((v + np.asarray(v_bias, np.float32).reshape(H, D)).astype(np.float32))
    if normalize:
        q = normalize_rows(q, eps)
        k = normalize_rows(k, eps)
    if scale_mul is not None:
        q = (q * np.asarray(scale_mul, np.float32).reshape(1, 1, H, 1)).astype(np.float32)
    q = q.transpose(0, 2, 1, 3)
    k = k.transpose(0, 2, 1, 3)
    v = v.transpose(0, 2, 1, 3)
    if table is not None:
        t = np.asarray(table, dtype=np.float32)
        cos = t[0, start:start + L]
        sin = t[1, start:start + L]
        q = rotate_pairs(np.ascontiguousarray(q), cos, sin)
        k = rotate_pairs(np.ascontiguousarray(k), cos, sin)
    return np.ascontiguousarray(q), np.ascontiguousarray(k), np.ascontiguousarray(v)
