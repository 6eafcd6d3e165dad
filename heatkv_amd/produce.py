"""QKV producer of the attention layer: normalize, scale, 2-D RoPE, permute, append.

The layer prologue of the reference forward (enable_real_pruning_fast.py:
2040-2072) under the bf16 autocast the reference generates with: the QKV
projection gives bf16 ``[B, L, 3, H, D]``; cosine attention L2-normalizes q
and k in fp32 (torch's autocast runs ``norm`` in fp32, so the quotient is
fp32), multiplies q by ``exp(min(scale_mul, max_scale_mul))`` per head, and
``apply_rotary_emb`` (infinity/models/basic.py:97-117) rotates each pair
``(2i, 2i+1)`` of q and k by the 2-D RoPE table row of its token.  q and k
come out fp32 ``[B, H, L, D]``, v bf16.  Under fp16 autocast the projection
is fp16, without autocast fp32; q and k are computed in fp32 the same way and
v keeps the projection's dtype.

:func:`qkv_produce` runs all of it in one HIP kernel (``hkv_qkv_produce``),
optionally with the fused QKV bias and with the append of the kept heads'
current rows into the slab.  :func:`rope2d_freqs_table` and
:func:`precompute_rope2d_freqs_grid` build the RoPE tables on the host like
``precompute_rope2d_freqs_grid`` (infinity/models/basic.py:39-94).
"""

from __future__ import annotations

from typing import Dict, Optional, Sequence, Tuple

import torch
import torch.nn.functional as F

from . import _lib

HEAD_DIM = 128


# ---------------------------------------------------------------- RoPE tables

def _freqs_grid_map(dim: int, max_height: int, max_width: int, base: float, scaling_factor: float):
    """cos/sin of the 2-D frequency grid ``[2, max_height, max_width, dim // 2]``
    (fp32, CPU): the first ``dim // 4`` entries of a row rotate with the row
    index, the rest with the column index (basic.py:41-54)."""
    half = dim // 2
    inv_freq = 1.0 / (base ** (torch.arange(0, half, 2, dtype=torch.int64).float() / half))
    rows = torch.arange(max_height, dtype=torch.int64).float() / scaling_factor
    cols = torch.arange(max_width, dtype=torch.int64).float() / scaling_factor
    f_rows = torch.outer(rows, inv_freq)
    f_cols = torch.outer(cols, inv_freq)
    grid = torch.cat([f_rows[:, None, :].expand(-1, max_width, -1),
                      f_cols[None, :, :].expand(max_height, -1, -1)], dim=-1)
    return torch.stack([torch.cos(grid), torch.sin(grid)], dim=0)


def _scale_rows(grid: torch.Tensor, ph: int, pw: int, mode: int, full_hw: Tuple[int, int],
                up_hw: Tuple[int, int]) -> torch.Tensor:
    """Table rows ``[2, ph * pw, dim // 2]`` of one ``ph x pw`` scale (basic.py:67-84)."""
    if mode == 0:
        rows = grid[:, :ph, :pw, :]
    elif mode == 1:
        uph, upw = up_hw
        rows = F.interpolate(grid[:, :uph, :upw, :].permute(0, 3, 1, 2), size=(ph, pw), mode="bilinear",
                             align_corners=True).permute(0, 2, 3, 1)
    elif mode == 2:
        fh, fw = full_hw
        ri = (torch.arange(ph) * (fh / ph)).round().int()
        ci = (torch.arange(pw) * (fw / pw)).round().int()
        rows = grid[:, ri[:, None].expand(ph, pw).reshape(-1), ci[None, :].expand(ph, pw).reshape(-1), :]
    else:
        raise ValueError(f"Unknown rope2d_normalized_by_hw: {mode}")
    return rows.reshape(2, ph * pw, -1)


def rope2d_freqs_table(dim: int, scale_schedule: Sequence[Sequence[int]], rope2d_normalized_by_hw: int = 2,
                       pad_to_multiplier: int = 1, max_height: int = 2048 // 16, max_width: int = 2048 // 16,
                       base: float = 10000.0, scaling_factor: float = 1.0) -> torch.Tensor:
    """RoPE table ``[2, T, dim // 2]`` (cos, sin; fp32, CPU) of one 1M-pixel scale
    schedule of ``(t, h, w)`` entries: the scales' rows back to back, zero rows up
    to a multiple of ``pad_to_multiplier`` (basic.py:56-88)."""
    grid = _freqs_grid_map(dim, max_height, max_width, base, scaling_factor)
    _, fh, fw = scale_schedule[-1]
    edge = grid.shape[1]
    if fh >= fw:
        up = (edge, int(edge / fh * fw))
    else:
        up = (int(edge / fw * fh), edge)
    table = torch.cat([_scale_rows(grid, int(ph), int(pw), int(rope2d_normalized_by_hw), (fh, fw), up)
                       for (_, ph, pw) in scale_schedule], dim=1)
    pad = table.shape[1] % max(1, int(pad_to_multiplier))
    if pad:
        table = torch.cat([table, torch.zeros(2, int(pad_to_multiplier) - pad, dim // 2)], dim=1)
    return table


def schedule_key(scale_schedule: Sequence[Sequence[int]]) -> str:
    """Dictionary key of a schedule in the reference's grid dict (basic.py:90-93, 107)."""
    return str(tuple((1, int(h), int(w)) for _, h, w in scale_schedule))


def precompute_rope2d_freqs_grid(dim: int, dynamic_resolution_h_w: Dict, rope2d_normalized_by_hw: int,
                                 pad_to_multiplier: int = 1, max_height: int = 2048 // 16,
                                 max_width: int = 2048 // 16, base: float = 10000.0, device=None,
                                 scaling_factor: float = 1.0) -> Dict[str, torch.Tensor]:
    """The reference's grid dict (basic.py:39-94): for every aspect ratio, the
    table of its ``'1M'`` schedule as ``[2, 1, 1, 1, T, dim // 2]``, registered
    under the key of every pixel budget's schedule of that ratio."""
    out = {}
    for h_div_w, budgets in dynamic_resolution_h_w.items():
        table = rope2d_freqs_table(dim, budgets["1M"]["scales"], rope2d_normalized_by_hw, pad_to_multiplier,
                                   max_height, max_width, base, scaling_factor)
        grid = table[:, None, None, None]
        if device is not None:
            grid = grid.to(device)
        for pn in budgets:
            out[schedule_key(budgets[pn]["scales"])] = grid
    return out


def rope_start(scale_schedule: Sequence[Sequence[int]], scale_ind: int) -> int:
    """Table row of the first token of scale ``scale_ind`` (basic.py:104-106)."""
    return int(sum(int(t) * int(h) * int(w) for t, h, w in scale_schedule[:scale_ind]))


def rope_table_for(rope2d_freqs_grid: Dict, scale_schedule: Sequence[Sequence[int]], device) -> torch.Tensor:
    """Device ``[2, T, dim // 2]`` view of the schedule's table; like the
    reference (basic.py:107), the device copy replaces the dict entry."""
    key = schedule_key(scale_schedule)
    grid = rope2d_freqs_grid[key]
    if grid.device != torch.device(device):
        grid = grid.to(device)
        rope2d_freqs_grid[key] = grid
    return grid.reshape(2, grid.shape[-2], grid.shape[-1])


def scale_mul_of(layer) -> torch.Tensor:
    """``exp(min(scale_mul_1H11, max_scale_mul))`` per head, fp32 ``[H]``
    (enable_real_pruning_fast.py:2052-2057)."""
    return layer.scale_mul_1H11.reshape(-1).float().clamp_max(layer.max_scale_mul).exp()


# ---------------------------------------------------------------- producer

def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _vector(t: Optional[torch.Tensor], n: int, name: str, device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    t = t.reshape(-1)
    if t.numel() != n:
        raise ValueError(f"{name} must have {n} elements (got {t.numel()})")
    return t.to(device=device, dtype=torch.float32).contiguous()


def qkv_produce(
    qkv: torch.Tensor,
    num_heads: int,
    *,
    scale_mul: Optional[torch.Tensor] = None,
    rope_table: Optional[torch.Tensor] = None,
    rope_start_row: int = 0,
    q_bias: Optional[torch.Tensor] = None,
    v_bias: Optional[torch.Tensor] = None,
    normalize: bool = True,
    eps: float = 1e-12,
    qk_dtype: torch.dtype = torch.float32,
    append: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
    k_split_rows: bool = False,
):
    """Attention-ready ``q, k, v`` ``[B, H, L, D]`` of one scale from the QKV
    projection output ``qkv`` (``[B, L, 3 * H * D]`` or ``[B, L, 3, H, D]``;
    bf16 under the reference's bf16 autocast, fp16 under fp16 autocast, fp32
    without autocast).

    * ``scale_mul``: per-head multiplier of q (``[H]``), e.g. :func:`scale_mul_of`;
    * ``rope_table``: ``[2, T, D // 2]`` fp32 device table (cos, sin), rows
      ``rope_start_row ...`` used for the scale's tokens; None skips RoPE;
    * ``q_bias``, ``v_bias``: ``[H * D]`` biases added in fp32 to the
      projection (leave None when the projection applied them);
    * ``append``: ``(slab_k, slab_v, offsets)`` -- slab ``[B, capacity, D]`` of
      k's / v's dtype and int32 ``[H]`` device offsets (-1 = not appended):
      rows of head h also go to ``slab[b, offsets[h] + l]``.

    q, k are ``qk_dtype``: fp32 like the reference, fp16 (the 11-bit
    significand of the TF32 products the reference's attention takes of fp32
    q/k, for values within fp16's range, e.g. cosine attention's), or bf16;
    v keeps the projection's dtype and values.  ``k_split_rows`` (fp32 only): k's rows (and the appended slab
    rows) hold the split rows of the fp32 values instead (the 128 bf16 high
    parts ``bf16(x)``, then the 128 low parts ``bf16(x - hi)``, 512 bytes like
    an fp32 row; the tensor keeps dtype float32 so byte copies of it stay
    valid), the K format the attention's split-row kernel reads: calls with
    ``k_split_rows=True`` then skip their own split.
    """
    if not qkv.is_cuda:
        raise RuntimeError("qkv_produce runs on the GPU only (HIP kernel); got a CPU tensor")
    if qkv.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise RuntimeError(f"qkv_produce takes a bfloat16, float16 or float32 QKV projection; got {qkv.dtype}")
    H = int(num_heads)
    D = HEAD_DIM
    if qkv.dim() == 5:
        B, L = int(qkv.shape[0]), int(qkv.shape[1])
        if tuple(qkv.shape[2:]) != (3, H, D):
            raise ValueError(f"qkv must be [B, L, 3, {H}, {D}] (got {tuple(qkv.shape)})")
    elif qkv.dim() == 3:
        B, L = int(qkv.shape[0]), int(qkv.shape[1])
        if int(qkv.shape[2]) != 3 * H * D:
            raise ValueError(f"qkv last dim must be 3 * heads * {D} = {3 * H * D} (got {qkv.shape[2]})")
    else:
        raise ValueError("qkv must be [B, L, 3*H*D] or [B, L, 3, H, D]")
    if qk_dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise ValueError("qk_dtype must be torch.float32, torch.float16 or torch.bfloat16")
    if k_split_rows and qk_dtype != torch.float32:
        raise ValueError("k_split_rows needs qk_dtype=torch.float32")
    qkv = qkv.contiguous()
    dev = qkv.device
    _lib.require_device(dev)
    q = torch.empty((B, H, L, D), device=dev, dtype=qk_dtype)
    k = torch.empty((B, H, L, D), device=dev, dtype=qk_dtype)
    v = torch.empty((B, H, L, D), device=dev, dtype=qkv.dtype)
    sm = _vector(scale_mul, H, "scale_mul", dev)
    qb = _vector(q_bias, H * D, "q_bias", dev)
    vb = _vector(v_bias, H * D, "v_bias", dev)
    rope_rows = 0
    if rope_table is not None:
        if rope_table.dim() != 3 or rope_table.shape[0] != 2 or rope_table.shape[2] != D // 2:
            raise ValueError(f"rope_table must be [2, T, {D // 2}] (got {tuple(rope_table.shape)})")
        rope_table = rope_table.to(device=dev, dtype=torch.float32).contiguous()
        rope_rows = int(rope_table.shape[1])
    slab_k = slab_v = offsets = None
    capacity = 0
    if append is not None:
        slab_k, slab_v, offsets = append
        if slab_k.dtype != qk_dtype or slab_v.dtype != qkv.dtype:
            raise ValueError("append slabs must have k's and v's dtypes")
        if (slab_k.dim() != 3 or tuple(slab_k.shape) != tuple(slab_v.shape) or int(slab_k.shape[0]) != B
                or int(slab_k.shape[2]) != D or not slab_k.is_contiguous() or not slab_v.is_contiguous()):
            raise ValueError(f"append slabs must be contiguous [{B}, capacity, {D}]")
        if offsets.dtype != torch.int32 or offsets.numel() != H or offsets.device != dev:
            raise ValueError(f"append offsets must be an int32 device tensor of {H} entries")
        capacity = int(slab_k.shape[1])
    if B == 0 or L == 0:
        return q, k, v
    code = _lib.load().hkv_qkv_produce(
        qkv.data_ptr(), 3 * H * D, _ptr(qb), _ptr(vb), _ptr(sm), _ptr(rope_table), rope_rows,
        int(rope_start_row), q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(slab_k), _ptr(slab_v),
        _ptr(offsets), capacity, B, H, L, D, _lib.dtype_code(qkv.dtype), _lib.dtype_code(qk_dtype),
        _lib.DTYPE_SPLIT_ROWS if k_split_rows else _lib.dtype_code(qk_dtype), _lib.dtype_code(qkv.dtype),
        1 if normalize else 0,
        float(eps), _lib.stream_handle(dev))
    _lib.check(code)
    return q, k, v
