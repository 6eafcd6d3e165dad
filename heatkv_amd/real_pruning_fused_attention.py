"""Operator surface of the fused segmented path, on gfx950 HIP kernels.

Drop-in for the reference module real_pruning_fused_attention.py: same
function names, keyword-only signatures, argument meaning, validation order
and error types/messages.  The work runs in libheatkv.so (C ABI in
include/heatkv.h) on the current HIP stream; nothing here synchronises.

Differences from the reference, all deliberate:

* ``fused_real_pruning_flat_segmented_attention(..., return_lse=True)``
  additionally returns the fp32 softmax log-sum-exp ``[B, H, L]``; the
  default return value is unchanged.
* There is no CPU path.  The reference answers ``allow_cpu_fallback=True``
  with a pure-torch loop (real_pruning_fused_attention.py:509-521); this
  module raises ``RuntimeError`` for non-GPU tensors either way, so a result
  is always the HIP kernel's.
* Tile-shape knobs (``REAL_PRUNING_FUSED_BLOCK_M``/``_BLOCK_N``/
  ``_NUM_WARPS``/``_NUM_STAGES``) are read and validated like the
  reference's but the kernel's tile shape is fixed by its MFMA layout.
* The dot-mode knobs (``REAL_PRUNING_FUSED_QK_DOT_MODE`` bf16 / tf32 / fp32,
  ``REAL_PRUNING_FUSED_VALUE_DOT_MODE`` bf16 / fp32) are validated like the
  reference's and passed to the kernels, which meet or exceed each mode's
  precision on 16-bit MFMAs with fp32 accumulation: 16-bit q/k products are
  exact in every mode; fp32 q and k are split into 2 bf16 pieces (~16
  significand bits, where the reference's bf16 / tf32 modes take a TF32
  product) or, in the fp32 mode, 3 pieces (fp32's 24 bits).  P is rounded to
  V's 16-bit type in the default value mode (fp32 V: P and V in 2 pieces,
  where the reference takes a TF32 product); the fp32 value mode splits P in
  3 pieces and V in as many as its type needs.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib


def _positive_int_env(name: str, default: int) -> int:
    """Integer env knob, falling back to ``default`` (real_pruning_fused_attention.py:274-283)."""
    raw = _lib.env_get(name)
    if raw is None:
        return int(default)
    try:
        value = int(raw)
    except ValueError:
        return int(default)
    return value if value > 0 else int(default)


def _fused_value_dot_mode_id() -> int:
    """PV dot mode knob (real_pruning_fused_attention.py:286-295)."""
    mode = _lib.env_get("REAL_PRUNING_FUSED_VALUE_DOT_MODE", "bf16").strip().lower()
    if mode in {"bf16", "flash"}:
        return 0
    if mode in {"fp32", "ieee", "mixed", "fp32_probs"}:
        return 2
    raise ValueError("REAL_PRUNING_FUSED_VALUE_DOT_MODE must be one of: bf16, fp32")


def _fused_qk_dot_mode_id() -> int:
    """QK dot mode knob (real_pruning_fused_attention.py:298-308)."""
    mode = _lib.env_get("REAL_PRUNING_FUSED_QK_DOT_MODE", "bf16").strip().lower()
    if mode in {"bf16", "tensorcore"}:
        return 0
    if mode in {"tf32", "fp32_tf32"}:
        return 1
    if mode in {"fp32", "ieee"}:
        return 2
    raise ValueError("REAL_PRUNING_FUSED_QK_DOT_MODE must be one of: bf16, tf32, fp32")


PLAN_INTS = 8


def segmented_attention_plan(segment_starts, segment_ends, segment_counts, *, batch_size: int,
                             current_len: int, capacity: int, device=None, slots: Optional[int] = None,
                             queries_per_item: int = 128):
    """Work plan of :func:`fused_real_pruning_flat_segmented_attention` for
    host copies of its offset tables (``[H, S]``, ``[H]``; torch CPU tensors
    or numpy arrays), ``batch_size``, ``current_len`` and slab ``capacity``:
    an int32 tensor ``[units, 8]`` on ``device`` (host when None) to pass as
    ``work_plan`` with every call on those tables.  ``queries_per_item`` is
    the kernel's (:func:`attention_queries_per_item`: 128, or 256 for fp32
    q/k with 16-bit v); the tensor carries it as ``hkv_queries_per_item``
    and the batch size and length as ``hkv_plan_shape``, and the operator
    checks both (a copy made with ``clone()`` / ``to()`` loses them and is
    refused).  Built on the host by
    ``hkv_segmented_attention_plan``; ``slots`` is the kernel's resident
    workgroups (:func:`attention_item_shape`), by default 2 per CU of the
    device for 128-query items (the 16-bit kernel) and 1 per CU for 256.
    No counterpart in the reference, whose Triton grid walks the tables
    directly."""
    import numpy as np

    def host(t):
        a = t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
        return np.ascontiguousarray(a, dtype=np.int32)

    st, en, ct = host(segment_starts), host(segment_ends), host(segment_counts)
    if st.ndim != 2 or st.shape != en.shape or ct.shape != (st.shape[0],):
        raise ValueError("segment tables must be [H, S], [H, S] and [H]")
    lib = _lib.load()
    if slots is None:
        if device is None:
            raise ValueError("segmented_attention_plan needs a device or slots")
        dev = torch.device(device)
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        slots = int(lib.hkv_segmented_attention_slots(idx))
        if slots < 0:
            _lib.check(slots)
        slots = slots * 128 // int(queries_per_item)  # one 256-query workgroup per CU
    H, S = st.shape
    args = (st.ctypes.data, en.ctypes.data, ct.ctypes.data, H, S, int(capacity), int(batch_size),
            int(current_len), int(queries_per_item), int(slots))
    n = int(lib.hkv_segmented_attention_plan(*args, None, 0))
    if n < 0:
        _lib.check(n)
    plan = np.zeros((max(n, 1), PLAN_INTS), dtype=np.int32)
    n = int(lib.hkv_segmented_attention_plan(*args, plan.ctypes.data, plan.shape[0]))
    if n < 0:
        _lib.check(n)
    out = torch.from_numpy(plan[:n].copy())
    if device is not None:
        out = out.to(device)
    out.hkv_queries_per_item = int(queries_per_item)
    out.hkv_plan_shape = (int(batch_size), int(current_len))
    return out


def _split_rows_path(q_dtype, k_dtype, v_dtype, qk_mode: int, value_mode: int) -> bool:
    """fp32 q/k with 16-bit v at dot modes other than fp32 run the split-row
    kernel: K is first written as split rows (hkv_split_rows).  HKV_ATTN_SPLIT_ROWS=0
    keeps them on the register-staged kernel (for comparisons)."""
    if _lib.env_get("HKV_ATTN_SPLIT_ROWS", "1").strip().lower() in {"0", "false", "no", "off"}:
        return False
    return (q_dtype == torch.float32 and k_dtype == torch.float32 and v_dtype in (torch.float16, torch.bfloat16)
            and qk_mode != 2 and value_mode != 2)


def split_rows_k_format(q_dtype, k_dtype, v_dtype) -> bool:
    """Whether fp32 K for these dtypes at the current dot-mode knobs goes to
    the split-row kernel, i.e. whether a producer may write K as split rows
    (``qkv_produce(..., k_split_rows=True)``) for calls with
    ``k_split_rows=True``."""
    return _split_rows_path(q_dtype, k_dtype, v_dtype, _fused_qk_dot_mode_id(), _fused_value_dot_mode_id())


def _check_split_rows_k(q_dtype, k_dtype, v_dtype, qk_mode: int, value_mode: int) -> None:
    if not (q_dtype == torch.float32 and k_dtype == torch.float32 and v_dtype in (torch.float16, torch.bfloat16)):
        raise ValueError("k_split_rows takes float32 q, float32-typed K holding split rows and 16-bit v")
    if qk_mode == 2 or value_mode == 2:
        raise ValueError("k_split_rows: split K rows feed the split-row kernel, which runs the default and "
                         "tf32 dot modes only (REAL_PRUNING_FUSED_QK_DOT_MODE / VALUE_DOT_MODE = fp32 need "
                         "float32 K)")


def _kernel_qk_dtypes(q_dtype, k_dtype, qk_mode: int, k_split_rows: bool):
    """q/k dtypes the kernels see: q and k of different dtypes (not split K
    rows) run widened to fp32 under the tf32 and fp32 QK modes
    (_promote_mixed_qk; the default mode refuses them)."""
    if q_dtype != k_dtype and not k_split_rows and qk_mode != 0:
        return torch.float32, torch.float32
    return q_dtype, k_dtype


_ITEM_SHAPES: dict = {}


def attention_item_shape(q_dtype, k_dtype, v_dtype, *, k_split_rows: bool = False, device=None):
    """``(queries_per_item, slots)`` of the kernel that
    :func:`fused_real_pruning_flat_segmented_attention` runs for these dtypes
    at the current dot-mode knobs on ``device`` (the current CUDA device when
    None), as the library reports them (``hkv_segmented_attention_item_shape``):
    the ``queries_per_item`` and ``slots`` of :func:`segmented_attention_plan`.
    Items are 128 queries, or 256 for the 8-wave form of the split-row
    kernel; slots are the resident workgroups of that kernel (2 per CU for
    the 16-bit kernel and the staged kernel's plain modes, 1 per CU for the
    split-row kernel and the staged kernel's split modes).  slots is None
    for a device that is not a GPU (no kernel runs there)."""
    dev = torch.device("cuda") if device is None else torch.device(device)
    if dev.type != "cuda":
        return (attention_queries_per_item(q_dtype, k_dtype, v_dtype, k_split_rows=k_split_rows), None)
    qk_mode, value_mode = _fused_qk_dot_mode_id(), _fused_value_dot_mode_id()
    qd, kd = _kernel_qk_dtypes(q_dtype, k_dtype, qk_mode, k_split_rows)
    split = k_split_rows or _split_rows_path(qd, kd, v_dtype, qk_mode, value_mode)
    codes = (_lib.dtype_code(qd), _lib.DTYPE_SPLIT_ROWS if split else _lib.dtype_code(kd), _lib.dtype_code(v_dtype))
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (codes, qk_mode, value_mode, idx)
    hit = _ITEM_SHAPES.get(key)
    if hit is None:
        slots = ctypes.c_int32(0)
        n = int(_lib.load().hkv_segmented_attention_item_shape(*codes, 1, qk_mode, value_mode, idx,
                                                               ctypes.byref(slots)))
        _lib.check(min(n, 0))
        hit = _ITEM_SHAPES[key] = (n, int(slots.value))
    return hit


def attention_queries_per_item(q_dtype, k_dtype, v_dtype, *, k_split_rows: bool = False) -> int:
    """Queries per work item of the kernel that :func:`fused_real_pruning_flat_segmented_attention`
    runs for these dtypes at the current dot-mode knobs (the ``queries_per_item``
    of :func:`segmented_attention_plan`), as the library reports it
    (``hkv_segmented_attention_item_shape``): 128, or 256 for the 8-wave form
    of the split-row kernel."""
    qk_mode, value_mode = _fused_qk_dot_mode_id(), _fused_value_dot_mode_id()
    qd, kd = _kernel_qk_dtypes(q_dtype, k_dtype, qk_mode, k_split_rows)
    if not (k_split_rows or _split_rows_path(qd, kd, v_dtype, qk_mode, value_mode)):
        return 128
    n = int(_lib.load().hkv_segmented_attention_item_shape(
        _lib.dtype_code(qd), _lib.DTYPE_SPLIT_ROWS, _lib.dtype_code(v_dtype), 1, qk_mode, value_mode, 0, None))
    _lib.check(min(n, 0))
    return n


def attention_fuses_append(q_dtype, k_dtype, v_dtype, *, k_split_rows: bool = False) -> bool:
    """Whether :func:`fused_real_pruning_flat_segmented_attention` takes
    ``append_offsets`` for these dtypes at the current dot-mode knobs: every
    path but the one that splits fp32 K itself (its slab K is a split copy)
    and q/k of different dtypes with 16-bit k (widened to fp32 for the call);
    K already in split rows (``k_split_rows``) takes it."""
    if k_split_rows:
        return True
    qk_mode, value_mode = _fused_qk_dot_mode_id(), _fused_value_dot_mode_id()
    qd, kd = _kernel_qk_dtypes(q_dtype, k_dtype, qk_mode, False)
    if kd != k_dtype:
        return False
    return not _split_rows_path(qd, kd, v_dtype, qk_mode, value_mode)


def _split_rows(t: torch.Tensor, stream) -> torch.Tensor:
    """fp32 ``[..., 128]`` rows as split rows ``[..., 256]`` bf16 (128 high
    parts, then 128 low parts), by the HIP kernel ``hkv_split_rows``."""
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    out = torch.empty(tuple(t.shape[:-1]) + (2 * t.shape[-1],), device=t.device, dtype=torch.bfloat16)
    rows = t.numel() // t.shape[-1]
    if rows > 0:
        _lib.check(_lib.load().hkv_split_rows(t.data_ptr(), out.data_ptr(), rows, stream.cuda_stream))
    return out


def concat_kv(old_k: torch.Tensor, new_k: torch.Tensor, old_v: torch.Tensor, new_v: torch.Tensor):
    """``(torch.cat((old_k, new_k), dim=2), torch.cat((old_v, new_v), dim=2))``
    for ``[B, H, T, D]`` K/V, as one HIP launch (``hkv_concat_kv``): the
    dense-prefix growth of the segmented cache
    (enable_real_pruning_fast.py:1972-2038 concatenates K and V separately).
    No counterpart in the reference module."""
    for a, b, what in ((old_k, new_k, "K"), (old_v, new_v, "V")):
        if a.ndim != 4 or b.ndim != 4 or a.shape[:2] != b.shape[:2] or a.shape[3] != b.shape[3]:
            raise ValueError(f"concat_kv: {what} tensors must be [B, H, T, D] with equal B, H, D")
        if a.dtype != b.dtype or a.device != b.device:
            raise ValueError(f"concat_kv: {what} tensors must share dtype and device")
    if old_k.shape[:3] != old_v.shape[:3] or new_k.shape[:3] != new_v.shape[:3]:
        raise ValueError("concat_kv: K and V must have the same [B, H, T]")
    if old_k.device.type != "cuda" or old_v.device != old_k.device:
        raise RuntimeError("concat_kv requires CUDA tensors")
    old_k, new_k, old_v, new_v = (t.contiguous() for t in (old_k, new_k, old_v, new_v))
    B, H, T, Dk = old_k.shape
    n = new_k.shape[2]
    Dv = old_v.shape[3]
    out_k = torch.empty((B, H, T + n, Dk), dtype=old_k.dtype, device=old_k.device)
    out_v = torch.empty((B, H, T + n, Dv), dtype=old_v.dtype, device=old_v.device)
    code = _lib.load().hkv_concat_kv(
        old_k.data_ptr(), new_k.data_ptr(), old_v.data_ptr(), new_v.data_ptr(), out_k.data_ptr(), out_v.data_ptr(),
        B * H, T, n, Dk * old_k.element_size(), Dv * old_v.element_size(), _lib.stream_handle(old_k.device))
    _lib.check(code)
    return out_k, out_v


def pack_flat_segments_kv(
    *,
    dst_k: torch.Tensor,
    dst_v: torch.Tensor,
    src_k: torch.Tensor,
    src_v: torch.Tensor,
    dst_starts: torch.Tensor,
    src_starts: torch.Tensor,
    lengths: torch.Tensor,
    max_length: Optional[int] = None,
    block_t: int = 32,
    _bind: Optional[list] = None,
):
    """Copy K/V row segments into the slab in place; returns ``(dst_k, dst_v)``.

    Item ``i`` copies ``lengths[i]`` rows from ``src[:, src_starts[i]:]`` to
    ``dst[:, dst_starts[i]:]`` for K and V.  Mirrors pack_flat_segments_kv
    (real_pruning_fused_attention.py:365-441); the copy is the HIP kernel
    ``hkv_pack_segments``.  ``_bind`` (internal): a list that receives what
    :class:`BoundPack` needs to repeat this launch.
    """
    for name, tensor in (("dst_k", dst_k), ("dst_v", dst_v), ("src_k", src_k), ("src_v", src_v)):
        if tensor.ndim != 3:
            raise ValueError(f"pack_flat_segments_kv expects {name} shaped [B, S, D]")
    if dst_k.shape != dst_v.shape:
        raise ValueError("pack_flat_segments_kv requires matching K/V destination shapes")
    if src_k.shape != src_v.shape:
        raise ValueError("pack_flat_segments_kv requires matching K/V source shapes")
    if dst_k.shape[0] != src_k.shape[0] or dst_k.shape[2] != src_k.shape[2]:
        raise ValueError("pack_flat_segments_kv requires matching batch and head_dim")
    if not all(t.is_cuda for t in (dst_k, dst_v, src_k, src_v)):
        raise RuntimeError("pack_flat_segments_kv requires CUDA tensors")
    _lib.load()
    if dst_starts.numel() == 0:
        return dst_k, dst_v
    if (
        dst_starts.device != dst_k.device
        or src_starts.device != dst_k.device
        or lengths.device != dst_k.device
    ):
        raise ValueError("pack segment metadata tensors must be on the destination device")
    if dst_starts.numel() != src_starts.numel() or dst_starts.numel() != lengths.numel():
        raise ValueError("pack segment metadata tensors must have matching lengths")
    if not dst_k.is_contiguous() or not dst_v.is_contiguous():
        raise ValueError("pack_flat_segments_kv requires contiguous destination tensors")
    if not src_k.is_contiguous():
        src_k = src_k.contiguous()
    if not src_v.is_contiguous():
        src_v = src_v.contiguous()
    head_dim = int(dst_k.shape[2])
    if head_dim > 128:
        raise RuntimeError("pack_flat_segments_kv currently supports head_dim <= 128")
    if src_k.dtype != dst_k.dtype or src_v.dtype != dst_v.dtype:
        raise ValueError("pack_flat_segments_kv requires matching source/destination dtypes")
    max_len = int(max_length) if max_length is not None else int(lengths.max().item())
    if max_len <= 0:
        return dst_k, dst_v
    block_t = int(block_t)
    if block_t <= 0:
        raise ValueError("block_t must be positive")
    row_limit = -(-max_len // block_t) * block_t
    _lib.require_device(dst_k.device)
    meta = [t if t.dtype == torch.int64 else t.to(torch.int64) for t in (dst_starts, src_starts, lengths)]
    meta = [t.contiguous() for t in meta]
    n_items = int(meta[0].numel())
    args = [
        src_k.data_ptr(), src_v.data_ptr(), dst_k.data_ptr(), dst_v.data_ptr(),
        int(src_k.stride(0)), int(dst_k.stride(0)),
        int(src_k.shape[1]), int(dst_k.shape[1]),
        int(dst_k.shape[0]), head_dim,
        int(dst_k.element_size()), int(dst_v.element_size()),
        meta[0].data_ptr(), meta[1].data_ptr(), meta[2].data_ptr(),
        n_items, min(row_limit, 2**31 - 1),
        _lib.stream_handle(dst_k.device),
    ]
    fn = _lib.load().hkv_pack_segments
    _lib.check(fn(*args))
    if _bind is not None:
        _bind.append((fn, args, meta))
    return dst_k, dst_v


def _promote_mixed_qk(q, persisted_k, current_k, qk_mode: int, append_offsets):
    """q and k of different dtypes: the reference's fp32-class QK modes cast
    both to fp32 before the product (real_pruning_fused_attention.py:143-153),
    so here the 16-bit side is widened to fp32 (exactly) and the call runs the
    fp32 q/k kernels.  The default mode's dot takes one operand type, so the
    reference's Triton compile fails there; this raises instead."""
    if qk_mode == 0:
        raise RuntimeError(
            "real_scale_fused_segmented requires q and k of one dtype under "
            "REAL_PRUNING_FUSED_QK_DOT_MODE=bf16; tf32 or fp32 take q and k of different dtypes")
    if q.dtype != torch.float32:
        q = q.float()
    if current_k.dtype != torch.float32:
        if append_offsets is not None:
            raise ValueError("append_offsets: k is widened to fp32 for an fp32 q, so the call cannot "
                             "append into the 16-bit slab; append after the call")
        current_k = current_k.float()
        persisted_k = persisted_k.float()
    return q, persisted_k, current_k


def fused_real_pruning_flat_segmented_attention(
    *,
    q: torch.Tensor,
    persisted_k: Optional[torch.Tensor],
    persisted_v: Optional[torch.Tensor],
    segment_starts: torch.Tensor,
    segment_ends: torch.Tensor,
    segment_counts: torch.Tensor,
    current_k: torch.Tensor,
    current_v: torch.Tensor,
    softmax_scale: float,
    allow_cpu_fallback: bool = False,
    softmax_mode: str = "exp",
    return_lse: bool = False,
    out_dtype: Optional[torch.dtype] = None,
    work_plan: Optional[torch.Tensor] = None,
    append_offsets: Optional[torch.Tensor] = None,
    k_split_rows: bool = False,
    append_also: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None,
    _bind: Optional[list] = None,
):
    """Attention of the current scale over the flat slab segments plus itself.

    ``persisted_k/v`` are ``[B, capacity, D]``; ``segment_starts/ends [H, S]``
    are row offsets into that slab grouped per head, ``segment_counts [H]``.
    Returns ``[B, L, H*D]`` in q's dtype, or ``out_dtype`` (an extension: the
    fp32 result rounded once to bf16 / fp16, what casting q's-dtype output
    would give), and ``lse [B, H, L]`` fp32 when ``return_lse``.  ``work_plan``
    (an extension): the plan :func:`segmented_attention_plan` built for these
    same tables, batch size and current length, on q's device; the kernel then
    skips ordering its work itself.  ``append_offsets`` (an extension): int32
    ``[H]`` on q's device; the same launch then also writes current rows
    ``[0, L)`` of (b, h) to slab rows ``[off, off + L)`` of batch row b, off =
    ``append_offsets[h]`` (-1: not written) -- the append that follows the
    attention in the reference's cache update, for rows outside every segment
    this call reads (:func:`attention_fuses_append` says which inputs take it).
    ``k_split_rows`` (an extension): q is fp32 and ``current_k`` /
    ``persisted_k`` are float32-typed tensors whose rows hold split rows of
    fp32 K (:func:`qkv_produce` with ``k_split_rows=True``), so the call skips
    its own split of K; same results as passing the fp32 K.  ``append_also``
    (an extension, with ``append_offsets``): ``(slab2_k, slab2_v, offsets2)``,
    a second destination of the same rows -- ``[B, capacity2, D]`` tensors of
    the slab's dtypes and int32 ``offsets2 [H]`` (-1: not written) -- written
    by the same copy (a dense-prefix step that also fills the slab of the
    first pruned target).  ``_bind``
    (internal): a list that receives what :class:`BoundSegmentedAttention`
    needs to repeat this launch.
    Mirrors fused_real_pruning_flat_segmented_attention
    (real_pruning_fused_attention.py:445-591); the work is the HIP kernel
    ``hkv_segmented_attention``.
    """
    if q.ndim != 4 or current_k.ndim != 4 or current_v.ndim != 4:
        raise ValueError("q, current_k, and current_v must have shape [B, H, L, D]")
    if q.shape != current_k.shape or q.shape != current_v.shape:
        raise ValueError("q, current_k, and current_v must have identical [B, H, L, D] shapes")
    if q.device != current_k.device or q.device != current_v.device:
        raise ValueError("q, current_k, and current_v must be on the same device")
    if persisted_k is None or persisted_v is None:
        batch_size = current_k.shape[0]
        head_dim = current_k.shape[3]
        persisted_k = current_k.new_empty((batch_size, 0, head_dim))
        persisted_v = current_v.new_empty((batch_size, 0, head_dim))
    if persisted_k.ndim != 3 or persisted_v.ndim != 3:
        raise ValueError("persisted_k and persisted_v must have shape [B, S, D]")
    if persisted_k.shape != persisted_v.shape:
        raise ValueError("persisted_k and persisted_v must have identical shapes")
    if persisted_k.shape[0] != q.shape[0]:
        raise ValueError("persisted K/V batch dimension must match q")
    if persisted_k.shape[2] != q.shape[3]:
        raise ValueError("persisted K/V head_dim must match q")
    if persisted_k.device != q.device or persisted_v.device != q.device:
        raise ValueError("persisted K/V must be on the same device as q")
    if persisted_k.dtype != current_k.dtype:
        raise ValueError("persisted_k dtype must match current_k")
    if persisted_v.dtype != current_v.dtype:
        raise ValueError("persisted_v dtype must match current_v")

    batch_size, num_heads, current_len, head_dim = q.shape
    if segment_starts.shape != segment_ends.shape:
        raise ValueError("segment_starts and segment_ends must have identical shapes")
    if segment_starts.ndim != 2 or segment_starts.shape[0] != num_heads:
        raise ValueError("segment_starts must have shape [H, S]")
    if tuple(segment_counts.shape) != (num_heads,):
        raise ValueError("segment_counts must have shape [H]")
    if (
        segment_starts.device != q.device
        or segment_ends.device != q.device
        or segment_counts.device != q.device
    ):
        raise ValueError("segment metadata must be on the same device as q")
    if softmax_mode not in {"exp", "exp2"}:
        raise ValueError(f"unsupported softmax_mode {softmax_mode!r}")

    if q.device.type != "cuda":
        # No host implementation ships with this library (see module docstring).
        raise RuntimeError("real_scale_fused_segmented requires CUDA tensors")

    _lib.load()
    if head_dim != 128:
        raise RuntimeError("real_scale_fused_segmented v1 only supports head_dim=128")
    if current_len <= 0:
        raise RuntimeError("real_scale_fused_segmented requires current_len > 0")
    for what, t in (("q", q), ("k", current_k), ("v", current_v)):
        if t.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise RuntimeError(
                f"real_scale_fused_segmented supports only float16, bfloat16, or float32 {what} tensors"
            )
    if out_dtype is None:
        out_dtype = q.dtype
    if out_dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("out_dtype must be torch.float16, torch.bfloat16 or torch.float32")

    # Knobs are validated like the reference's (bad values raise ValueError).
    for knob, default in (("REAL_PRUNING_FUSED_BLOCK_M", 64), ("REAL_PRUNING_FUSED_BLOCK_N", 64),
                          ("REAL_PRUNING_FUSED_NUM_WARPS", 4), ("REAL_PRUNING_FUSED_NUM_STAGES", 3)):
        _positive_int_env(knob, default)
    qk_mode = _fused_qk_dot_mode_id()
    value_mode = _fused_value_dot_mode_id()
    promoted = q.dtype != current_k.dtype and not k_split_rows
    if promoted:
        q, persisted_k, current_k = _promote_mixed_qk(q, persisted_k, current_k, qk_mode, append_offsets)

    _lib.require_device(q.device)
    if append_offsets is not None and not (persisted_k.is_contiguous() and persisted_v.is_contiguous()):
        raise ValueError("append_offsets: the slab must be contiguous (the append writes it in place)")
    q = q.contiguous()
    persisted_k = persisted_k.contiguous()
    persisted_v = persisted_v.contiguous()
    segment_starts = segment_starts.to(dtype=torch.int32).contiguous()
    segment_ends = segment_ends.to(dtype=torch.int32).contiguous()
    segment_counts = segment_counts.to(dtype=torch.int32).contiguous()
    current_k = current_k.contiguous()
    current_v = current_v.contiguous()

    output = torch.empty((batch_size, current_len, num_heads * head_dim), device=q.device, dtype=out_dtype)
    lse = (
        torch.empty((batch_size, num_heads, current_len), device=q.device, dtype=torch.float32)
        if return_lse
        else None
    )
    if k_split_rows:
        _check_split_rows_k(q.dtype, current_k.dtype, current_v.dtype, qk_mode, value_mode)
    split = k_split_rows or _split_rows_path(q.dtype, current_k.dtype, current_v.dtype, qk_mode, value_mode)
    if work_plan is not None:
        if (work_plan.dtype != torch.int32 or work_plan.ndim != 2 or work_plan.shape[1] != PLAN_INTS
                or not work_plan.is_contiguous()):
            raise ValueError(f"work_plan must be a contiguous int32 tensor [units, {PLAN_INTS}]")
        if work_plan.device != q.device:
            raise ValueError("work_plan must be on the same device as q")
        want = attention_queries_per_item(q.dtype, current_k.dtype, current_v.dtype, k_split_rows=k_split_rows)
        have = getattr(work_plan, "hkv_queries_per_item", None)
        shape = getattr(work_plan, "hkv_plan_shape", None)
        if have is None or shape is None:
            raise ValueError("work_plan must be a tensor made by segmented_attention_plan (it records the item "
                             "size, batch size and length it was built for; clone() / to() drop that record)")
        if tuple(shape) != (batch_size, current_len):
            raise ValueError(f"work_plan was built for batch {shape[0]} and length {shape[1]}; this call has "
                             f"batch {batch_size} and length {current_len}")
        if have != want:
            raise ValueError(f"work_plan was built for {have}-query items; this call's kernel takes {want} "
                             "(segmented_attention_plan(..., queries_per_item=attention_queries_per_item(...)))")
    if append_offsets is not None:
        if split and not k_split_rows:
            raise ValueError("append_offsets: the split-row K path writes a split copy of the slab; "
                             "append after the call (attention_fuses_append)")
        if (append_offsets.dtype != torch.int32 or tuple(append_offsets.shape) != (num_heads,)
                or append_offsets.device != q.device):
            raise ValueError("append_offsets must be an int32 tensor [H] on q's device")
        if persisted_k.dtype != current_k.dtype or persisted_v.dtype != current_v.dtype:
            raise ValueError("append_offsets: the slab and the current rows must share their dtypes")
        append_offsets = append_offsets.contiguous()
    if append_also is not None:
        if append_offsets is None:
            raise ValueError("append_also repeats the append of append_offsets; pass both")
        slab2_k, slab2_v, offsets2 = append_also
        if (slab2_k.ndim != 3 or slab2_k.shape != slab2_v.shape or slab2_k.shape[0] != batch_size
                or slab2_k.shape[2] != head_dim):
            raise ValueError("append_also: slab2_k and slab2_v must be [B, capacity2, D] tensors of one shape")
        if slab2_k.dtype != current_k.dtype or slab2_v.dtype != current_v.dtype:
            raise ValueError("append_also: the second slab and the current rows must share their dtypes")
        if slab2_k.device != q.device or slab2_v.device != q.device:
            raise ValueError("append_also: the second slab must be on q's device")
        if not (slab2_k.is_contiguous() and slab2_v.is_contiguous()):
            raise ValueError("append_also: the second slab must be contiguous (the append writes it in place)")
        if (offsets2.dtype != torch.int32 or tuple(offsets2.shape) != (num_heads,)
                or offsets2.device != q.device):
            raise ValueError("append_also: its offsets must be an int32 tensor [H] on q's device")
        offsets2 = offsets2.contiguous()
    stream = torch.cuda.current_stream(q.device)
    ws = _lib.attention_workspace(q.device, stream)
    k_code = _lib.dtype_code(current_k.dtype)
    converted = promoted or (split and not k_split_rows)
    if split:
        # fp32 K as split rows for the split-row kernel (the q split happens in it)
        if not k_split_rows:
            persisted_k = _split_rows(persisted_k, stream)
            current_k = _split_rows(current_k, stream)
        k_code = _lib.DTYPE_SPLIT_ROWS
    args = [
        q.data_ptr(), persisted_k.data_ptr(), persisted_v.data_ptr(),
        segment_starts.data_ptr(), segment_ends.data_ptr(), segment_counts.data_ptr(),
        current_k.data_ptr(), current_v.data_ptr(), output.data_ptr(),
        lse.data_ptr() if lse is not None else None,
        batch_size, num_heads, current_len,
        int(persisted_k.shape[1]), int(segment_starts.shape[1]), head_dim,
        _lib.dtype_code(q.dtype), k_code, _lib.dtype_code(current_v.dtype),
        _lib.dtype_code(out_dtype), float(softmax_scale), 1 if softmax_mode == "exp2" else 0, qk_mode, value_mode,
        work_plan.data_ptr() if work_plan is not None else None,
        int(work_plan.shape[0]) if work_plan is not None else 0,
        ws.data_ptr() if ws is not None else None, int(ws.numel()) if ws is not None else 0,
    ]
    lib = _lib.load()
    if append_offsets is None:
        fn = lib.hkv_segmented_attention
    elif append_also is None:
        fn = lib.hkv_segmented_attention_append
        args.append(append_offsets.data_ptr())
    else:
        fn = lib.hkv_segmented_attention_append2
        args += [append_offsets.data_ptr(), slab2_k.data_ptr(), slab2_v.data_ptr(), int(slab2_k.shape[1]),
                 offsets2.data_ptr()]
    args.append(stream.cuda_stream)
    _lib.check(fn(*args))
    if _bind is not None:
        # what a pre-bound call needs to repeat this launch for new q / k / v
        # / slab tensors of the same shapes (None when this call converted its
        # inputs: those copies are per call)
        keep = (q, persisted_k, persisted_v, current_k, current_v, segment_starts, segment_ends, segment_counts,
                work_plan, append_offsets, ws, append_also)
        _bind.append(None if converted or lse is not None else (fn, args, output.shape, out_dtype, keep))
    if return_lse:
        return output, lse
    return output


class BoundSegmentedAttention:
    """A pre-validated launch of :func:`fused_real_pruning_flat_segmented_attention`
    for callers that repeat one call shape many times (the segmented cache's
    per-(layer, scale) steps): built from one call of the operator (which runs
    every check), it holds that call's arguments bound in the library
    (``hkv_segmented_attention_bind``) and repeats the launch
    (``hkv_segmented_attention_call``) for new q, current K/V and slab tensors
    with the same shapes, dtypes and device, on the same stream, with the same
    tables, plan, append offsets and knobs: the operator's validation and
    argument marshalling are skipped, only the new tensors' pointers pass.
    ``__call__`` returns None, launching nothing, when the new tensors or the
    stream do not match (or a HIP graph is being captured); the caller then
    calls the operator."""

    __slots__ = ("_block", "_addr", "_call", "_out_shape", "_out_dtype", "_keep", "_dev", "_device", "_stream",
                 "_qs", "_ps", "_qdt", "_kdt", "_vdt", "_skdt", "_svdt")

    def __init__(self, record, *, q, current_k, current_v, persisted_k, persisted_v):
        fn, a, out_shape, out_dtype, keep = record
        lib = _lib.load()
        size = int(lib.hkv_segmented_attention_bound_bytes())
        self._block = (ctypes.c_int64 * ((size + 7) // 8))()
        self._addr = ctypes.addressof(self._block)
        append = a[28] if len(a) > 29 else None
        if len(a) > 30:
            # the second append destination (slab2 K/V, capacity, offsets) is bound with the rest
            _lib.check(lib.hkv_segmented_attention_bind2(
                self._addr, size, a[3], a[4], a[5], a[10], a[11], a[12], a[13], a[14], a[15], a[16], a[17], a[18],
                a[19], a[20], a[21], a[22], a[23], a[24], a[25], a[26], a[27], append, a[29], a[30], a[31], a[32]))
        else:
            _lib.check(lib.hkv_segmented_attention_bind(
                self._addr, size, a[3], a[4], a[5], a[10], a[11], a[12], a[13], a[14], a[15], a[16], a[17], a[18],
                a[19], a[20], a[21], a[22], a[23], a[24], a[25], a[26], a[27], append))
        self._call = lib.hkv_segmented_attention_call
        self._out_shape = tuple(out_shape)
        self._out_dtype = out_dtype
        self._keep = keep  # tables, plan, offsets and workspace the bound pointers refer to
        self._dev = q.get_device()
        self._device = q.device
        self._stream = a[-1]
        self._qs = q.shape
        self._ps = persisted_k.shape
        self._qdt, self._kdt, self._vdt = q.dtype, current_k.dtype, current_v.dtype
        self._skdt, self._svdt = persisted_k.dtype, persisted_v.dtype

    @classmethod
    def bind(cls, **kwargs):
        """Calls the operator with ``kwargs`` and returns ``(output, bound)``;
        ``bound`` is None when the call cannot be repeated this way (its
        inputs were converted for the launch, or it returned the LSE)."""
        rec = []
        out = fused_real_pruning_flat_segmented_attention(**kwargs, _bind=rec)
        bound = None
        if rec and rec[0] is not None and not torch.cuda.is_current_stream_capturing():
            bound = cls(rec[0], q=kwargs["q"], current_k=kwargs["current_k"], current_v=kwargs["current_v"],
                        persisted_k=kwargs["persisted_k"], persisted_v=kwargs["persisted_v"])
        return out, bound

    def __call__(self, q, current_k, current_v, persisted_k, persisted_v):
        qs, ps, dev = self._qs, self._ps, self._dev
        if (q.shape != qs or current_k.shape != qs or current_v.shape != qs or persisted_k.shape != ps
                or persisted_v.shape != ps or q.dtype is not self._qdt or current_k.dtype is not self._kdt
                or current_v.dtype is not self._vdt or persisted_k.dtype is not self._skdt
                or persisted_v.dtype is not self._svdt or q.get_device() != dev or current_k.get_device() != dev
                or current_v.get_device() != dev or persisted_k.get_device() != dev
                or persisted_v.get_device() != dev or not q.is_contiguous() or not current_k.is_contiguous()
                or not current_v.is_contiguous() or not persisted_k.is_contiguous()
                or not persisted_v.is_contiguous()):
            return None
        stream = torch._C._cuda_getCurrentRawStream(dev)
        if stream != self._stream or torch.cuda.is_current_stream_capturing():
            return None
        out = torch.empty(self._out_shape, dtype=self._out_dtype, device=self._device)
        code = self._call(self._addr, q.data_ptr(), persisted_k.data_ptr(), persisted_v.data_ptr(),
                          current_k.data_ptr(), current_v.data_ptr(), out.data_ptr(), stream)
        if code != 0:
            _lib.check(code)
        return out


class BoundPack:
    """A pre-validated launch of :func:`pack_flat_segments_kv` (same copy
    items, source and destination shapes, dtypes, device and stream) repeated
    for new source and destination tensors: only their pointers pass.
    ``__call__`` returns False, copying nothing, when the tensors or the
    stream do not match (or a HIP graph is being captured)."""

    __slots__ = ("_fn", "_args", "_meta", "_dev", "_stream", "_ss", "_ds", "_sdt", "_ddt")

    def __init__(self, record, *, src_k, src_v, dst_k, dst_v):
        self._fn, args, self._meta = record  # meta: the copy items the recorded pointers refer to
        self._args = list(args)
        self._dev = dst_k.get_device()
        self._stream = args[-1]
        self._ss, self._ds = src_k.shape, dst_k.shape
        self._sdt, self._ddt = (src_k.dtype, src_v.dtype), (dst_k.dtype, dst_v.dtype)

    @classmethod
    def bind(cls, src_shape=None, **kwargs):
        """Calls :func:`pack_flat_segments_kv` with ``kwargs``; returns the
        bound copy, or None when nothing was launched (no items) or a HIP
        graph is being captured.  ``src_shape``: the shape later calls pass
        their sources in, when not ``kwargs["src_k"]``'s (a contiguous
        ``[B, H, n, D]`` whose flat view was packed)."""
        rec = []
        pack_flat_segments_kv(**kwargs, _bind=rec)
        if not rec or torch.cuda.is_current_stream_capturing():
            return None
        bound = cls(rec[0], src_k=kwargs["src_k"], src_v=kwargs["src_v"], dst_k=kwargs["dst_k"],
                    dst_v=kwargs["dst_v"])
        if src_shape is not None:
            bound._ss = torch.Size(src_shape)
        return bound

    def __call__(self, src_k, src_v, dst_k, dst_v) -> bool:
        ss, ds, dev = self._ss, self._ds, self._dev
        if (src_k.shape != ss or src_v.shape != ss or dst_k.shape != ds or dst_v.shape != ds
                or (src_k.dtype, src_v.dtype) != self._sdt or (dst_k.dtype, dst_v.dtype) != self._ddt
                or src_k.get_device() != dev or src_v.get_device() != dev or dst_k.get_device() != dev
                or dst_v.get_device() != dev or not src_k.is_contiguous() or not src_v.is_contiguous()
                or not dst_k.is_contiguous() or not dst_v.is_contiguous()):
            return False
        stream = torch._C._cuda_getCurrentRawStream(dev)
        if stream != self._stream or torch.cuda.is_current_stream_capturing():
            return False
        a = self._args
        a[0] = src_k.data_ptr()
        a[1] = src_v.data_ptr()
        a[2] = dst_k.data_ptr()
        a[3] = dst_v.data_ptr()
        code = self._fn(*a)
        if code != 0:
            _lib.check(code)
        return True
