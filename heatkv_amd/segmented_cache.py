"""Per-layer KV state of the fused segmented path: dense prefix, slab, appends.

``SegmentedLayerCache.step`` is the key/value half of the reference's patched
``SelfAttention.forward`` (``_real_pruning_scale_specific_fast_forward``,
enable_real_pruning_fast.py:1951-2254) for one layer and one scale: it takes
the scale's q, k, v ``[B, H, n, D]`` (after the QKV projection, normalization
and RoPE of the caller) and returns the attention output ``[B, n, H*D]``.
Control flow, all device work on torch's current stream, no host sync:

* dense prefix (:1972-2038): while no head of this layer is pruned at the
  current target, attention runs over the whole dense cache ``[B, H, T, D]``
  plus the current scale, and the cache grows by concatenation (one HIP
  launch for K and V, ``concat_kv``); when the next
  target prunes a head, the dense cache is packed into the slab with the
  schedule's activation copy items (:1639-1711 -> :888-908);
* segmented (:2122-2155): attention over the slab segments of the target's
  offset tables plus the current scale;
* compact (:2176-2253): at the final scale the state is reset; otherwise the
  current scale's kept heads are appended to the slab (:1791-1807 -> :969-995)
  or, if the slab is not active yet, the dense cache and the current scale
  are packed into it (:1713-1789).

Every attention call is the HIP segmented-attention kernel: the dense prefix
uses it too, with the dense cache viewed as a slab ``[B, H*T, D]`` holding one
segment per head (the same softmax over the same keys as the reference's
SDPA).  Every copy into the slab is the HIP pack kernel.
"""

from __future__ import annotations

import os
from typing import Callable, Dict, Mapping, Optional, Set, Tuple

import torch

from . import _lib
from . import phase_profile as prof
from .real_pruning_fused_attention import (
    BoundPack,
    BoundSegmentedAttention,
    attention_fuses_append,
    attention_item_shape,
    concat_kv,
    fused_real_pruning_flat_segmented_attention,
    pack_flat_segments_kv,
    segmented_attention_plan,
)
from .slab_schedule import CopyPlan, SlabSchedule

RemovedLookup = Callable[[int], Mapping[int, Set[int]]]


def _env_flag(name: str, default: bool) -> bool:
    raw = _lib.env_get(name)
    if raw is None:
        return default
    return raw.strip().lower() not in {"0", "false", "no", "off"}


def baseline_prefix_enabled() -> bool:
    """REAL_PRUNING_FUSED_SEGMENTED_BASELINE_PREFIX (default on; enable_real_pruning_fast.py:1062-1066)."""
    return _env_flag("REAL_PRUNING_FUSED_SEGMENTED_BASELINE_PREFIX", True)


def work_plans_enabled(device) -> bool:
    """HKV_ATTN_PLAN (default on): attention calls on a GPU carry a host work
    plan of their (static) tables, built once per tables, batch and length.
    While a HIP graph is being captured no plan is built (its upload would be
    a captured host copy): a call uses the plan made by an eager call before
    the capture, so that replays compute exactly what eager calls compute,
    and none if there was no such call."""
    return _env_flag("HKV_ATTN_PLAN", True) and torch.device(device).type == "cuda"


def fused_append_enabled() -> bool:
    """HKV_FUSED_APPEND (default on): the attention launch of a step also
    writes the current rows that the append for the next scale places outside
    every segment it reads (``append_offsets``); the copy after it moves only
    the rest.  Under HIP-graph capture only a split made by an eager call is
    used."""
    return _env_flag("HKV_FUSED_APPEND", True)


def _capturing() -> bool:
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def fused_softmax_mode() -> str:
    """REAL_PRUNING_FUSED_SOFTMAX_MODE, 'exp' or 'exp2' (enable_real_pruning_fast.py:166-170)."""
    mode = _lib.env_get("REAL_PRUNING_FUSED_SOFTMAX_MODE", "exp")
    return mode if mode in {"exp", "exp2"} else "exp"


def has_removed(removed: Mapping[int, Set[int]]) -> bool:
    return any(len(v) > 0 for v in removed.values())


# Environment knobs a step's launches depend on; a cache replays recorded
# steps only while they read as they did when the steps were recorded (they
# are read once per generation, at its first step).
_STEP_KNOBS = ("REAL_PRUNING_FUSED_QK_DOT_MODE", "REAL_PRUNING_FUSED_VALUE_DOT_MODE",
               "REAL_PRUNING_FUSED_SOFTMAX_MODE", "REAL_PRUNING_FUSED_SEGMENTED_BASELINE_PREFIX",
               "REAL_PRUNING_FUSED_BLOCK_M", "REAL_PRUNING_FUSED_BLOCK_N", "REAL_PRUNING_FUSED_NUM_WARPS",
               "REAL_PRUNING_FUSED_NUM_STAGES", "HKV_ATTN_SPLIT", "HKV_ATTN_PLAN", "HKV_FUSED_APPEND",
               "HKV_ATTN_SPLIT_ROWS")

# os.environ keeps its values in a dict of encoded keys (CPython on POSIX;
# os.environ[...] = ... updates it): reading the knobs from it directly takes
# ~0.5 us per generation and layer instead of ~6 us through os.environ.get.
_ENV_DATA = getattr(os.environ, "_data", None)
_STEP_KNOB_KEYS = None
if isinstance(_ENV_DATA, dict):
    try:
        _STEP_KNOB_KEYS = tuple(os.environ.encodekey(n) for n in _STEP_KNOBS)
    except Exception:  # pragma: no cover - another platform's os.environ
        _STEP_KNOB_KEYS = None


def _step_knobs() -> tuple:
    """The knobs a replayed step depends on, as the environment has them now."""
    if _STEP_KNOB_KEYS is not None:
        return tuple(map(_ENV_DATA.get, _STEP_KNOB_KEYS))
    return tuple(os.environ.get(n) for n in _STEP_KNOBS)


class _StepReplay:
    """One recorded step of a generation (scale, shapes, dtypes and arguments
    fixed), repeated by later generations without the step's host logic: the
    attention launch through a :class:`BoundSegmentedAttention` and the state
    changes that followed it.  ``run`` returns None (doing nothing) when the
    cache is not in the state the step was recorded in, or the launch cannot
    be repeated as bound; the caller then takes the full step."""

    __slots__ = ("args", "kind", "attn", "old_len", "new_len", "final", "k_split_rows", "copy", "activate",
                 "buf_shapes", "dual", "scale")

    def __init__(self, args, kind, attn, old_len, new_len, final, copy=None, activate=None, buf_shapes=None,
                 dual=False, scale=-1):
        self.args = args  # the step's (out_dtype, softmax_scale, softmax_mode, appended, k_split_rows)
        k_split_rows = bool(args[4])
        self.kind = kind  # "slab": segmented step; "dense": dense prefix kept in place
        self.attn = attn
        self.old_len = old_len
        self.new_len = new_len
        self.final = final
        self.k_split_rows = k_split_rows
        self.copy = copy  # (plan, tag) of the residual append, or None
        self.activate = activate  # target whose slab is packed after a dense step, or None
        self.buf_shapes = buf_shapes  # ((shape, dtype), (shape, dtype)) of the dense buffer
        self.dual = dual  # the launch also wrote the rows into the slab (dense step; the bound slab storage)
        self.scale = scale

    def run(self, cache: "SegmentedLayerCache", q, k, v):
        if cache.logical_len != self.old_len:
            return None
        if self.old_len == 0:
            cache.k_split_rows = self.k_split_rows
        elif cache.k_split_rows != self.k_split_rows:
            return None
        if self.kind == "slab":
            if not cache.active or cache.cached_k is None:
                return None
            out = self.attn(q, k, v, cache.cached_k, cache.cached_v)
            if out is None:
                return None
            if self.final:
                cache.reset()
                return out
            if self.copy is not None:
                cache._copy(self.copy[0], k, v, self.copy[1])
            cache.logical_len = self.new_len
            return out
        if cache.active:
            return None
        if cache.dense_buf is None:
            if self.old_len != 0:
                return None
            (sk, dk), (sv, dv) = self.buf_shapes
            cache.dense_buf = (torch.empty(sk, dtype=dk, device=k.device), torch.empty(sv, dtype=dv, device=v.device))
        buf_k, buf_v = cache.dense_buf
        views = cache._dense_views
        if views is None:
            B, H, cap = buf_k.shape[0], buf_k.shape[1], buf_k.shape[2]
            views = cache._dense_views = (buf_k.view(B, H * cap, buf_k.shape[3]),
                                          buf_v.view(B, H * cap, buf_v.shape[3]))
        out = self.attn(q, k, v, views[0], views[1])
        if out is None:
            return None
        if self.final:
            cache.reset()
            return out
        cache.logical_len = self.new_len
        cache._dual_next = self.scale + 1 if self.dual and cache._dual_next == self.scale else -1
        if self.activate is not None:
            cache._activate_after_dense(buf_k, buf_v, self.activate)
            cache.dense_buf = None
            cache._dense_views = None
        return out


class SegmentedLayerCache:
    """KV cache of one attention layer under a static slab schedule."""

    def __init__(self, schedule: SlabSchedule, removed: RemovedLookup, *, num_heads: int,
                 num_scales: Optional[int] = None):
        self.schedule = schedule
        self.removed = removed
        self.num_heads = int(num_heads)
        self.num_scales = int(schedule.num_scales if num_scales is None else num_scales)
        self._tables_by_len: Dict[tuple, Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}
        self._dense_current_plans: Dict[tuple, Tuple[CopyPlan, CopyPlan]] = {}
        # steps recorded by an earlier generation, by scale
        self._replays: Dict[int, _StepReplay] = {}
        self._packs: Dict[tuple, BoundPack] = {}  # bound slab copies, by copy tag
        self._knobs: Optional[tuple] = None
        # the slab's storage, kept for the next generations (same shape and
        # dtypes): bound second appends of dense steps refer to it
        self._slab_store: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self.reset()

    # ------------------------------------------------------------------ state

    def reset(self) -> None:
        """Empty cache (kv_caching(True) and the final scale; :2257-2266, :2176-2185)."""
        self.cached_k: Optional[torch.Tensor] = None
        self.cached_v: Optional[torch.Tensor] = None
        self.logical_len = 0
        self.active = False  # cached_k/v hold the slab
        # K rows held as split rows (float32-typed; qkv_produce(k_split_rows=True)),
        # fixed by the first step after a reset
        self.k_split_rows = False
        # the dense prefix kept in place: (K, V) [B, H, rows, D] sized for every
        # dense scale, each step's rows written by its attention launch
        self.dense_buf: Optional[Tuple[torch.Tensor, torch.Tensor]] = None
        self._dense_views = None  # dense_buf seen as slabs [B, H*rows, D] (replayed steps)
        # the next dense scale whose rows the in-place steps also wrote into
        # the slab storage (-1: a step did not), so the activation has nothing to pack
        self._dual_next = 0

    def _slab_storage(self, batch: int, head_dim: int, device, k_dtype, v_dtype) -> Tuple[torch.Tensor, torch.Tensor]:
        """The slab's K/V storage ``[B, capacity, D]``, allocated when its shape,
        dtypes or device change and kept across generations (the reference
        allocates it per generation, :1092-1144; contents of unowned rows are
        undefined either way).  A new storage drops the recorded steps, whose
        bound second appends point at the old one."""
        cap = int(self.schedule.capacity)
        st = self._slab_store
        if (st is None or tuple(st[0].shape) != (batch, cap, head_dim) or st[0].dtype != k_dtype
                or st[1].dtype != v_dtype or st[0].device != torch.device(device)):
            st = self._slab_store = (torch.empty((batch, cap, head_dim), device=device, dtype=k_dtype),
                                     torch.empty((batch, cap, head_dim), device=device, dtype=v_dtype))
            self._replays.clear()
            prof.stat_add("storage_allocations")
            prof.stat_add("storage_capacity_slots", cap)
        return st

    def _ensure_slab(self, batch: int, head_dim: int, device, k_dtype, v_dtype) -> None:
        """Slab K/V ``[B, capacity, D]`` (:1092-1144) as the cache."""
        self.cached_k, self.cached_v = self._slab_storage(batch, head_dim, device, k_dtype, v_dtype)

    # ------------------------------------------------------------------ copies

    def _copy(self, plan: CopyPlan, src_k: torch.Tensor, src_v: torch.Tensor, tag) -> None:
        """Pack ``plan``'s items from ``src`` ``[B, H, n, D]`` into the slab."""
        if len(plan) == 0:
            return
        B, H, n, D = src_k.shape
        if n != plan.sequence_len:
            raise RuntimeError("static precomputed copy run sequence length mismatch")
        prof.stat_add("static_copy_calls")
        prof.record_kv_copy("static_copy", slots=plan.slots, k_tensor=src_k, v_tensor=src_v)
        if not prof._enabled:
            bound = self._packs.get(tag)
            if bound is not None and bound(src_k, src_v, self.cached_k, self.cached_v):
                return
        dst_starts, src_starts, lengths = self.schedule.device_plan(plan, src_k.device, tag)
        kw = dict(dst_k=self.cached_k, dst_v=self.cached_v,
                  src_k=src_k.reshape(B, H * n, D), src_v=src_v.reshape(B, H * n, D),
                  dst_starts=dst_starts, src_starts=src_starts, lengths=lengths, max_length=plan.max_length)
        if src_k.is_cuda and not prof._enabled and not _capturing():
            # later copies of this plan go through the bound launch (same 4-D
            # source shape: the flat view has the source's pointer)
            bound = BoundPack.bind(src_shape=src_k.shape, **kw)
            if bound is not None:
                self._packs[tag] = bound
        else:
            pack_flat_segments_kv(**kw)

    def _activate_after_dense(self, dense_k, dense_v, target: int) -> None:
        """The slab becomes the cache at ``target``: when every dense step of
        this generation also wrote its rows into the slab storage, there is
        nothing left to pack; else the dense cache is packed."""
        if self._dual_next == target and self._slab_store is not None:
            B, H, T, D = dense_k.shape
            self._ensure_slab(B, D, dense_k.device, dense_k.dtype, dense_v.dtype)
            self.active = True
            prof.stat_add("static_pack_state_calls")
            return
        self._activate_from_dense(dense_k, dense_v, target)

    def _activation_target(self) -> Optional[int]:
        """The first target with removed heads (the slab's activation), or None."""
        return next((t for t in range(1, self.num_scales) if has_removed(self.removed(t))), None)

    def _dual_offsets(self, target: int, scale: int, heads: int, device) -> torch.Tensor:
        """Slab offsets of scale ``scale``'s rows of each head at ``target``
        (-1: not live there), on ``device``, made once: where the in-place
        dense step of ``scale`` also writes its rows."""
        key = ("dual", int(target), int(scale), heads, str(device))
        hit = self._tables_by_len.get(key)
        if hit is None:
            offs = torch.full((heads,), -1, dtype=torch.int32)
            for seg in self.schedule.live_segments(int(target)):
                if seg.source_scale == scale and 0 <= seg.head < heads:
                    offs[seg.head] = int(seg.offset)
            hit = self._tables_by_len[key] = offs.to(device)
        return hit

    def _activate_from_dense(self, dense_k, dense_v, target: int) -> None:
        """Pack the dense cache into a new slab for ``target`` (:1639-1711)."""
        B, H, T, D = dense_k.shape
        self._ensure_slab(B, D, dense_k.device, dense_k.dtype, dense_v.dtype)
        self.active = True
        plan = self.schedule.activation_plans.get(int(target))
        if plan is None or plan.sequence_len != T:
            raise RuntimeError("segmented static pack: no activation plan for this cache length")
        prof.stat_add("static_pack_state_calls")
        self._copy(plan, dense_k, dense_v, ("activation", int(target)))

    def _dense_and_current_plans(self, target: int, scale: int, old_len: int, cur_len: int):
        """Copy items of the live segments at ``target``: sources before ``scale`` from the
        dense cache, source ``scale`` from the current tensors (:871-967)."""
        key = (target, scale, old_len, cur_len)
        hit = self._dense_current_plans.get(key)
        if hit is not None:
            return hit
        old, cur = [], []
        for seg in self.schedule.live_segments(target):
            if seg.source_scale == scale:
                a = max(seg.scale_start, old_len) - old_len
                b = min(seg.scale_end, old_len + cur_len) - old_len
                if a < b:
                    cur.append((seg.offset, seg.head * cur_len + a, b - a))
            else:
                b = min(seg.scale_end, old_len)
                if seg.scale_start < b:
                    old.append((seg.offset, seg.head * old_len + seg.scale_start, b - seg.scale_start))

        def plan(items, n):
            items.sort()
            return CopyPlan([i[0] for i in items], [i[1] for i in items], [i[2] for i in items], n)

        hit = (plan(old, old_len), plan(cur, cur_len))
        self._dense_current_plans[key] = hit
        return hit

    # ------------------------------------------------------------------ dense prefix in place

    def dense_kv(self) -> Optional[Tuple[torch.Tensor, torch.Tensor]]:
        """The dense prefix so far, ``[B, H, logical_len, D]`` K and V (a view of
        the in-place buffer, or the concatenated tensors), or None once the
        slab holds the cache (or before the first step)."""
        if self.active:
            return None
        if self.dense_buf is not None:
            return tuple(t[:, :, :self.logical_len] for t in self.dense_buf)
        if self.cached_k is None:
            return None
        return self.cached_k, self.cached_v

    def _dense_capacity(self) -> int:
        """Rows per head of the dense prefix kept in place: every token of the
        scales before the first target with removed heads (the slab's
        activation), or before the final scale when none has any."""
        act = next((t for t in range(1, self.num_scales) if has_removed(self.removed(t))), self.num_scales - 1)
        return int(self.schedule.scale_ranges[act - 1][1]) if act >= 1 else 0

    def _in_place_tables(self, heads: int, cap: int, old_len: int, device, batch: int, L: int, shape: tuple,
                         store: bool):
        """Tables presenting rows ``[0, old_len)`` of each head of the in-place
        dense prefix ``[B, H, cap, D]`` as a slab ``[B, H*cap, D]``, their work
        plan, and the append offsets ``h*cap + old_len`` of this step's rows
        (None when nothing is stored), made once.  ``shape``: the kernel's
        ``(queries_per_item, slots)`` (attention_item_shape)."""
        key = ("in_place", heads, cap, old_len, str(device), batch, L, shape, store)
        hit = self._tables_by_len.get(key)
        if hit is None:
            starts = (torch.arange(heads, dtype=torch.int32) * cap).reshape(heads, 1)
            ends = starts + old_len
            counts = torch.ones((heads,), dtype=torch.int32)
            plan = (segmented_attention_plan(starts, ends, counts, batch_size=batch, current_len=L,
                                             capacity=heads * cap, device=device, queries_per_item=shape[0],
                                             slots=shape[1])
                    if work_plans_enabled(device) and not _capturing() else None)
            offs = (starts.reshape(heads) + old_len).to(device) if store else None
            hit = (starts.to(device), ends.to(device), counts.to(device), plan, offs)
            self._tables_by_len[key] = hit
        return hit

    def _in_place_ok(self, q, k, v) -> bool:
        """Whether this generation's dense prefix can be kept in place: the
        attention launch must take the append of the step's rows."""
        return fused_append_enabled() and attention_fuses_append(q.dtype, k.dtype, v.dtype,
                                                                 k_split_rows=self.k_split_rows)

    def _dense_step_in_place(self, q, k, v, scale_ind: int, scale: float, mode, out_dtype, final: bool,
                             record=None):
        """A dense-prefix step (:1972-2038) on the in-place buffer: attention over
        the rows so far plus the current scale, whose rows the same launch
        writes behind them (the reference concatenates them onto the cache);
        at the first target with removed heads the full buffer is packed into
        the slab."""
        B, H, L, D = q.shape
        old_len = self.logical_len
        if self.dense_buf is None:
            cap = self._dense_capacity()
            self.dense_buf = (torch.empty((B, H, cap, k.shape[3]), dtype=k.dtype, device=k.device),
                              torch.empty((B, H, cap, v.shape[3]), dtype=v.dtype, device=v.device))
        buf_k, buf_v = self.dense_buf
        cap = int(buf_k.shape[2])
        store = not final
        if store and old_len + L > cap:
            raise RuntimeError("dense prefix longer than its in-place buffer")
        shape = attention_item_shape(q.dtype, k.dtype, v.dtype, k_split_rows=self.k_split_rows, device=q.device)
        st, en, ct, plan, offs = self._in_place_tables(H, cap, old_len, q.device, B, L, shape, store)
        kw = dict(q=q, persisted_k=buf_k.reshape(B, H * cap, buf_k.shape[3]),
                  persisted_v=buf_v.reshape(B, H * cap, buf_v.shape[3]), segment_starts=st, segment_ends=en,
                  segment_counts=ct, current_k=k, current_v=v, softmax_scale=scale, softmax_mode=mode,
                  out_dtype=out_dtype, work_plan=plan, append_offsets=offs, k_split_rows=self.k_split_rows)
        # the same launch also writes the step's rows into the slab storage at
        # their offsets of the activation target, so that target packs nothing
        act = self._activation_target()
        dual = store and act is not None and scale_ind < act and self._dual_next == scale_ind
        if dual:
            slab_k, slab_v = self._slab_storage(B, k.shape[3], k.device, k.dtype, v.dtype)
            kw["append_also"] = (slab_k, slab_v, self._dual_offsets(act, scale_ind, H, q.device))
        self._dual_next = scale_ind + 1 if dual else -1
        bound = None
        with prof.phase("attention"):
            if record is not None:
                out, bound = BoundSegmentedAttention.bind(**kw)
            else:
                out = fused_real_pruning_flat_segmented_attention(**kw)
        activate = None
        if final:
            self.reset()
        else:
            self.logical_len = old_len + L
            if has_removed(self.removed(scale_ind + 1)):
                if self.logical_len != cap:
                    raise RuntimeError("dense prefix packed into the slab before its buffer is full")
                activate = scale_ind + 1
                with prof.phase("compact"):
                    self._activate_after_dense(buf_k, buf_v, activate)
                self.dense_buf = None
                self._dense_views = None
        if bound is not None:
            self._replays[scale_ind] = _StepReplay(
                record, "dense", bound, old_len, old_len + L, final,
                activate=activate, buf_shapes=((tuple(buf_k.shape), buf_k.dtype), (tuple(buf_v.shape), buf_v.dtype)),
                dual=dual, scale=scale_ind)
        return out

    # ------------------------------------------------------------------ attention

    def _dense_tables(self, heads: int, T: int, device, batch: int, L: int, shape: tuple):
        """Offset tables that present a dense cache ``[B, H, T, D]`` as a slab
        ``[B, H*T, D]``, and their work plan for ``batch`` x ``L`` queries
        (``shape``: the kernel's ``(queries_per_item, slots)``)."""
        key = (heads, T, str(device), batch, L, shape)
        hit = self._tables_by_len.get(key)
        if hit is None:
            starts = (torch.arange(heads, dtype=torch.int32) * T).reshape(heads, 1)
            ends = starts + T
            counts = torch.ones((heads,), dtype=torch.int32)
            plan = (segmented_attention_plan(starts, ends, counts, batch_size=batch, current_len=L,
                                             capacity=heads * T, device=device, queries_per_item=shape[0],
                                             slots=shape[1])
                    if work_plans_enabled(device) and not _capturing() else None)
            hit = (starts.to(device), ends.to(device), counts.to(device), plan)
            self._tables_by_len[key] = hit
        return hit

    def _empty_tables(self, heads: int, device, batch: int, L: int, shape: tuple):
        """Tables with no segment (attention over the current scale only) and
        their work plan, made once."""
        key = ("empty", heads, str(device), batch, L, shape)
        hit = self._tables_by_len.get(key)
        if hit is None:
            empty = torch.zeros((heads, 0), dtype=torch.int32)
            counts = torch.zeros((heads,), dtype=torch.int32)
            plan = (segmented_attention_plan(empty, empty, counts, batch_size=batch, current_len=L, capacity=0,
                                             device=device, queries_per_item=shape[0], slots=shape[1])
                    if work_plans_enabled(device) and not _capturing() else None)
            hit = (empty.to(device), empty.to(device), counts.to(device), plan)
            self._tables_by_len[key] = hit
        return hit

    def _attend_dense(self, q, k, v, scale, mode, out_dtype=None):
        B, H, L, D = q.shape
        shape = attention_item_shape(q.dtype, k.dtype, v.dtype, k_split_rows=self.k_split_rows, device=q.device)
        if self.cached_k is None or self.logical_len == 0:
            tables = self._empty_tables(H, q.device, B, L, shape)
            slab_k = slab_v = None
        else:
            T = self.cached_k.shape[2]
            tables = self._dense_tables(H, T, q.device, B, L, shape)
            slab_k = self.cached_k.reshape(B, H * T, D)
            slab_v = self.cached_v.reshape(B, H * T, D)
        return fused_real_pruning_flat_segmented_attention(
            q=q, persisted_k=slab_k, persisted_v=slab_v, segment_starts=tables[0],
            segment_ends=tables[1], segment_counts=tables[2], current_k=k, current_v=v,
            softmax_scale=scale, softmax_mode=mode, out_dtype=out_dtype, work_plan=tables[3],
            k_split_rows=self.k_split_rows)

    # ------------------------------------------------------------------ step

    def producer_append(self, scale_ind: int, k_dtype: torch.dtype, device):
        """``(slab_k, slab_v, offsets)`` for a producer that appends the kept heads'
        rows of ``scale_ind`` into the slab before this scale's attention, or
        None.  Only heads whose slab rows this scale's attention does not read
        are offered (:meth:`SlabSchedule.fused_append`); the rest stay with the
        copy after attention.  A step of the same scale must then be called
        with ``appended=True``."""
        if (not self.active or self.cached_k is None or scale_ind + 1 >= self.num_scales
                or self.cached_k.dtype != k_dtype):
            return None
        offsets, _ = self.schedule.fused_append(int(scale_ind), device)
        if offsets is None:
            return None
        return self.cached_k, self.cached_v, offsets

    def _fused_append_offsets(self, scale_ind: int, q, k, v) -> Optional[torch.Tensor]:
        """``append_offsets`` of this step's attention launch, or None."""
        if not fused_append_enabled() or not attention_fuses_append(q.dtype, k.dtype, v.dtype,
                                                                    k_split_rows=self.k_split_rows):
            return None
        if self.cached_k.dtype != k.dtype or self.cached_v.dtype != v.dtype:
            return None
        hit = self.schedule.fused_append(int(scale_ind), k.device, build=not _capturing())
        return None if hit is None else hit[0]

    def step(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale_ind: int,
             softmax_scale: float, softmax_mode: Optional[str] = None, appended: bool = False,
             out_dtype: Optional[torch.dtype] = None, k_split_rows: bool = False) -> torch.Tensor:
        """Attention of scale ``scale_ind`` and the cache update for the next scale.

        ``appended``: the producer already wrote the rows offered by
        :meth:`producer_append` for this scale; only the other heads are copied.
        ``out_dtype``: element type of the output (q's by default).
        ``k_split_rows``: k (fp32-typed) holds split rows of fp32 K
        (``qkv_produce(..., k_split_rows=True)``); every step of a generation
        passes the same value, and the cache's K rows keep that format."""
        record = None
        if not prof._enabled:
            if self.logical_len == 0:
                knobs = _step_knobs()
                if knobs != self._knobs:
                    self._replays.clear()
                    self._knobs = knobs
            record = (out_dtype, softmax_scale, softmax_mode, appended, k_split_rows)
            rp = self._replays.get(scale_ind)
            if rp is not None and rp.args == record:
                out = rp.run(self, q, k, v)
                if out is not None:
                    return out
            if not q.is_cuda or _capturing():
                record = None  # record eager GPU steps only
        if appended and not self.active:
            raise RuntimeError("appended=True needs an active slab (see producer_append)")
        if self.logical_len == 0:
            self.k_split_rows = bool(k_split_rows)
        elif bool(k_split_rows) != self.k_split_rows:
            raise ValueError("k_split_rows must be the same for every step of a generation "
                             f"(cache holds {'split' if self.k_split_rows else 'plain'} K rows)")
        mode = fused_softmax_mode() if softmax_mode is None else softmax_mode
        final = scale_ind + 1 >= self.num_scales
        old_len = self.logical_len
        logical = old_len + int(k.shape[2])

        if baseline_prefix_enabled() and not self.active and not has_removed(self.removed(scale_ind)):
            # dense prefix (:1972-2038)
            if self.dense_buf is not None or (old_len == 0 and self._in_place_ok(q, k, v)):
                return self._dense_step_in_place(q, k, v, scale_ind, softmax_scale, mode, out_dtype, final,
                                                 record)
            with prof.phase("attention"):
                out = self._attend_dense(q, k, v, softmax_scale, mode, out_dtype)
            if final:
                self.reset()
                return out
            with prof.phase("materialize"):
                if self.cached_k is None or old_len == 0:
                    dense_k, dense_v = k.contiguous(), v.contiguous()
                else:
                    dense_k, dense_v = concat_kv(self.cached_k, k, self.cached_v, v)
                    prof.stat_add("dense_attention_cat_calls")
            self.logical_len = logical
            if has_removed(self.removed(scale_ind + 1)):
                with prof.phase("compact"):
                    self._activate_from_dense(dense_k, dense_v, scale_ind + 1)
            else:
                self.cached_k, self.cached_v = dense_k, dense_v
            return out

        dense_candidate = None
        fused = False
        bound = None
        if old_len == 0:
            with prof.phase("attention"):
                out = self._attend_dense(q, k, v, softmax_scale, mode, out_dtype)
        elif not self.active and not has_removed(self.removed(scale_ind)):
            with prof.phase("attention"):
                out = self._attend_dense(q, k, v, softmax_scale, mode, out_dtype)
            with prof.phase("materialize"):
                dense_candidate = concat_kv(self.cached_k, k, self.cached_v, v)
                prof.stat_add("dense_attention_cat_calls")
        else:
            was_active = self.active
            with prof.phase("materialize"):
                if not self.active:
                    self._activate_from_dense(self.cached_k, self.cached_v, scale_ind)
                starts, ends, counts = self.schedule.device_tables(scale_ind, q.device)
                plan = (self.schedule.device_work_plan(scale_ind, q.device, int(q.shape[0]), int(q.shape[2]),
                                                       build=not _capturing(),
                                                       item_shape=attention_item_shape(
                                                           q.dtype, k.dtype, v.dtype,
                                                           k_split_rows=self.k_split_rows, device=q.device))
                        if work_plans_enabled(q.device) else None)
                offsets = None if final or appended else self._fused_append_offsets(scale_ind, q, k, v)
                fused = offsets is not None
            kw = dict(q=q, persisted_k=self.cached_k, persisted_v=self.cached_v,
                      segment_starts=starts, segment_ends=ends, segment_counts=counts,
                      current_k=k, current_v=v, softmax_scale=softmax_scale, softmax_mode=mode,
                      out_dtype=out_dtype, work_plan=plan, append_offsets=offsets,
                      k_split_rows=self.k_split_rows)
            with prof.phase("attention"):
                if record is not None and was_active:
                    out, bound = BoundSegmentedAttention.bind(**kw)
                else:
                    out = fused_real_pruning_flat_segmented_attention(**kw)

        with prof.phase("compact"):
            if final:
                self.reset()
                if bound is not None:
                    self._replays[scale_ind] = _StepReplay(record, "slab", bound, old_len, logical, True)
                return out
            nxt = self.removed(scale_ind + 1)
            if not self.active and not has_removed(nxt):
                if dense_candidate is not None:
                    self.cached_k, self.cached_v = dense_candidate
                elif self.cached_k is None or old_len == 0:
                    self.cached_k, self.cached_v = k.contiguous(), v.contiguous()
                else:
                    self.cached_k, self.cached_v = concat_kv(self.cached_k, k, self.cached_v, v)
            elif self.active:
                # append the current scale's kept heads (:969-995)
                prof.stat_add("static_append_current_calls")
                if appended or fused:
                    # the producer or the attention launch wrote the offered heads
                    _, plan = self.schedule.fused_append(int(scale_ind), k.device)
                    tag = ("append_rest", int(scale_ind))
                else:
                    plan = self.schedule.append_plans.get((int(scale_ind), int(scale_ind) + 1))
                    tag = ("append", int(scale_ind))
                if plan is not None:
                    self._copy(plan, k, v, tag)
                if bound is not None:
                    self._replays[scale_ind] = _StepReplay(
                        record, "slab", bound, old_len, logical, False,
                        copy=(plan, tag) if plan is not None and len(plan) > 0 else None)
            else:
                # pack the dense cache and the current scale into a new slab (:1713-1789)
                dense_k, dense_v = self.cached_k, self.cached_v
                self._ensure_slab(k.shape[0], k.shape[3], k.device, k.dtype, v.dtype)
                self.active = True
                old_plan, cur_plan = self._dense_and_current_plans(
                    scale_ind + 1, scale_ind, old_len, int(k.shape[2]))
                if dense_k is not None and old_len > 0:
                    self._copy(old_plan, dense_k, dense_v, ("dense_old", scale_ind + 1, old_len))
                self._copy(cur_plan, k, v, ("dense_cur", scale_ind + 1, int(k.shape[2])))
        self.logical_len = logical
        return out
