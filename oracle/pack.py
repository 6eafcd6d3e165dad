"""numpy restatement of the slab pack/append copy (test infrastructure only).

Follows ``_pack_flat_segments_kv_kernel`` (real_pruning_fused_attention.py:33-73):
for every copy item ``i`` and batch row ``b``

    dst[b, dst_starts[i] + t, :] = src[b, src_starts[i] + t, :]   for t < lengths[i]

for K and for V; rows outside the items are left untouched (masked stores).
The source is the flat ``[B, H * n, D]`` view of ``[B, H, n, D]`` current K/V
(enable_real_pruning_fast.py:773-775), so ``src_starts[i] = head * n + start``.

Pinning: the result is a byte copy, so tests compare it against direct slicing
of the per-head source (``src[b, h, start:start+len]``) through
``expected_live_rows`` and check that bytes outside every destination item are
unchanged.
"""

from __future__ import annotations


def pack_flat_segments(dst, src, dst_starts, src_starts, lengths):
    """In-place copy into ``dst`` ``[B, C, D]`` from ``src`` ``[B, S, D]``; returns ``dst``."""
    for d0, s0, n in zip(dst_starts, src_starts, lengths):
        d0 = int(d0)
        s0 = int(s0)
        n = int(n)
        if n <= 0:
            continue
        dst[:, d0 : d0 + n, :] = src[:, s0 : s0 + n, :]
    return dst


def expected_live_rows(dense, segments, target, scale_ranges):
    """``{(source, head): rows}`` that the slab must hold at ``target``.

    ``dense`` is the ``[B, H, T, D]`` cache of every scale's K (or V) in token
    order; a live segment (``start_target <= target < end_target``) of
    (source s, head h) must hold ``dense[:, h, range(s), :]`` at its offset.
    """
    out = {}
    for seg in segments:
        if not (seg["start_target"] <= target < seg["end_target"]):
            continue
        a, b = scale_ranges[seg["source_scale"]]
        out[(seg["source_scale"], seg["head"])] = (int(seg["offset"]), dense[:, seg["head"], a:b, :])
    return out
