"""numpy restatement of the reference CPU attention path (test infrastructure only).

Follows ``_flat_segmented_attention_reference``
(real_pruning_fused_attention.py:312-361):

* for every (batch b, head h) the keys are the slab rows of head h's segments in
  table order (``segment_starts[h, i] .. segment_ends[h, i]`` for
  ``i < segment_counts[h]``), skipping entries with ``start >= end``
  (:341-346), followed by the current-scale rows ``current_k[b, h]`` (:347-348);
* ``softmax(scale * q k^T) v`` with no mask (:353-359, SDPA with ``scale=``);
* the output is laid out ``[B, L, H * D]`` (:361).

The reference returns no log-sum-exp; this restatement adds
``lse[b, h, l] = logsumexp_j(scale * q_l . k_j)`` (natural log) because the
tolerance contract names one.

Pinning (tests/test_oracle_attention.py): brute-force pure-Python loops on tiny
shapes, ``torch.nn.functional.scaled_dot_product_attention`` (the library
routine the reference calls) on every (b, h), closed forms (identical keys ->
mean of values; one key -> that value), and invariance under segment
permutation and slab relocation.
"""

from __future__ import annotations

import numpy as np


def gather_head_keys(slab, starts, ends, counts, head, batch):
    """Rows of ``slab[batch]`` that head ``head`` attends to, in table order.

    Mirrors real_pruning_fused_attention.py:338-346 (``start >= end`` skipped).
    Returns ``(rows, index_list)`` where ``index_list`` is the list of slab row
    indices, useful for the loaders' tests.
    """
    n = int(counts[head])
    idx = []
    for i in range(n):
        s = int(starts[head, i])
        e = int(ends[head, i])
        if s >= e:
            continue
        idx.extend(range(s, e))
    idx = np.asarray(idx, dtype=np.int64)
    if slab is None:
        return None, idx
    return slab[batch, idx, :], idx


def flat_segmented_attention(
    q,
    slab_k,
    slab_v,
    starts,
    ends,
    counts,
    cur_k,
    cur_v,
    softmax_scale,
    *,
    dtype=np.float32,
    heads=None,
    batches=None,
    workers=1,
):
    """Segmented attention over a flat slab + current keys.

    Arguments are numpy arrays: ``q``, ``cur_k``, ``cur_v`` ``[B, H, L, D]``;
    ``slab_k``, ``slab_v`` ``[B, C, D]`` (``C`` may be 0, or ``None`` meaning
    empty as in :327-331); ``starts``, ``ends`` ``[H, S]``; ``counts`` ``[H]``.

    Returns ``(out [B, L, H*D], lse [B, H, L])`` in ``dtype`` (fp32 by default,
    fp64 when a tighter reference is wanted).  ``heads``/``batches`` restrict
    the work to a subset (the unlisted outputs are left NaN); used by the
    bounded CPU-baseline sample.  ``workers > 1`` runs the (b, h) pairs on a
    thread pool (numpy's matmul and exp release the GIL); every pair is the
    same arithmetic either way, so the result does not depend on it.
    """
    q = np.asarray(q, dtype=dtype)
    cur_k = np.asarray(cur_k, dtype=dtype)
    cur_v = np.asarray(cur_v, dtype=dtype)
    B, H, L, D = q.shape
    if slab_k is None or slab_v is None:
        slab_k = np.zeros((B, 0, D), dtype=dtype)
        slab_v = np.zeros((B, 0, D), dtype=dtype)
    slab_k = np.asarray(slab_k)
    slab_v = np.asarray(slab_v)
    starts = np.asarray(starts)
    ends = np.asarray(ends)
    counts = np.asarray(counts)
    out = np.full((B, L, H * D), np.nan, dtype=dtype)
    lse = np.full((B, H, L), np.nan, dtype=dtype)
    scale = dtype(softmax_scale)
    head_list = range(H) if heads is None else heads
    batch_list = range(B) if batches is None else batches

    def one(h, idx, b):
        keys = np.concatenate([slab_k[b, idx, :].astype(dtype), cur_k[b, h]], axis=0)
        vals = np.concatenate([slab_v[b, idx, :].astype(dtype), cur_v[b, h]], axis=0)
        s = (q[b, h] @ keys.T) * scale  # [L, N]
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(axis=1, keepdims=True)
        o = (p @ vals) / l
        out[b, :, h * D : (h + 1) * D] = o
        lse[b, h, :] = (m + np.log(l))[:, 0]

    pairs = []
    for h in head_list:
        _, idx = gather_head_keys(None, starts, ends, counts, h, 0)
        pairs.extend((h, idx, b) for b in batch_list)
    if workers > 1 and len(pairs) > 1:
        from concurrent.futures import ThreadPoolExecutor

        with ThreadPoolExecutor(max_workers=int(workers)) as ex:
            for f in [ex.submit(one, *p) for p in pairs]:
                f.result()
    else:
        for p in pairs:
            one(*p)
    return out, lse


def brute_force_attention(q_rows, keys, vals, softmax_scale):
    """Pure-Python double loop for tiny cases (pins ``flat_segmented_attention``).

    ``q_rows`` is a list of query vectors, ``keys``/``vals`` lists of key/value
    vectors.  Returns ``(outputs, lses)`` as Python floats, computed in double
    precision with the textbook definition (no max subtraction shortcut beyond
    the standard one, which cancels exactly in exact arithmetic).
    """
    import math

    outs = []
    lses = []
    for qv in q_rows:
        scores = [softmax_scale * sum(a * b for a, b in zip(qv, kv)) for kv in keys]
        mx = max(scores)
        w = [math.exp(s - mx) for s in scores]
        tot = sum(w)
        outs.append(
            [sum(w[j] * vals[j][d] for j in range(len(keys))) / tot for d in range(len(vals[0]))]
        )
        lses.append(mx + math.log(tot))
    return outs, lses


def attention_flops(counts, starts, ends, batch, cur_len, head_dim):
    """Algorithmic FLOPs of one call: sum over (b, h) of 4 * L * (R_h + L) * D.

    R_h counts retained prior rows (segments with start < end).  Tile padding
    and masked lanes are not counted.
    """
    H = len(counts)
    total = 0
    for h in range(H):
        _, idx = gather_head_keys(None, starts, ends, counts, h, 0)
        total += 4 * cur_len * (len(idx) + cur_len) * head_dim
    return batch * total


def flat_segmented_attention_sdpa(q, slab_k, slab_v, starts, ends, counts, cur_k, cur_v, softmax_scale):
    """torch restatement of the reference CPU path, as it is written there.

    ``_flat_segmented_attention_reference`` (real_pruning_fused_attention.py:
    312-361): for every (b, h) gather head h's slab segments in table order
    (entries with ``start >= end`` skipped), append the current K/V, and call
    ``torch.nn.functional.scaled_dot_product_attention(..., scale=softmax_scale)``;
    output ``[B, L, H * D]``.  Inputs are torch CPU tensors, computed in fp32
    (the inputs are upcast first).  Used as the timed CPU baseline; pinned
    against :func:`flat_segmented_attention` in tests/test_oracle_attention.py.
    """
    import torch
    import torch.nn.functional as F

    q = q.float()
    cur_k = cur_k.float()
    cur_v = cur_v.float()
    B, H, L, D = q.shape
    if slab_k is None or slab_v is None:
        slab_k = q.new_zeros((B, 0, D))
        slab_v = q.new_zeros((B, 0, D))
    slab_k = slab_k.float()
    slab_v = slab_v.float()
    out = q.new_empty((B, L, H * D))
    for h in range(H):
        _, idx = gather_head_keys(None, np.asarray(starts), np.asarray(ends), np.asarray(counts), h, 0)
        index = torch.from_numpy(idx)
        keys = torch.cat([slab_k.index_select(1, index), cur_k[:, h]], dim=1)  # [B, N, D]
        vals = torch.cat([slab_v.index_select(1, index), cur_v[:, h]], dim=1)
        o = F.scaled_dot_product_attention(q[:, h:h + 1], keys[:, None], vals[:, None], scale=softmax_scale)
        out[:, :, h * D:(h + 1) * D] = o[:, 0]
    return out
