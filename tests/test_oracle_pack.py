"""Pins the pack oracle (oracle/pack.py) against checks independent of its code.

* element-by-element brute force of the copy rule of
  _pack_flat_segments_kv_kernel (real_pruning_fused_attention.py:48-73):
  dst[b, dst_start + t, d] = src[b, src_start + t, d] for t < length;
* rows outside every destination item keep their bytes;
* ``expected_live_rows`` against per-head slicing of the dense cache;
* a planted off-by-one in the oracle's destination fails the brute force.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import pack as opack


def _brute(dst, src, dst_starts, src_starts, lengths):
    out = dst.copy()
    B, _, D = src.shape
    for d0, s0, n in zip(dst_starts, src_starts, lengths):
        for b in range(B):
            for t in range(int(n)):
                for d in range(D):
                    out[b, int(d0) + t, d] = src[b, int(s0) + t, d]
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_pack_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    B, S, C, D = 2, 40, 60, 5
    src = rng.standard_normal((B, S, D)).astype(np.float32)
    dst = rng.standard_normal((B, C, D)).astype(np.float32)
    lengths = [0, 3, 7, 1, 5]
    src_starts = [int(rng.integers(0, S - n + 1)) for n in lengths]
    dst_starts = [2, 4, 12, 30, 41]  # disjoint destinations, unaligned
    got = opack.pack_flat_segments(dst.copy(), src, dst_starts, src_starts, lengths)
    assert np.array_equal(got, _brute(dst, src, dst_starts, src_starts, lengths))
    owned = np.zeros(C, bool)
    for d0, n in zip(dst_starts, lengths):
        owned[d0:d0 + n] = True
    assert np.array_equal(got[:, ~owned], dst[:, ~owned])


def test_planted_off_by_one_is_caught(monkeypatch):
    rng = np.random.default_rng(3)
    src = rng.standard_normal((1, 20, 3)).astype(np.float32)
    dst = np.zeros((1, 30, 3), np.float32)
    args = ([5], [2], [4])

    def shifted(dst_, src_, dst_starts, src_starts, lengths):
        for d0, s0, n in zip(dst_starts, src_starts, lengths):
            dst_[:, d0 + 1:d0 + 1 + n] = src_[:, s0:s0 + n]
        return dst_

    monkeypatch.setattr(opack, "pack_flat_segments", shifted)
    got = opack.pack_flat_segments(dst.copy(), src, *args)
    assert not np.array_equal(got, _brute(dst, src, *args))


def test_expected_live_rows_slices_the_dense_cache():
    rng = np.random.default_rng(4)
    ranges = {0: (0, 1), 1: (1, 5), 2: (5, 21)}
    dense = rng.standard_normal((2, 3, 21, 4)).astype(np.float32)
    segs = [
        dict(source_scale=1, head=2, start_target=2, end_target=3, offset=7),
        dict(source_scale=0, head=0, start_target=1, end_target=3, offset=0),
        dict(source_scale=2, head=1, start_target=3, end_target=3, offset=50),  # never live
    ]
    live = opack.expected_live_rows(dense, segs, 2, ranges)
    assert set(live) == {(1, 2), (0, 0)}
    off, rows = live[(1, 2)]
    assert off == 7 and np.array_equal(rows, dense[:, 2, 1:5])
    off, rows = live[(0, 0)]
    assert off == 0 and np.array_equal(rows, dense[:, 0, 0:1])
