"""GPU: the round split of the 16-bit attention kernel.

With a workspace (the Python operator passes one unless HKV_ATTN_SPLIT=0),
launches with fewer than two rounds of items per CU slot cut some (batch,
head, 128-query tile) items into two parts of their key-tile stream, the
heaviest ones first (between one and two rounds: 2G - N of them, with the
whole items issued before the parts; at most one round: min(N, G - N)); the
part that completes an item last merges both parts' partial records.  An item with fewer than 16 key tiles runs whole
(its second part leaves at once).  The parts of a cut item are adjacent
workgroups when the current scale alone gives every item 16 tiles, else all
first parts precede all second parts.  These cases cover merges of long and
short items, short items whose second part leaves, every item cut (grouped
parts), a mix of cut and whole-running items, a second round made of cut
items (adjacent parts), workspace reuse and determinism, against the oracle
and against the uncut mode (HKV_ATTN_SPLIT=0, no workspace).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import fused_real_pruning_flat_segmented_attention
from heatkv_amd import workloads as W
from oracle import segmented_attention as oattn
from support import assert_attention_close, bits, to_np

pytestmark = pytest.mark.gpu


def _slots(device):
    return 2 * torch.cuda.get_device_properties(device).multi_processor_count


def _call(q, sk, sv, st, en, ct, ck, cv, scale):
    out, lse = fused_real_pruning_flat_segmented_attention(
        q=q, persisted_k=sk, persisted_v=sv, segment_starts=st, segment_ends=en,
        segment_counts=ct, current_k=ck, current_v=cv, softmax_scale=scale, return_lse=True)
    torch.cuda.synchronize(q.device)
    return out, lse


def _both_modes(monkeypatch, args):
    monkeypatch.setenv("HKV_ATTN_SPLIT", "1")
    cut = _call(*args)
    cut2 = _call(*args)  # the workspace is reused: its counters must be back at zero
    monkeypatch.setenv("HKV_ATTN_SPLIT", "0")
    whole = _call(*args)
    (o1, l1), (o2, l2) = cut, cut2
    # deterministic: parts merge in part order whichever finishes last
    assert np.array_equal(bits(o1), bits(o2)) and np.array_equal(bits(l1), bits(l2))
    return cut, whole


def _dev(device, *ts):
    return [None if t is None else t.to(device) for t in ts]


def _check_vs_oracle(q, sk, sv, st, en, ct, ck, cv, scale, results, heads=None):
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), st.numpy(), en.numpy(), ct.numpy(), to_np(ck), to_np(cv),
        scale, heads=heads)
    D = q.shape[-1]
    hs = range(q.shape[1]) if heads is None else heads
    for (o, l), what in results:
        o, l = to_np(o), to_np(l)
        for h in hs:
            assert_attention_close(o[:, :, h * D:(h + 1) * D], l[:, h], ref_out[:, :, h * D:(h + 1) * D],
                                   ref_lse[:, h], what=f"{what} h={h}")


def test_config2_cut_matches_whole_items(device, monkeypatch):
    wl = W.config(2)
    items = wl.batch * wl.heads * math.ceil(wl.cur_len / 128)
    print(f"[split] config 2 items={items} slots={_slots(device)}", flush=True)
    slab_k, slab_v = W.build_slab(wl, device)
    args = (*_dev(device, wl.q), slab_k, slab_v, *_dev(device, *wl.tables()),
            *_dev(device, wl.cur_k, wl.cur_v), wl.softmax_scale)
    (o1, l1), (ow, lw) = _both_modes(monkeypatch, args)
    # the two modes differ only by the rounding of the merged statistics
    assert_attention_close(to_np(o1), to_np(l1), to_np(ow), to_np(lw), max_abs=2e-2, mean_abs=5e-4,
                           lse_abs=1e-4, what="cut vs whole items")


def test_every_item_cut_long_keys(device, monkeypatch):
    """8 items (fewer than slots): every item cut in two, each over thousands
    of retained rows in several segments."""
    B, H, L = 1, 8, 128
    cap = 5000 * 8
    print(f"[split] every item cut H={H} cap={cap}", flush=True)
    g = torch.Generator().manual_seed(51)
    q, ck, cv = (torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    sk = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    sv = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    S = 3
    st = torch.zeros((H, S), dtype=torch.int32)
    en = torch.zeros((H, S), dtype=torch.int32)
    ct = torch.full((H,), S, dtype=torch.int32)
    for h in range(H):  # head h keeps about 5000 (h + 1) rows in 3 unaligned segments
        n = 5000 * (h + 1) - 7 * h
        cuts = [0, n // 3 + h, 2 * n // 3 - h, n]
        base = int(torch.randint(0, cap - n + 1, (1,), generator=g))
        for i in range(S):
            st[h, i], en[h, i] = base + cuts[i], base + cuts[i + 1]
    scale = 1.0 / math.sqrt(128)
    args = (*_dev(device, q, sk, sv, st, en, ct, ck, cv), scale)
    cut, whole = _both_modes(monkeypatch, args)
    _check_vs_oracle(q, sk, sv, st, en, ct, ck, cv, scale, [(cut, "cut"), (whole, "whole")])


@pytest.mark.parametrize("L", [1, 70])
def test_items_shorter_than_their_parts(device, monkeypatch, L):
    """Items of one to three tiles: too short for two parts, so the second
    part of each leaves and the first runs the item whole."""
    B, H, cap, S = 2, 20, 400, 3
    print(f"[split] short items H={H} L={L}", flush=True)
    g = torch.Generator().manual_seed(53 + L)
    q, ck, cv = (torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    sk = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    sv = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    st = torch.randint(0, cap, (H, S), generator=g, dtype=torch.int32)
    en = torch.clamp(st + torch.randint(-2, 90, (H, S), generator=g, dtype=torch.int32), max=cap)
    ct = torch.randint(0, S + 1, (H,), generator=g, dtype=torch.int32)
    scale = 0.07
    args = (*_dev(device, q, sk, sv, st, en, ct, ck, cv), scale)
    cut, whole = _both_modes(monkeypatch, args)
    _check_vs_oracle(q, sk, sv, st, en, ct, ck, cv, scale, [(cut, "cut"), (whole, "whole")])


def test_items_just_above_slots(device, monkeypatch):
    """slots + 3 items: the slots - 3 heaviest cut in two, the 6 lightest run
    whole first; heads of mixed retained length."""
    H = _slots(device) + 3
    B, L, cap, S = 1, 100, 3000, 2
    print(f"[split] items just above slots H={H}", flush=True)
    g = torch.Generator().manual_seed(57)
    q, ck, cv = (torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    sk = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    sv = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    st = torch.randint(0, cap // 2, (H, S), generator=g, dtype=torch.int32)
    en = st + torch.randint(0, 1400, (H, S), generator=g, dtype=torch.int32)
    ct = torch.randint(0, S + 1, (H,), generator=g, dtype=torch.int32)
    scale = 0.09
    args = (*_dev(device, q, sk, sv, st, en, ct, ck, cv), scale)
    cut, whole = _both_modes(monkeypatch, args)
    rows = [sum(max(0, int(en[h, i]) - int(st[h, i])) for i in range(int(ct[h]))) for h in range(H)]
    order = sorted(range(H), key=lambda h: (-rows[h], h))
    heads = sorted({order[0], order[1], order[2], order[3], order[H // 2], order[-2], order[-1]})
    _check_vs_oracle(q, sk, sv, st, en, ct, ck, cv, scale, [(cut, "cut"), (whole, "whole")], heads=heads)


def test_config5_batches_cut(device, monkeypatch):
    """Skewed retained lengths, batch 16: two full batch rows against the oracle."""
    monkeypatch.setenv("HKV_ATTN_SPLIT", "1")
    wl = W.config(5)
    print("[split] config 5 batches 3, 12", flush=True)
    slab_k, slab_v = W.build_slab(wl, device)
    out, lse = _call(*_dev(device, wl.q), slab_k, slab_v, *_dev(device, *wl.tables()),
                     *_dev(device, wl.cur_k, wl.cur_v), wl.softmax_scale)
    st, en, ct = (t.numpy() for t in wl.tables())
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(wl.q), to_np(slab_k), to_np(slab_v), st, en, ct, to_np(wl.cur_k), to_np(wl.cur_v),
        wl.softmax_scale, batches=[3, 12])
    o, l = to_np(out), to_np(lse)
    for b in (3, 12):
        assert_attention_close(o[b], l[b], ref_out[b], ref_lse[b], what=f"config 5 b={b}")


def test_second_round_of_cut_items(device, monkeypatch):
    """The 2B shape of scale 11 (L = 2304: 576 items for 512 slots on a 256-CU
    device): the 448 heaviest items are cut, so the second round is made of
    halves."""
    B, H, L, cap, S = 2, 16, 2304, 6425, 9
    print(f"[split] second round B={B} H={H} L={L}", flush=True)
    g = torch.Generator().manual_seed(61)
    q, ck, cv = (torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    sk = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    sv = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16)
    st = torch.randint(0, cap - 600, (H, S), generator=g, dtype=torch.int32)
    en = st + torch.randint(0, 600, (H, S), generator=g, dtype=torch.int32)
    ct = torch.randint(0, S + 1, (H,), generator=g, dtype=torch.int32)
    scale = 1.0 / math.sqrt(128)
    args = (*_dev(device, q, sk, sv, st, en, ct, ck, cv), scale)
    cut, whole = _both_modes(monkeypatch, args)
    rows = [sum(max(0, int(en[h, i]) - int(st[h, i])) for i in range(int(ct[h]))) for h in range(H)]
    order = sorted(range(H), key=lambda h: (-rows[h], h))
    heads = sorted({order[0], order[7], order[-1]})
    _check_vs_oracle(q, sk, sv, st, en, ct, ck, cv, scale, [(cut, "cut"), (whole, "whole")], heads=heads)
