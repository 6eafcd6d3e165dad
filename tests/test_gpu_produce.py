"""GPU parity of the QKV producer (hkv_qkv_produce) and of the layer forward built on it.

* Kernel against the oracle (oracle/produce.py, pinned by
  tests/test_oracle_produce.py) at the 2B shapes: q within 4e-6 * scale_mul[h]
  and k within 4e-6 absolute (fp32; the squared norm is summed in another
  order, a few ulp), v bit-exact; bf16 q/k outputs within one bf16 rounding of
  the oracle's fp32 values.
* Fused append: slab rows bit-exact equal to the produced k/v rows, nothing
  else written; a whole 13-scale generation under the reference's HeatKV
  policy (orders/2b.json, budget 0.1) with the producer appending ahead of
  attention gives bit-identical outputs and slabs to the unfused path.
* Patched layer forward (Infinity SelfAttention attributes, bf16 autocast):
  the attention output entering the output projection against fp32 attention
  over the oracle's q/k/v of the same projection, over the keys the policy
  keeps, within the attention tolerances.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

from heatkv_amd import policy as POL
from heatkv_amd import produce as P
from heatkv_amd import segmented_cache as sc
from heatkv_amd.enable import enable_real_pruning_scale_specific_fused_segmented
from heatkv_amd.harness import seeded_orders
from heatkv_amd.slab_schedule import SIDES_1M, build_static_slot_schedule
from oracle import produce as O
from oracle import segmented_attention as oattn
from support import SelfAttention, assert_attention_close, bits, to_np

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
SCHED_1M = [(1, s, s) for s in SIDES_1M]
D = 128


def _qkv(B, L, H, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn((B, L, 3 * H * D), generator=g) * 2).to(torch.bfloat16)


def _scale_mul(H, seed):
    g = torch.Generator().manual_seed(seed)
    raw = torch.rand(H, generator=g) * 5.0  # log-scale values, some above log(100)
    return raw.clamp_max(math.log(100)).exp()


def _check_qk(got_q, got_k, want_q, want_k, sm, H):
    gq, gk = to_np(got_q.float()), to_np(got_k.float())
    for h in range(H):
        err_q = np.max(np.abs(gq[:, h] - want_q[:, h]))
        assert err_q <= 4e-6 * float(sm[h]), (h, err_q)
    err_k = np.max(np.abs(gk - want_k))
    assert err_k <= 4e-6, err_k


@pytest.mark.parametrize("scale_ind,B,H", [(12, 2, 16), (11, 2, 16), (0, 2, 16), (1, 1, 3), (6, 4, 24), (9, 2, 16)])
def test_producer_against_oracle(device, scale_ind, B, H):
    side = SIDES_1M[scale_ind]
    L = side * side
    print(f"[produce] scale {scale_ind} B {B} L {L} H {H}", flush=True)
    qkv = _qkv(B, L, H, 10 + scale_ind)
    sm = _scale_mul(H, 20 + scale_ind)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128)
    start = P.rope_start(SCHED_1M, scale_ind)
    q, k, v = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                            rope_start_row=start)
    torch.cuda.synchronize(device)
    assert q.dtype == k.dtype == torch.float32 and v.dtype == torch.bfloat16
    assert tuple(q.shape) == (B, H, L, D)
    wq, wk, wv = O.produce(qkv.float().numpy().reshape(B, L, 3, H, D), scale_mul=sm.numpy(), table=table.numpy(),
                           start=start)
    _check_qk(q, k, wq, wk, sm, H)
    assert np.array_equal(to_np(v.float()), wv)


def test_producer_bias_no_normalize_and_bf16_out(device):
    B, L, H = 2, 576, 16
    qkv = _qkv(B, L, H, 3)
    g = torch.Generator().manual_seed(4)
    qb = torch.randn(H * D, generator=g)
    vb = torch.randn(H * D, generator=g)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128)
    start = P.rope_start(SCHED_1M, 8)
    arr = qkv.float().numpy().reshape(B, L, 3, H, D)
    # fused biases, cosine normalization on
    q, k, v = P.qkv_produce(qkv.to(device), H, rope_table=table.to(device), rope_start_row=start,
                            q_bias=qb.to(device), v_bias=vb.to(device))
    wq, wk, wv = O.produce(arr, table=table.numpy(), start=start, q_bias=qb.numpy(), v_bias=vb.numpy())
    _check_qk(q, k, wq, wk, np.ones(H), H)
    assert np.array_equal(to_np(v.float()), wv)
    # no normalization (non-cosine attention): rotation of the raw values
    q, k, _ = P.qkv_produce(qkv.to(device), H, rope_table=table.to(device), rope_start_row=start, normalize=False)
    wq, wk, _ = O.produce(arr, table=table.numpy(), start=start, normalize=False)
    assert np.array_equal(to_np(q), wq) and np.array_equal(to_np(k), wk)
    # bf16 q/k outputs: one bf16 rounding (at most 2^-8 relative) of a value
    # within the fp32 tolerance of the oracle's; nearly all equal the oracle's
    # value rounded
    sm = _scale_mul(H, 5)
    q, k, _ = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                            rope_start_row=start, qk_dtype=torch.bfloat16)
    wq, wk, _ = O.produce(arr, scale_mul=sm.numpy(), table=table.numpy(), start=start)
    for got, want, atol in ((q, wq, 4e-6 * sm.numpy()[None, :, None, None]), (k, wk, 4e-6)):
        g32 = to_np(got.float())
        assert np.mean(g32 != O.bf16_round(want)) < 1e-3
        assert np.all(np.abs(g32 - want) <= np.abs(want) * 2.0 ** -8 + atol)
    # fp16 q/k outputs (TF32's significand): one fp16 rounding (2^-11 relative)
    q, k, _ = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                            rope_start_row=start, qk_dtype=torch.float16)
    assert q.dtype == k.dtype == torch.float16
    for got, want, atol in ((q, wq, 4e-6 * sm.numpy()[None, :, None, None]), (k, wk, 4e-6)):
        g32 = to_np(got.float())
        assert np.mean(g32 != want.astype(np.float16).astype(np.float32)) < 1e-3
        # 2^-11 relative rounding, or half the subnormal spacing 2^-25 below 2^-14
        assert np.all(np.abs(g32 - want) <= np.abs(want) * 2.0 ** -11 + 2.0 ** -25 + atol)


@pytest.mark.parametrize("proj", [torch.float16, torch.float32])
def test_producer_fp16_fp32_projection(device, proj):
    """fp16 (fp16 autocast) and fp32 (no autocast) projections: q, k against
    the oracle as for bf16, v keeps the projection's dtype and values
    (bit-exact; with v_bias rounded once to that dtype), the appended slab
    rows equal the outputs; fp32 k as split rows is the split of the fp32 k."""
    B, L, H, cap = 2, 400, 8, 900
    g = torch.Generator().manual_seed(21)
    qkv = (torch.randn((B, L, 3 * H * D), generator=g) * 2).to(proj)
    vb = torch.randn(H * D, generator=g)
    sm = _scale_mul(H, 22)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128)
    start = P.rope_start(SCHED_1M, 9)
    arr = qkv.float().numpy().reshape(B, L, 3, H, D)
    vt = "fp16" if proj == torch.float16 else "fp32"
    slab_k = torch.zeros((B, cap, D), device=device)
    slab_v = torch.zeros((B, cap, D), device=device, dtype=proj)
    offs = torch.tensor([0, -1, 400, -1, -1, -1, -1, 850], dtype=torch.int32, device=device)
    q, k, v = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                            rope_start_row=start, v_bias=vb.to(device), append=(slab_k, slab_v, offs))
    wq, wk, wv = O.produce(arr, scale_mul=sm.numpy(), table=table.numpy(), start=start, v_bias=vb.numpy(),
                           v_type=vt)
    assert v.dtype == proj
    _check_qk(q, k, wq, wk, sm.numpy(), H)
    assert np.array_equal(to_np(v.float()), wv)
    for h, off in ((0, 0), (2, 400), (7, 850)):
        n = min(L, cap - off)
        assert torch.equal(slab_k[:, off:off + n], k[:, h, :n]) and torch.equal(slab_v[:, off:off + n], v[:, h, :n])
    # no bias: v is the projection's v, bit for bit
    _, k2, v2 = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                              rope_start_row=start)
    assert np.array_equal(bits(v2), bits(qkv.reshape(B, L, 3, H, D)[:, :, 2].permute(0, 2, 1, 3).contiguous()))
    _, ks, _ = P.qkv_produce(qkv.to(device), H, scale_mul=sm.to(device), rope_table=table.to(device),
                             rope_start_row=start, k_split_rows=True)
    assert np.array_equal(bits(ks), bits(_split(k2)))


def test_producer_zero_rows_5d_input_and_empty(device):
    B, L, H = 1, 16, 2
    qkv = _qkv(B, L, H, 6).reshape(B, L, 3, H, D)
    qkv[0, 3, 0, 1] = 0  # a zero q row: 0 / eps = 0
    qkv[0, 5, 1, 0] = 0  # a zero k row
    q, k, _ = P.qkv_produce(qkv.to(device), H)
    assert torch.all(q[0, 1, 3] == 0) and torch.all(k[0, 0, 5] == 0)
    wq, wk, _ = O.produce(qkv.float().numpy())
    _check_qk(q, k, wq, wk, np.ones(H), H)
    q, k, v = P.qkv_produce(torch.empty((2, 0, 3 * H * D), dtype=torch.bfloat16, device=device), H)
    assert q.shape == (2, H, 0, D) and v.shape == (2, H, 0, D)


def test_producer_append_rows(device):
    B, L, H, cap = 2, 144, 6, 1000
    qkv = _qkv(B, L, H, 7).to(device)
    sm = _scale_mul(H, 8).to(device)
    slab_k = torch.full((B, cap, D), 7.5, device=device)
    slab_v = torch.full((B, cap, D), -3.25, device=device, dtype=torch.bfloat16)
    # head 0 -> 0, head 2 -> 500, head 3 -> 900 (rows 900..999 fit, 44 rows fall
    # outside and are not written), head 5 -> 144; heads 1 and 4 not appended
    offs = torch.tensor([0, -1, 500, 900, -1, 144], dtype=torch.int32, device=device)
    q, k, v = P.qkv_produce(qkv, H, scale_mul=sm, append=(slab_k, slab_v, offs))
    q2, k2, v2 = P.qkv_produce(qkv, H, scale_mul=sm)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    sk, sv = bits(slab_k), bits(slab_v)
    written = np.zeros(cap, bool)
    for h, off in enumerate(offs.tolist()):
        if off < 0:
            continue
        n = min(L, cap - off)
        assert np.array_equal(sk[:, off:off + n], bits(k[:, h, :n])), h
        assert np.array_equal(sv[:, off:off + n], bits(v[:, h, :n])), h
        written[off:off + n] = True
    assert np.all(to_np(slab_k)[:, ~written] == 7.5)
    assert np.all(to_np(slab_v.float())[:, ~written] == -3.25)


def test_generation_with_fused_append_matches_unfused(device):
    """13-scale generation (B=2, H=16) under orders/2b.json at budget 0.1:
    producer + fused append + residual copy vs producer + full copy."""
    orders = json.load(open(os.path.join(HERE, "golden", "orders_2b.json")))
    ctrl = POL.controller_for_budget(0.1, orders, num_layers=32, num_heads=16, protected_prefix_scales=3)
    layer, H, B = 29, 16, 2
    sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
    removed = lambda t: ctrl.removed_heads_by_source_for(layer, t)  # noqa: E731
    fused = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    plain = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128).to(device)
    sm = _scale_mul(H, 9).to(device)
    n_fused = 0
    for t, side in enumerate(SIDES_1M):
        qkv = _qkv(B, side * side, H, 1000 + t).to(device)
        start = P.rope_start(SCHED_1M, t)
        app = fused.producer_append(t, torch.float32, device)
        n_fused += app is not None
        q, k, v = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start, append=app)
        out_f = fused.step(q, k, v, t, 1.0, appended=app is not None)
        q2, k2, v2 = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start)
        out_p = plain.step(q2, k2, v2, t, 1.0)
        torch.cuda.synchronize(device)
        print(f"[fused append] step {t} fused {app is not None}", flush=True)
        assert torch.equal(out_f, out_p), t
        if fused.active and t + 1 < len(SIDES_1M):
            for seg in sched.live_segments(t + 1):
                rows = slice(seg.offset, seg.offset + seg.length)
                assert torch.equal(fused.cached_k[:, rows], plain.cached_k[:, rows]), (t, seg)
                assert torch.equal(fused.cached_v[:, rows], plain.cached_v[:, rows]), (t, seg)
    assert n_fused >= 3


def _split(t: torch.Tensor) -> torch.Tensor:
    """hkv_split_rows of fp32 rows, viewed as float32 (the producer's split-row K form)."""
    from heatkv_amd.real_pruning_fused_attention import _split_rows

    return _split_rows(t.contiguous(), torch.cuda.current_stream(t.device)).view(torch.float32)


def test_producer_split_rows_k(device):
    """qkv_produce(k_split_rows=True): k's rows (and the appended slab rows)
    are bit for bit hkv_split_rows of the fp32 k the producer writes without
    it; q and v unchanged; slab rows not appended untouched."""
    B, L, H, cap = 2, 144, 6, 1000
    qkv = _qkv(B, L, H, 17).to(device)
    sm = _scale_mul(H, 18).to(device)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128).to(device)
    start = P.rope_start(SCHED_1M, 5)
    slab_k = torch.full((B, cap, D), 7.5, device=device)
    slab_v = torch.full((B, cap, D), -3.25, device=device, dtype=torch.bfloat16)
    offs = torch.tensor([0, -1, 500, 900, -1, 144], dtype=torch.int32, device=device)
    q, k, v = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start,
                            append=(slab_k, slab_v, offs), k_split_rows=True)
    q2, k2, v2 = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start)
    ks = _split(k2)
    torch.cuda.synchronize(device)
    assert k.dtype == torch.float32 and tuple(k.shape) == (B, H, L, D)
    assert torch.equal(q, q2) and torch.equal(v, v2)
    assert np.array_equal(bits(k), bits(ks))
    sk = bits(slab_k)
    written = np.zeros(cap, bool)
    for h, off in enumerate(offs.tolist()):
        if off < 0:
            continue
        n = min(L, cap - off)
        assert np.array_equal(sk[:, off:off + n], bits(ks[:, h, :n])), h
        written[off:off + n] = True
    assert np.all(to_np(slab_k)[:, ~written] == 7.5)
    with pytest.raises(ValueError, match="k_split_rows"):
        P.qkv_produce(qkv, H, qk_dtype=torch.bfloat16, k_split_rows=True)


def test_generation_split_rows_k_matches_fp32_k(device):
    """13-scale generation (B=2, H=16) under orders/2b.json at budget 0.1 at
    the model's precision (fp32 q/k): the producer writing K as split rows
    (k_split_rows, the cache keeping them; appends fused into the producer
    and the attention launch) gives outputs bit-identical to fp32 K split on
    every call, and every live slab K row is the split of the fp32 path's."""
    orders = json.load(open(os.path.join(HERE, "golden", "orders_2b.json")))
    ctrl = POL.controller_for_budget(0.1, orders, num_layers=32, num_heads=16, protected_prefix_scales=3)
    layer, H, B = 29, 16, 2
    sched = build_static_slot_schedule(ctrl, layer_idx=layer, num_heads=H)
    removed = lambda t: ctrl.removed_heads_by_source_for(layer, t)  # noqa: E731
    split = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    plain = sc.SegmentedLayerCache(sched, removed, num_heads=H)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128).to(device)
    sm = _scale_mul(H, 19).to(device)
    for t, side in enumerate(SIDES_1M):
        qkv = _qkv(B, side * side, H, 2000 + t).to(device)
        start = P.rope_start(SCHED_1M, t)
        app = split.producer_append(t, torch.float32, device)
        q, k, v = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start, append=app,
                                k_split_rows=True)
        out_s = split.step(q, k, v, t, 1.0, appended=app is not None, k_split_rows=True)
        q2, k2, v2 = P.qkv_produce(qkv, H, scale_mul=sm, rope_table=table, rope_start_row=start)
        out_p = plain.step(q2, k2, v2, t, 1.0)
        torch.cuda.synchronize(device)
        print(f"[split-row K] step {t} producer append {app is not None}", flush=True)
        assert torch.equal(out_s, out_p), t
        if split.active and t + 1 < len(SIDES_1M):
            for seg in sched.live_segments(t + 1):
                rows = slice(seg.offset, seg.offset + seg.length)
                assert torch.equal(split.cached_k[:, rows], _split(plain.cached_k[:, rows])), (t, seg)
                assert torch.equal(split.cached_v[:, rows], plain.cached_v[:, rows]), (t, seg)
    # a generation keeps one K format
    steps = [P.qkv_produce(_qkv(B, side * side, H, 3000 + t).to(device), H, scale_mul=sm, k_split_rows=True)
             for t, side in enumerate(SIDES_1M[:2])]
    split.step(*steps[0], 0, 1.0, k_split_rows=True)
    with pytest.raises(ValueError, match="same for every step"):
        split.step(*steps[1], 1, 1.0, k_split_rows=False)


@pytest.mark.parametrize("budget,qk_mode,amp", [(1.0, "bf16", "bf16"), (0.3, "bf16", "bf16"),
                                                 (0.3, "tf32", "bf16"), (0.3, "bf16", "fp16"),
                                                 (0.3, "bf16", "none")])
@torch.no_grad()
def test_patched_layer_forward(device, budget, qk_mode, amp, monkeypatch):
    """Two cosine-attention layers (H=4, C=512) through a 13-scale generation
    with the patched forward under bf16 autocast; per layer and step, the
    attention output entering proj against fp32 attention over the oracle's
    q/k/v of the same projection output and the policy's kept keys (scales
    of 1600+ tokens: batch row 1 and heads 0 and 3).  In TF32 dot mode the
    producer writes fp16 q/k, and the oracle attends over q and k rounded to
    fp16 (TF32's significand).  ``amp``: bf16 autocast (the reference's), fp16
    autocast (fp16 projection and v), or none (an fp32 model: fp32 v)."""
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", qk_mode)
    H, B, start_scale = 4, 2, 3
    torch.manual_seed(0)
    model = torch.nn.ModuleList([SelfAttention(512, H) for _ in range(2)]).to(device)
    orders = seeded_orders(2, H, 12 - start_scale, seed=3)
    enable_real_pruning_scale_specific_fused_segmented(model, budget, orders, protected_prefix_scales=start_scale)
    ctrl = model[0].heatkv_controller
    grid = P.precompute_rope2d_freqs_grid(D, {1.0: {"1M": {"scales": SCHED_1M}}}, 2, pad_to_multiplier=128)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128).numpy()
    captured = {}
    for li, layer in enumerate(model):
        layer.kv_caching(True)
        layer.proj.register_forward_hook(
            lambda mod, inp, out, li=li: captured.__setitem__(li, inp[0].detach().float()))
    removed_any = False
    hist = {li: [] for li in range(2)}
    g = torch.Generator().manual_seed(11)
    for t, side in enumerate(SIDES_1M):
        L = side * side
        big = L >= 1600
        heads = [0, 3] if big else list(range(H))
        bs = [1] if big else list(range(B))
        x = torch.randn((B, L, 512), generator=g).to(device)
        for li, layer in enumerate(model):
            amp_dtype = {"bf16": torch.bfloat16, "fp16": torch.float16, "none": None}[amp]
            with torch.autocast("cuda", dtype=amp_dtype or torch.bfloat16, enabled=amp_dtype is not None):
                qkv = torch.nn.functional.linear(
                    x, layer.mat_qkv.weight, bias=torch.cat((layer.q_bias, layer.zero_k_bias, layer.v_bias)))
                y = layer(x, None, None, SCHED_1M, grid, t)
            torch.cuda.synchronize(device)
            assert y.dtype == (amp_dtype or torch.float32) and tuple(y.shape) == (B, L, 512)
            assert qkv.dtype == (amp_dtype or torch.float32)
            arr = qkv.float().cpu().numpy().reshape(B, L, 3, H, D)
            sm = (layer.scale_mul_1H11.reshape(-1).float().clamp_max(layer.max_scale_mul).exp()).cpu().numpy()
            q, k, v = O.produce(arr, scale_mul=sm, table=table, start=P.rope_start(SCHED_1M, t))
            if qk_mode == "tf32":
                q = q.astype(np.float16).astype(np.float32)
                k = k.astype(np.float16).astype(np.float32)
                assert layer.heatkv_cache.cached_k is None or layer.heatkv_cache.cached_k.dtype == torch.float16
            hist[li].append((k, v))
            rem = ctrl.removed_heads_by_source_for(li, t)
            removed_any |= any(len(s) > 0 for s in rem.values())
            out = to_np(captured[li])
            for h in heads:
                srcs = [s for s in range(t) if h not in rem.get(s, set())]
                kk = np.concatenate([hist[li][s][0][:, h] for s in srcs] + [k[:, h]], axis=1)
                vv = np.concatenate([hist[li][s][1][:, h] for s in srcs] + [v[:, h]], axis=1)
                z = np.zeros((1, 0), np.int32)
                o, _ = oattn.flat_segmented_attention(q[bs, h:h + 1], None, None, z, z, np.zeros(1, np.int32),
                                                      kk[bs, None], vv[bs, None], 1.0)
                sl = slice(h * D, (h + 1) * D)
                assert_attention_close(out[bs][:, :, sl], None, o, None, what=f"layer {li} step {t} h {h}")
            x = y.float()
    assert removed_any == (budget < 1.0)
