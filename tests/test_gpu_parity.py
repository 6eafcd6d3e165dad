"""GPU parity: HIP pack + segmented attention (through the C ABI) against the oracle.

Every call goes through heatkv_amd's Python surface into libheatkv.so.
Attention is checked against oracle/segmented_attention.py (fp32 numpy) with
the contract tolerances (out max-abs 2e-2, mean-abs 2e-3, LSE max-abs 1e-3);
slab packing and offset tables bit-exact against oracle/slot_schedule.py and
oracle/pack.py.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import fused_real_pruning_flat_segmented_attention, pack_flat_segments_kv
from heatkv_amd import workloads as W
from oracle import pack as opack
from oracle import segmented_attention as oattn
from oracle import slot_schedule as osched
from support import assert_attention_close, bits, to_np

pytestmark = pytest.mark.gpu


def _run(q, slab_k, slab_v, tables, ck, cv, scale, device, **kw):
    st, en, ct = (t.to(device) for t in tables)
    out, lse = fused_real_pruning_flat_segmented_attention(
        q=q.to(device), persisted_k=None if slab_k is None else slab_k.to(device),
        persisted_v=None if slab_v is None else slab_v.to(device),
        segment_starts=st, segment_ends=en, segment_counts=ct,
        current_k=ck.to(device), current_v=cv.to(device), softmax_scale=scale,
        return_lse=True, **kw)
    torch.cuda.synchronize(device)
    return out, lse


def _oracle_schedule(wl):
    ranges = osched.scale_token_ranges(wl.sides)
    H, n_prior = wl.keep.shape
    static = {}
    for t in range(1, len(wl.sides)):
        static[t] = {s: {0: {h for h in range(H) if not bool(wl.keep[h, s])}}
                     for s in range(min(t, n_prior))}
    pol = osched.PolicyView(static, num_layers=1, source_start=0, source_end=n_prior - 1)
    return osched.build_schedule(pol, ranges, layer=0, num_heads=H), ranges


@pytest.mark.parametrize("cfg", [1, 2, 5])
def test_slab_pack_bit_exact(cfg, device):
    wl = W.config(cfg)
    print(f"[pack] config {cfg} B={wl.batch} H={wl.heads} cap={wl.schedule.capacity}", flush=True)
    slab_k, slab_v = W.build_slab(wl, device)
    osch, ranges = _oracle_schedule(wl)
    assert osch["capacity"] == wl.schedule.capacity
    st, en, ct = wl.tables()
    ost, oen, oct_ = osch["metadata_cpu_by_target"][wl.target]
    assert np.array_equal(st.numpy(), ost) and np.array_equal(en.numpy(), oen)
    assert np.array_equal(ct.numpy(), oct_)
    dense_k = torch.cat([wl.prior_k, wl.cur_k], dim=2)
    dense_v = torch.cat([wl.prior_v, wl.cur_v], dim=2)
    sk, sv = bits(slab_k), bits(slab_v)
    owned = np.zeros(wl.schedule.capacity, dtype=bool)
    for dense, slab in ((dense_k, sk), (dense_v, sv)):
        exp = opack.expected_live_rows(dense, osch["segments"], wl.target, ranges)
        for (s, h), (off, rows) in exp.items():
            n = rows.shape[1]
            assert np.array_equal(slab[:, off:off + n, :], bits(rows)), (s, h)
            owned[off:off + n] = True
    # rows no live segment owns keep the NaN fill (never written)
    nan_bits = bits(torch.full((1,), float("nan"), dtype=slab_k.dtype))[0]
    assert (sk[:, ~owned, :] == nan_bits).all()


def _check_workload(wl, device, heads=None, batches=None):
    slab_k, slab_v = W.build_slab(wl, device)
    out, lse = _run(wl.q, slab_k, slab_v, wl.tables(), wl.cur_k, wl.cur_v, wl.softmax_scale, device)
    st, en, ct = (t.numpy() for t in wl.tables())
    osch, _ = _oracle_schedule(wl)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(wl.q), to_np(slab_k), to_np(slab_v), st, en, ct, to_np(wl.cur_k), to_np(wl.cur_v),
        wl.softmax_scale, heads=heads, batches=batches)
    o = to_np(out)
    l = to_np(lse)
    B, H, L, D = wl.q.shape
    hs = range(H) if heads is None else heads
    bs = range(B) if batches is None else batches
    for b in bs:
        for h in hs:
            assert_attention_close(o[b, :, h * D:(h + 1) * D], l[b, h], ref_out[b, :, h * D:(h + 1) * D],
                                   ref_lse[b, h], what=f"{wl.name} b={b} h={h}")


def test_attention_config1(device):
    print("[attn] config 1", flush=True)
    _check_workload(W.config(1), device)


def test_attention_config2_heads(device):
    wl = W.config(2)
    r = wl.retained_rows()
    order = sorted(range(wl.heads), key=lambda h: r[h])
    heads = sorted({order[0], order[1], order[-1], order[-2]})
    print(f"[attn] config 2 heads {heads} R={[r[h] for h in heads]}", flush=True)
    _check_workload(wl, device, heads=heads, batches=[1])


def test_attention_priority_flag_is_schedule_only(device):
    """The work plan's field 6 (set when the items differ in length: the
    16-bit kernel then alternates its wave priority by tile) changes only the
    order in which each SIMD issues its two workgroups' instructions: the 2B
    final step gives the same bits with the field set and cleared."""
    print("[attn] config 2, plan priority field set vs cleared", flush=True)
    wl = W.config(2)
    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    plan = wl.schedule.device_work_plan(wl.target, device, wl.batch, wl.cur_len)
    assert bool((plan[plan[:, 0] >= 0, 6] == 1).all())
    cleared = plan.clone()
    cleared[:, 6] = 0
    cleared.hkv_queries_per_item = plan.hkv_queries_per_item
    cleared.hkv_plan_shape = plan.hkv_plan_shape
    q, ck, cv = (t.to(device) for t in (wl.q, wl.cur_k, wl.cur_v))
    res = []
    for p in (plan, cleared):
        out, lse = fused_real_pruning_flat_segmented_attention(
            q=q, persisted_k=slab_k, persisted_v=slab_v, segment_starts=st, segment_ends=en,
            segment_counts=ct, current_k=ck, current_v=cv, softmax_scale=wl.softmax_scale,
            return_lse=True, work_plan=p)
        torch.cuda.synchronize(device)
        res.append((out, lse))
    assert np.array_equal(bits(res[0][0]), bits(res[1][0]))
    assert np.array_equal(bits(res[0][1]), bits(res[1][1]))


def test_attention_config5_heads(device):
    wl = W.config(5)
    r = wl.retained_rows()
    order = sorted(range(wl.heads), key=lambda h: r[h])
    heads = sorted({order[0], order[len(order) // 2], order[-1]})
    print(f"[attn] config 5 heads {heads} R={[r[h] for h in heads]}", flush=True)
    _check_workload(wl, device, heads=heads, batches=[0, 15])


def _random_case(seed, B, H, L, cap, S, *, dtype=torch.bfloat16, kdtype=None, vdtype=None):
    """Random slab + tables with skipped (start >= end) and unaligned segments."""
    g = torch.Generator().manual_seed(seed)
    kdtype = kdtype or dtype
    vdtype = vdtype or dtype
    q = torch.randn((B, H, L, 128), generator=g).to(dtype)
    ck = torch.randn((B, H, L, 128), generator=g).to(kdtype)
    cv = torch.randn((B, H, L, 128), generator=g).to(vdtype)
    slab_k = torch.randn((B, cap, 128), generator=g).to(kdtype)
    slab_v = torch.randn((B, cap, 128), generator=g).to(vdtype)
    st = torch.zeros((H, S), dtype=torch.int32)
    en = torch.zeros((H, S), dtype=torch.int32)
    ct = torch.randint(0, S + 1, (H,), generator=g, dtype=torch.int32)
    for h in range(H):
        for i in range(S):
            a = int(torch.randint(0, cap, (1,), generator=g))
            n = int(torch.randint(-3, 70, (1,), generator=g))  # n <= 0: skipped entry
            st[h, i] = a
            en[h, i] = min(cap, a + n) if n > 0 else a + n
    return q, slab_k, slab_v, (st, en, ct), ck, cv


@pytest.mark.parametrize(
    "seed,B,H,L,cap,S",
    [(11, 1, 2, 1, 50, 3), (12, 2, 3, 5, 200, 5), (13, 1, 4, 33, 300, 7), (14, 2, 2, 130, 97, 4),
     (15, 1, 1, 257, 1000, 12), (16, 3, 5, 64, 0, 0),
     # work planning: one wave up to 64 heads x 64 entries, all threads beyond
     (17, 1, 64, 40, 3000, 64), (18, 1, 65, 20, 500, 3), (19, 2, 3, 70, 2000, 65),
     (20, 1, 2, 10, 100000, 200)],
)
def test_attention_random_tables(seed, B, H, L, cap, S, device):
    print(f"[attn] random seed={seed} B={B} H={H} L={L} cap={cap} S={S}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(seed, B, H, L, cap, S)
    scale = 1.0 / math.sqrt(128)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"seed {seed}")


@pytest.mark.parametrize("scale", [-0.3, 0.0, 1.0, 0.02])
def test_attention_scales(scale, device):
    print(f"[attn] scale {scale}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(21, 2, 3, 70, 300, 5)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale)
    # with scale 1 the scores are O(10), so a bf16-rounded probability weighs
    # more; the contract tolerance still holds for the output
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"scale {scale}")


@pytest.mark.parametrize(
    "qk,v",
    [(torch.float16, torch.float16), (torch.float32, torch.bfloat16), (torch.float32, torch.float32),
     (torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16)],
)
def test_attention_dtypes(qk, v, device):
    print(f"[attn] dtypes qk={qk} v={v}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(31, 2, 2, 90, 400, 6, dtype=qk, kdtype=qk, vdtype=v)
    scale = 1.0 / math.sqrt(128)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device)
    assert out.dtype == qk
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale)
    # fp32 q/k products are split into bf16 high and low parts (beyond TF32)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"{qk}/{v}")


@pytest.mark.parametrize("vdt", [torch.bfloat16, torch.float32])
def test_attention_fp32_qk_cosine_scores(vdt, device):
    """fp32 q/k as a cosine-attention model passes them: unit-norm q and k, q
    scaled by 20..100 per head, softmax scale 1, so scores reach +-100; a bf16
    rounding of q or k (relative 2^-9) would move them by ~0.2 and the LSE by
    far more than 1e-3.  Checked against the oracle in fp64."""
    print(f"[attn] fp32 q/k cosine scores, v={vdt}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(71, 2, 3, 90, 400, 6, dtype=torch.float32,
                                             kdtype=torch.float32, vdtype=vdt)
    mul = torch.tensor([20.0, 55.0, 100.0]).view(1, 3, 1, 1)
    q = torch.nn.functional.normalize(q, dim=-1) * mul
    ck = torch.nn.functional.normalize(ck, dim=-1)
    sk = torch.nn.functional.normalize(sk, dim=-1)
    out, lse = _run(q, sk, sv, tables, ck, cv, 1.0, device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), 1.0,
        dtype=np.float64)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"cosine fp32 q/k, v={vdt}")


def test_attention_no_persisted(device):
    print("[attn] persisted None", flush=True)
    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn((2, 3, 40, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    tables = (torch.zeros((3, 0), dtype=torch.int32), torch.zeros((3, 0), dtype=torch.int32),
              torch.zeros((3,), dtype=torch.int32))
    out, lse = _run(q, None, None, tables, k, v, 0.1, device)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float(), scale=0.1)
    ref = ref.transpose(1, 2).reshape(2, 40, 3 * 128)
    assert_attention_close(to_np(out), None, to_np(ref), None, what="no persisted")


@pytest.mark.parametrize("kdt,vdt,D", [(torch.bfloat16, torch.bfloat16, 128), (torch.float32, torch.bfloat16, 128),
                                       (torch.float16, torch.float32, 64), (torch.bfloat16, torch.bfloat16, 3)])
def test_pack_random_items(kdt, vdt, D, device):
    print(f"[pack] random items {kdt} {vdt} D={D}", flush=True)
    g = torch.Generator().manual_seed(7)
    B, S_src, cap = 3, 500, 700
    src_k = torch.randn((B, S_src, D), generator=g).to(kdt)
    src_v = torch.randn((B, S_src, D), generator=g).to(vdt)
    dst_k0 = torch.randn((B, cap, D), generator=g).to(kdt)
    dst_v0 = torch.randn((B, cap, D), generator=g).to(vdt)
    n_items = 9
    lengths = torch.randint(0, 90, (n_items,), generator=g)
    lengths[0] = 0
    src_starts = torch.stack([torch.randint(0, S_src - int(n) + 1, (1,), generator=g)[0] for n in lengths])
    # non-overlapping destinations at unaligned offsets
    dst_starts = torch.cumsum(torch.cat([torch.tensor([3]), lengths[:-1] + 5]), 0)
    max_len = int(lengths.max())
    dk, dv = dst_k0.clone().to(device), dst_v0.clone().to(device)
    pack_flat_segments_kv(dst_k=dk, dst_v=dv, src_k=src_k.to(device), src_v=src_v.to(device),
                          dst_starts=dst_starts.to(device), src_starts=src_starts.to(device),
                          lengths=lengths.to(device), max_length=max_len)
    torch.cuda.synchronize(device)
    ek = opack.pack_flat_segments(dst_k0.clone(), src_k, dst_starts.tolist(), src_starts.tolist(), lengths.tolist())
    ev = opack.pack_flat_segments(dst_v0.clone(), src_v, dst_starts.tolist(), src_starts.tolist(), lengths.tolist())
    assert np.array_equal(bits(dk), bits(ek))
    assert np.array_equal(bits(dv), bits(ev))


def test_pack_max_length_truncates(device):
    """Items longer than the grid bound copy block_t * ceil(max_length / block_t) rows."""
    print("[pack] max_length truncation", flush=True)
    B, D = 1, 128
    src = torch.arange(B * 200 * D, dtype=torch.float32).reshape(B, 200, D).to(torch.bfloat16)
    dst = torch.zeros((B, 300, D), dtype=torch.bfloat16)
    dk, dv = dst.clone().to(device), dst.clone().to(device)
    meta = [torch.tensor(x, dtype=torch.int64, device=device) for x in ([10], [0], [150])]
    pack_flat_segments_kv(dst_k=dk, dst_v=dv, src_k=src.to(device), src_v=src.to(device),
                          dst_starts=meta[0], src_starts=meta[1], lengths=meta[2], max_length=40)
    torch.cuda.synchronize(device)
    exp = dst.clone()
    exp[:, 10:10 + 64] = src[:, :64]  # 32 * ceil(40 / 32) rows
    assert np.array_equal(bits(dk), bits(exp))


_CONFIG4 = []


def _config4():
    if not _CONFIG4:
        _CONFIG4.append(W.config(4))
    return _CONFIG4[0]


def test_attention_config4_unpruned_equals_dense_sdpa(device):
    """8B-class shape at budget 1.0: every prior token is kept, so each head's
    result is dense attention over the whole prefix plus the current scale
    (the reference's dense path) -- checked with torch SDPA in fp32 on the CPU."""
    wl = W.with_budget(_config4(), 1.0)
    print(f"[attn] config 4 budget 1.0 capacity {wl.schedule.capacity}", flush=True)
    slab_k, slab_v = W.build_slab(wl, device)
    out, lse = _run(wl.q, slab_k, slab_v, wl.tables(), wl.cur_k, wl.cur_v, wl.softmax_scale, device)
    o = to_np(out)
    D = 128
    b = 5
    for h in (0, 17, 31):
        k = torch.cat([wl.prior_k[b, h], wl.cur_k[b, h]], dim=0).float()
        v = torch.cat([wl.prior_v[b, h], wl.cur_v[b, h]], dim=0).float()
        q = wl.q[b, h].float()
        ref = torch.nn.functional.scaled_dot_product_attention(q[None, None], k[None, None], v[None, None],
                                                               scale=wl.softmax_scale)[0, 0]
        s = (q @ k.T) * wl.softmax_scale
        ref_lse = torch.logsumexp(s, dim=-1)
        assert_attention_close(o[b, :, h * D:(h + 1) * D], to_np(lse)[b, h], ref.numpy(), ref_lse.numpy(),
                               what=f"config 4 dense b={b} h={h}")


def test_attention_config4_budget_005(device):
    wl = W.with_budget(_config4(), 0.05)
    r = wl.retained_rows()
    order = sorted(range(wl.heads), key=lambda h: r[h])
    heads = sorted({order[0], order[-1]})
    print(f"[attn] config 4 budget 0.05 heads {heads} R={[r[h] for h in heads]}", flush=True)
    _check_workload(wl, device, heads=heads, batches=[2])


@pytest.mark.parametrize("qk,out", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                    (torch.float32, torch.float16), (torch.bfloat16, torch.bfloat16)])
def test_attention_out_dtype_is_a_single_rounding(qk, out, device):
    """out_dtype writes the kernel's fp32 result rounded once: bit-identical to
    the output in fp32 cast afterwards (both the 16-bit and the staged kernel)."""
    wl = W.config(1)
    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    kw = dict(q=wl.q.to(device, qk), persisted_k=slab_k.to(qk), persisted_v=slab_v, segment_starts=st,
              segment_ends=en, segment_counts=ct, current_k=wl.cur_k.to(device, qk),
              current_v=wl.cur_v.to(device), softmax_scale=wl.softmax_scale)
    got = fused_real_pruning_flat_segmented_attention(**kw, out_dtype=out)
    full = fused_real_pruning_flat_segmented_attention(**kw, out_dtype=torch.float32)
    torch.cuda.synchronize(device)
    assert got.dtype == out and full.dtype == torch.float32
    assert torch.equal(got, full.to(out))
    with pytest.raises(ValueError, match="out_dtype"):
        fused_real_pruning_flat_segmented_attention(**kw, out_dtype=torch.int32)


@pytest.mark.parametrize("H,S", [(16, 40), (3, 70)])
def test_attention_fp32_qk_random_tables(H, S, device):
    """fp32 q/k (the register-staged kernel) over random tables on both
    planning paths (one wave for 16 x 40 entries, all threads for 70)."""
    print(f"[attn] fp32 q/k random H={H} S={S}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(21 + H, 1, H, 50, 4000, S, kdtype=torch.float32,
                                             dtype=torch.float32, vdtype=torch.bfloat16)
    scale = 1.0 / math.sqrt(128)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"fp32 q/k H={H} S={S}")


@pytest.mark.parametrize("split", ["0", "1"])
def test_attention_output_not_16_byte_aligned(split, device, monkeypatch):
    """16-bit output through the C ABI at an address 8 bytes past 16-byte
    alignment: the kernel then stores from registers instead of staging
    rows in LDS, with the same bits (whole items and, with the workspace,
    merged parts)."""
    from heatkv_amd import _lib

    monkeypatch.setenv("HKV_ATTN_SPLIT", split)
    B, H, L, cap, S = 1, 4, 200, 3000, 1
    print(f"[attn] unaligned output split={split}", flush=True)
    q, sk, sv, _, ck, cv = _random_case(31, B, H, L, cap, 0)
    # every head keeps the whole slab: 51 key tiles per item, so with the
    # workspace the 8 items are cut into parts and merged
    st = torch.zeros((H, S), dtype=torch.int32, device=device)
    en = torch.full((H, S), cap, dtype=torch.int32, device=device)
    ct = torch.ones((H,), dtype=torch.int32, device=device)
    scale = 1.0 / math.sqrt(128)
    qd, skd, svd, ckd, cvd = (t.to(device) for t in (q, sk, sv, ck, cv))
    want = fused_real_pruning_flat_segmented_attention(
        q=qd, persisted_k=skd, persisted_v=svd, segment_starts=st, segment_ends=en, segment_counts=ct,
        current_k=ckd, current_v=cvd, softmax_scale=scale)
    buf = torch.zeros(B * L * H * 128 + 4, dtype=torch.bfloat16, device=device)
    assert (buf.data_ptr() + 8) % 16 == 8
    ws = _lib.attention_workspace(device) if split == "1" else None
    stream = torch.cuda.current_stream(device)
    code = _lib.load().hkv_segmented_attention(
        qd.data_ptr(), skd.data_ptr(), svd.data_ptr(), st.data_ptr(), en.data_ptr(), ct.data_ptr(),
        ckd.data_ptr(), cvd.data_ptr(), buf.data_ptr() + 8, None, B, H, L, cap, S, 128,
        _lib.dtype_code(qd.dtype), _lib.dtype_code(ckd.dtype), _lib.dtype_code(cvd.dtype), 0, float(scale), 0, 0, 0, None, 0,
        ws.data_ptr() if ws is not None else None, int(ws.numel()) if ws is not None else 0,
        stream.cuda_stream)
    _lib.check(code)
    torch.cuda.synchronize(device)
    got = buf[4:].reshape(B, L, H * 128)
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("seed", list(range(40, 52)))
def test_attention_random_shapes(seed, device, monkeypatch):
    """Random batch, head count (1-70), table width (0-70), query length and
    slab size, with and without the round split: both planning paths, cut
    and whole items, partial tiles, against the oracle."""
    g = torch.Generator().manual_seed(seed)

    def pick(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    B, H, L, cap, S = pick(1, 3), pick(1, 70), pick(1, 300), pick(0, 5000), pick(0, 70)
    if cap == 0:
        S = 0
    split = "1" if seed % 2 else "0"
    monkeypatch.setenv("HKV_ATTN_SPLIT", split)
    print(f"[attn] random shape seed={seed} B={B} H={H} L={L} cap={cap} S={S} split={split}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(seed, B, H, L, cap, S)
    scale = 1.0 / math.sqrt(128)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"seed {seed}")


@pytest.mark.parametrize("seed", list(range(60, 70)))
def test_attention_random_shapes_planned(seed, device, monkeypatch):
    """Random shapes (as above, up to 2300 queries so that items get cut)
    with the host work plan of their tables, with and without the workspace
    (without it, cut units run whole), against the oracle."""
    from heatkv_amd import segmented_attention_plan

    g = torch.Generator().manual_seed(seed)

    def pick(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    B, H, L, cap, S = pick(1, 3), pick(1, 40), pick(1, 2300), pick(0, 5000), pick(0, 40)
    if cap == 0:
        S = 0
    split = "1" if seed % 2 else "0"
    monkeypatch.setenv("HKV_ATTN_SPLIT", split)
    print(f"[attn] planned random shape seed={seed} B={B} H={H} L={L} cap={cap} S={S} split={split}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(seed, B, H, L, cap, S)
    plan = segmented_attention_plan(*tables, batch_size=B, current_len=L, capacity=cap, device=device)
    scale = 1.0 / math.sqrt(128)
    out, lse = _run(q, sk, sv, tables, ck, cv, scale, device, work_plan=plan)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale, workers=16)
    assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse, what=f"planned seed {seed}")


@pytest.mark.parametrize("seed", list(range(70, 76)))
def test_attention_random_shapes_split_rows(seed, device, monkeypatch):
    """fp32 q/k with bf16 v (the split-row kernel, K written as split rows per
    call) on random shapes, with the host work plan of the kernel's item size
    (every other seed without the workspace: cut units run whole) and without
    a plan, against the oracle; scores of O(10) (q and k of norm ~sqrt(128) /
    3.5) so the split's ~16 bits matter."""
    from heatkv_amd import attention_queries_per_item, segmented_attention_plan

    g = torch.Generator().manual_seed(seed)

    def pick(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    B, H, L, cap, S = pick(1, 3), pick(1, 24), pick(1, 2300), pick(0, 4000), pick(0, 30)
    if cap == 0:
        S = 0
    monkeypatch.setenv("HKV_ATTN_SPLIT", "1" if seed % 2 else "0")
    qpi = attention_queries_per_item(torch.float32, torch.float32, torch.bfloat16)
    assert qpi in (128, 256)
    print(f"[attn] split rows random shape seed={seed} B={B} H={H} L={L} cap={cap} S={S}", flush=True)
    q, sk, sv, tables, ck, cv = _random_case(seed, B, H, L, cap, S, dtype=torch.float32, kdtype=torch.float32,
                                             vdtype=torch.bfloat16)
    scale = 0.3
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q), to_np(sk), to_np(sv), *(t.numpy() for t in tables), to_np(ck), to_np(cv), scale, workers=16)
    plan = segmented_attention_plan(*tables, batch_size=B, current_len=L, capacity=cap, device=device,
                                    queries_per_item=qpi)
    for wp in (plan, None):
        out, lse = _run(q, sk, sv, tables, ck, cv, scale, device, work_plan=wp)
        assert_attention_close(to_np(out), to_np(lse), ref_out, ref_lse,
                                what=f"split rows seed {seed} plan={wp is not None}")
    # a plan of the other item size does not fit the kernel
    other = 384 - qpi
    plan_other = segmented_attention_plan(*tables, batch_size=B, current_len=L, capacity=cap, device=device,
                                          queries_per_item=other)
    with pytest.raises(ValueError, match=f"{other}-query items"):
        _run(q, sk, sv, tables, ck, cv, scale, device, work_plan=plan_other)


def test_attention_k_split_rows_matches_fp32_k(device):
    """The operator on K given as split rows (k_split_rows=True, as the
    producer writes it) against the same call on fp32 K (split by the call
    itself): outputs and LSE bit-identical; the fused append on split rows
    writes the split rows; the wrong dtypes or an fp32 dot mode are refused."""
    from heatkv_amd.real_pruning_fused_attention import _split_rows

    g = torch.Generator().manual_seed(31)
    B, H, L, cap = 2, 5, 200, 700
    stream = torch.cuda.current_stream(device)
    split = lambda t: _split_rows(t.contiguous(), stream).view(torch.float32)  # noqa: E731
    q = (torch.nn.functional.normalize(torch.randn((B, H, L, 128), generator=g), dim=-1) * 30).to(device)
    ck = torch.nn.functional.normalize(torch.randn((B, H, L, 128), generator=g), dim=-1).to(device)
    cv = torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16).to(device)
    sk = torch.nn.functional.normalize(torch.randn((B, cap, 128), generator=g), dim=-1).to(device)
    sv = torch.randn((B, cap, 128), generator=g).to(torch.bfloat16).to(device)
    st = torch.tensor([[0, 100, 0], [150, 0, 0], [0, 0, 0], [300, 400, 500], [10, 0, 0]], dtype=torch.int32)
    en = torch.tensor([[64, 140, 0], [151, 0, 0], [0, 0, 0], [380, 420, 600], [12, 0, 0]], dtype=torch.int32)
    ct = torch.tensor([2, 1, 0, 3, 1], dtype=torch.int32)
    tables = dict(segment_starts=st.to(device), segment_ends=en.to(device), segment_counts=ct.to(device))
    kw = dict(q=q, persisted_v=sv, current_v=cv, softmax_scale=1.0, return_lse=True, **tables)
    out_f, lse_f = fused_real_pruning_flat_segmented_attention(persisted_k=sk, current_k=ck, **kw)
    out_s, lse_s = fused_real_pruning_flat_segmented_attention(persisted_k=split(sk), current_k=split(ck),
                                                               k_split_rows=True, **kw)
    torch.cuda.synchronize(device)
    assert torch.equal(out_f, out_s) and torch.equal(lse_f, lse_s)
    # the append of 50 current rows of heads 1 and 3 into slab rows [600, 650)
    # and [650, 700) (outside every segment the call reads)
    offs = torch.tensor([-1, 600, -1, 650, -1], dtype=torch.int32, device=device)
    slab_k = split(sk).clone()
    slab_v = sv.clone()
    n = 50
    fused_real_pruning_flat_segmented_attention(
        q=q[:, :, :n].contiguous(), persisted_k=slab_k, persisted_v=slab_v, current_k=split(ck[:, :, :n]),
        current_v=cv[:, :, :n].contiguous(), softmax_scale=1.0, k_split_rows=True, append_offsets=offs,
        **tables)
    torch.cuda.synchronize(device)
    want_k, want_v = split(sk).clone(), sv.clone()
    for h, off in ((1, 600), (3, 650)):
        want_k[:, off:off + n] = split(ck[:, h, :n])
        want_v[:, off:off + n] = cv[:, h, :n]
    assert torch.equal(slab_k, want_k) and torch.equal(slab_v, want_v)
    with pytest.raises(ValueError, match="k_split_rows"):
        fused_real_pruning_flat_segmented_attention(persisted_k=split(sk).bfloat16(), current_k=ck.bfloat16(),
                                                    k_split_rows=True, **dict(kw, q=q.bfloat16()))


def test_attention_k_split_rows_refuses_fp32_dot_mode(device, monkeypatch):
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "fp32")
    B, H, L = 1, 2, 64
    q = torch.randn((B, H, L, 128), device=device)
    v = torch.randn((B, H, L, 128), device=device).bfloat16()
    z = torch.zeros((H, 0), dtype=torch.int32, device=device)
    c = torch.zeros((H,), dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="dot modes"):
        fused_real_pruning_flat_segmented_attention(q=q, persisted_k=None, persisted_v=None, segment_starts=z,
                                                    segment_ends=z, segment_counts=c, current_k=q, current_v=v,
                                                    softmax_scale=1.0, k_split_rows=True)


def test_split_rows_bit_exact(device):
    """hkv_split_rows against the split restated in numpy: hi = x rounded to
    bf16 (nearest even), lo = (x - hi) rounded to bf16 (x - hi is exact in
    fp32), including values that round up across a power of two, ties, zeros,
    signs and magnitudes from 1e-30 to 1e38 (no subnormals: their rounding
    follows the device's denormal mode)."""
    from heatkv_amd import _lib

    g = torch.Generator().manual_seed(11)
    x = torch.randn((333, 128), generator=g) * torch.logspace(-30, 30, 128).view(1, 128)
    x[0, :8] = torch.tensor([0.0, -0.0, 1.0, -1.0, 1.00390625, 1.0 + 2 ** -8 + 2 ** -20, 3.0, -3.0])
    x[1, :4] = torch.tensor([255.99999, 65535.9, -1.5e38, 1e-30])
    xd = x.to(device)
    out = torch.empty((333, 256), dtype=torch.bfloat16, device=device)
    stream = torch.cuda.current_stream(device)
    _lib.check(_lib.load().hkv_split_rows(xd.data_ptr(), out.data_ptr(), 333, stream.cuda_stream))
    torch.cuda.synchronize(device)
    got = out.cpu().view(torch.int16).numpy().astype(np.uint16)

    def bf16_rne(a):  # float32 numpy -> bf16 bits, round to nearest even
        u = a.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return r

    xn = x.numpy().astype(np.float32)
    hi = bf16_rne(xn)
    hi_f = (hi.astype(np.uint32) << 16).view(np.float32)
    lo = bf16_rne((xn - hi_f).astype(np.float32))
    assert np.array_equal(got[:, :128], hi)
    assert np.array_equal(got[:, 128:], lo)


@pytest.mark.parametrize("kdt,vdt,T,n", [(torch.bfloat16, torch.bfloat16, 21, 36), (torch.float32, torch.bfloat16, 0, 4),
                                         (torch.float16, torch.float16, 57, 0), (torch.float32, torch.float32, 600, 700)])
def test_concat_kv_bit_exact(kdt, vdt, T, n, device):
    """concat_kv (one launch for K and V) equals torch.cat of each, bit for bit,
    including empty old or new parts and groups larger than one 64 KiB chunk."""
    from heatkv_amd.real_pruning_fused_attention import concat_kv

    g = torch.Generator().manual_seed(T + n)
    B, H, D = 2, 3, 128
    ok, nk = (torch.randn((B, H, t, D), generator=g).to(kdt).to(device) for t in (T, n))
    ov, nv = (torch.randn((B, H, t, D), generator=g).to(vdt).to(device) for t in (T, n))
    out_k, out_v = concat_kv(ok, nk, ov, nv)
    torch.cuda.synchronize(device)
    for got, want in ((out_k, torch.cat((ok, nk), dim=2)), (out_v, torch.cat((ov, nv), dim=2))):
        assert got.shape == want.shape and got.dtype == want.dtype
        assert torch.equal(got.view(torch.int16 if got.element_size() == 2 else torch.int32),
                           want.view(torch.int16 if want.element_size() == 2 else torch.int32))


@pytest.mark.parametrize("seed,qkdt,vdt,planned,split", [
    (80, torch.bfloat16, torch.bfloat16, True, "1"), (81, torch.bfloat16, torch.bfloat16, False, "1"),
    (82, torch.float16, torch.float16, True, "0"), (83, torch.bfloat16, torch.float16, False, "0"),
    (84, torch.float32, torch.float32, True, "1"), (85, torch.float32, torch.bfloat16, False, "1"),
    (86, torch.bfloat16, torch.bfloat16, True, "0")])
def test_attention_fused_append(seed, qkdt, vdt, planned, split, device, monkeypatch):
    """append_offsets (hkv_segmented_attention_append): the output and LSE
    equal the plain call's bit for bit, and the slab afterwards equals the
    slab with each appended head's current rows written at its offset (heads
    at -1 and one whose rows would pass the capacity untouched), on random
    shapes whose segments stay below the appended rows; the 16-bit kernel
    runs the copy in its own launch, the register-staged kernel (fp32 K or V)
    after it."""
    from heatkv_amd import segmented_attention_plan

    monkeypatch.setenv("HKV_ATTN_SPLIT", split)
    monkeypatch.setenv("HKV_ATTN_SPLIT_ROWS", "0")  # fp32 q/k with bf16 v on the staged kernel
    g = torch.Generator().manual_seed(seed)

    def pick(lo, hi):
        return int(torch.randint(lo, hi + 1, (1,), generator=g))

    B, H, L, cap0, S = pick(1, 3), pick(2, 24), pick(1, 700), pick(0, 3000), pick(0, 20)
    if cap0 == 0:
        S = 0
    cap = cap0 + H * L
    print(f"[attn] fused append seed={seed} B={B} H={H} L={L} cap={cap} S={S} {qkdt} {vdt} "
          f"planned={planned} split={split}", flush=True)
    q, sk0, sv0, tables, ck, cv = _random_case(seed, B, H, L, cap0, S, dtype=qkdt, kdtype=qkdt, vdtype=vdt)
    # rows [cap0, cap) hold H slots of L rows above every segment
    sk = torch.cat((sk0, torch.randn((B, H * L, 128), generator=g).to(qkdt)), dim=1)
    sv = torch.cat((sv0, torch.randn((B, H * L, 128), generator=g).to(vdt)), dim=1)
    slots = torch.randperm(H, generator=g).tolist()
    offsets = [cap0 + slots[h] * L if bool(torch.rand((1,), generator=g) < 0.75) else -1 for h in range(H)]
    offsets[-1] = cap - L + 1  # past the capacity: not written
    want_k, want_v = sk.clone(), sv.clone()
    for h, off in enumerate(offsets):
        if 0 <= off <= cap - L:
            want_k[:, off:off + L] = ck[:, h]
            want_v[:, off:off + L] = cv[:, h]
    plan = (segmented_attention_plan(*tables, batch_size=B, current_len=L, capacity=cap, device=device)
            if planned else None)
    scale = 1.0 / math.sqrt(128)
    out_a, lse_a = _run(q, sk, sv, tables, ck, cv, scale, device, work_plan=plan)
    slab_k, slab_v = sk.to(device), sv.to(device)
    out_b, lse_b = _run(q, slab_k, slab_v, tables, ck, cv, scale, device, work_plan=plan,
                        append_offsets=torch.tensor(offsets, dtype=torch.int32, device=device))
    assert np.array_equal(bits(out_b), bits(out_a))
    assert np.array_equal(bits(lse_b), bits(lse_a))
    assert np.array_equal(bits(slab_k), bits(want_k))
    assert np.array_equal(bits(slab_v), bits(want_v))


@pytest.mark.parametrize("seed,qkdt,vdt,planned", [
    (95, torch.bfloat16, torch.bfloat16, True), (96, torch.float16, torch.float16, False),
    (97, torch.float32, torch.float32, True)])
def test_attention_fused_append_two_destinations(seed, qkdt, vdt, planned, device, monkeypatch):
    """append_also (hkv_segmented_attention_append2): the output and LSE equal
    the plain call's bit for bit, the first slab equals the one-destination
    append's, and the second slab equals itself with each head's current rows
    written at its own offset (heads at -1 and one past the second capacity
    untouched); the 16-bit kernel copies in its own launch, the staged kernel
    (fp32) after it."""
    from heatkv_amd import segmented_attention_plan

    monkeypatch.setenv("HKV_ATTN_SPLIT_ROWS", "0")
    g = torch.Generator().manual_seed(seed)
    B, H, L, cap0, S = 2, 6, 37, 500, 3
    cap = cap0 + H * L
    print(f"[attn] two-destination append seed={seed} {qkdt} {vdt} planned={planned}", flush=True)
    q, sk0, sv0, tables, ck, cv = _random_case(seed, B, H, L, cap0, S, dtype=qkdt, kdtype=qkdt, vdtype=vdt)
    sk = torch.cat((sk0, torch.randn((B, H * L, 128), generator=g).to(qkdt)), dim=1)
    sv = torch.cat((sv0, torch.randn((B, H * L, 128), generator=g).to(vdt)), dim=1)
    offsets = [cap0 + h * L for h in range(H)]
    offsets[1] = -1
    cap2 = 3 * H * L
    s2k = torch.randn((B, cap2, 128), generator=g).to(qkdt)
    s2v = torch.randn((B, cap2, 128), generator=g).to(vdt)
    offsets2 = [int(x) for x in torch.randperm(3 * H, generator=g)[:H] * L]
    offsets2[2] = -1
    offsets2[3] = cap2 - L + 1  # past the second capacity: not written
    want_k, want_v = sk.clone(), sv.clone()
    want2_k, want2_v = s2k.clone(), s2v.clone()
    for h in range(H):
        if offsets[h] >= 0:
            want_k[:, offsets[h]:offsets[h] + L] = ck[:, h]
            want_v[:, offsets[h]:offsets[h] + L] = cv[:, h]
        if 0 <= offsets2[h] <= cap2 - L:
            want2_k[:, offsets2[h]:offsets2[h] + L] = ck[:, h]
            want2_v[:, offsets2[h]:offsets2[h] + L] = cv[:, h]
    plan = (segmented_attention_plan(*tables, batch_size=B, current_len=L, capacity=cap, device=device)
            if planned else None)
    scale = 1.0 / math.sqrt(128)
    out_a, lse_a = _run(q, sk, sv, tables, ck, cv, scale, device, work_plan=plan)
    slab_k, slab_v = sk.to(device), sv.to(device)
    d2k, d2v = s2k.to(device), s2v.to(device)
    out_b, lse_b = _run(q, slab_k, slab_v, tables, ck, cv, scale, device, work_plan=plan,
                        append_offsets=torch.tensor(offsets, dtype=torch.int32, device=device),
                        append_also=(d2k, d2v, torch.tensor(offsets2, dtype=torch.int32, device=device)))
    assert np.array_equal(bits(out_b), bits(out_a))
    assert np.array_equal(bits(lse_b), bits(lse_a))
    assert np.array_equal(bits(slab_k), bits(want_k)) and np.array_equal(bits(slab_v), bits(want_v))
    assert np.array_equal(bits(d2k), bits(want2_k)) and np.array_equal(bits(d2v), bits(want2_v))
    # without append_offsets the second destination is refused
    with pytest.raises(ValueError, match="append_offsets"):
        _run(q, slab_k, slab_v, tables, ck, cv, scale, device,
             append_also=(d2k, d2v, torch.tensor(offsets2, dtype=torch.int32, device=device)))


def test_attention_fused_append_rejects(device, monkeypatch):
    """append_offsets is refused where the call would not write the caller's
    slab: the split-row K path (a split copy of the slab) and a slab that is
    not contiguous; and for a wrongly shaped offsets tensor."""
    monkeypatch.setenv("HKV_ATTN_SPLIT_ROWS", "1")
    B, H, L, cap = 1, 2, 8, 64
    q, sk, sv, tables, ck, cv = _random_case(90, B, H, L, cap, 2, dtype=torch.float32, kdtype=torch.float32,
                                             vdtype=torch.bfloat16)
    offs = torch.tensor([0, 8], dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="split"):
        _run(q, sk, sv, tables, ck, cv, 0.1, device, append_offsets=offs)
    q, sk, sv, tables, ck, cv = _random_case(91, B, H, L, cap, 2)
    wide_k = torch.zeros((B, cap, 256), dtype=sk.dtype, device=device)
    with pytest.raises(ValueError, match="contiguous"):
        _run(q, wide_k[:, :, :128], sv, tables, ck, cv, 0.1, device, append_offsets=offs)
    with pytest.raises(ValueError, match=r"\[H\]"):
        _run(q, sk, sv, tables, ck, cv, 0.1, device, append_offsets=offs[:1])
