"""Every output row of the benchmark workloads against the oracle, through the C ABI.

Each call goes straight to ``hkv_segmented_attention`` (libheatkv.so) with the
output and LSE buffers prefilled with NaN, so a (batch, head, query tile) that
the work plan drops, or a row that no workgroup writes, fails the comparison
(the oracle's values are finite).  The calls carry the product's attention
workspace, so the round split and the XCD-grouped item order run exactly as
in the operator.  Compared against oracle/segmented_attention.py (fp32 numpy,
the reference CPU path restated) with the contract tolerances: out max-abs
2e-2, mean-abs 2e-3, LSE max-abs 1e-3.

Workloads: the 2B final step (B=2, H=16, budget 0.1), the 8B-class final step
(B=8, H=32) at budgets 0.05, 0.1, 0.2 and 1.0 (every prior token kept), and
the skewed-ragged step (B=16, H=16, retained lengths log-uniform in
[0, 6425]) -- every (b, h) of each; the generation sweep's mid-scale steps
(1024 and 2304 queries: fewer than two rounds of items, so the plan cuts
most of them) with the sweep's own tables and work plan; and the 2B final
step at the model's precision (fp32 q of norm 30, unit fp32 k, bf16 v,
scale 1: the staged kernel) against the oracle in fp64.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from heatkv_amd import _lib, segmented_attention_plan
from heatkv_amd import workloads as W
from oracle import segmented_attention as oattn
from support import assert_attention_close, to_np

pytestmark = pytest.mark.gpu

ORACLE_WORKERS = 16


def model_precision(q, slab_k, ck):
    """q, slab K and current K as the cosine-attention model passes them under
    bf16 autocast: fp32, unit-norm k, q scaled to norm 30 (softmax scale 1).
    Slab rows that no segment owns stay NaN."""
    F = torch.nn.functional
    return (F.normalize(q.float(), dim=-1) * 30.0, F.normalize(slab_k.float(), dim=-1),
            F.normalize(ck.float(), dim=-1))


def abi_attention(wl, device, *, workspace=True, planned=False, model=False, split_rows=False, plan=None):
    """One call of hkv_segmented_attention on ``wl`` into NaN-prefilled out / lse
    (``planned``: with the host work plan of its tables; ``model``: fp32 q/k at
    the model's precision, scale 1, see model_precision; ``split_rows``: K
    passed as split rows, the split-row kernel; ``plan``: this work plan)."""
    slab_k, slab_v = W.build_slab(wl, device)
    st, en, ct = wl.schedule.device_tables(wl.target, device)
    q, ck, cv = (t.to(device) for t in (wl.q, wl.cur_k, wl.cur_v))
    scale = float(wl.softmax_scale)
    if model:
        q, slab_k, ck = model_precision(q, slab_k, ck)
        scale = 1.0
    B, H, L, D = q.shape
    out = torch.full((B, L, H * D), float("nan"), dtype=q.dtype, device=device)
    lse = torch.full((B, H, L), float("nan"), dtype=torch.float32, device=device)
    ws = _lib.attention_workspace(device) if workspace else None
    if planned and plan is None:
        hst, hen, hct = wl.tables()
        qpi = 128
        if split_rows:
            qpi = _lib.load().hkv_segmented_attention_item_shape(
                _lib.dtype_code(torch.float32), _lib.DTYPE_SPLIT_ROWS, _lib.dtype_code(cv.dtype), H, 0, 0, 0, None)
        plan = segmented_attention_plan(hst, hen, hct, batch_size=B, current_len=L,
                                        capacity=wl.schedule.capacity, device=device, queries_per_item=qpi)
    stream = torch.cuda.current_stream(device)
    k_args = (slab_k, ck, _lib.dtype_code(ck.dtype))
    if split_rows:
        sk2 = torch.empty(tuple(slab_k.shape[:-1]) + (256,), dtype=torch.bfloat16, device=device)
        ck2 = torch.empty(tuple(ck.shape[:-1]) + (256,), dtype=torch.bfloat16, device=device)
        for src, dst in ((slab_k.contiguous(), sk2), (ck.contiguous(), ck2)):
            _lib.check(_lib.load().hkv_split_rows(src.data_ptr(), dst.data_ptr(), src.numel() // 128,
                                                  stream.cuda_stream))
        k_args = (sk2, ck2, _lib.DTYPE_SPLIT_ROWS)
    code = _lib.load().hkv_segmented_attention(
        q.data_ptr(), k_args[0].data_ptr(), slab_v.data_ptr(), st.data_ptr(), en.data_ptr(), ct.data_ptr(),
        k_args[1].data_ptr(), cv.data_ptr(), out.data_ptr(), lse.data_ptr(), B, H, L, int(slab_k.shape[1]),
        int(st.shape[1]), D, _lib.dtype_code(q.dtype), k_args[2], _lib.dtype_code(cv.dtype), 0,
        scale, 0, 0, 0, plan.data_ptr() if plan is not None else None,
        int(plan.shape[0]) if plan is not None else 0, ws.data_ptr() if ws is not None else None,
        int(ws.numel()) if ws is not None else 0, stream.cuda_stream)
    _lib.check(code)
    torch.cuda.synchronize(device)
    return q, slab_k, slab_v, ck, out, lse


def check_every_row(wl, device, **kw):
    B, H, L, D = wl.q.shape
    print(f"[full] {wl.name} budget={wl.budget} B={B} H={H} L={L} cap={wl.schedule.capacity} "
          f"R={sorted(set(wl.retained_rows()))[:3]}..{max(wl.retained_rows())}", flush=True)
    q, slab_k, slab_v, ck, out, lse = abi_attention(wl, device, **kw)
    o, l = to_np(out), to_np(lse)
    assert np.isfinite(o).all(), f"{wl.name}: rows left unwritten (NaN) in the output"
    assert np.isfinite(l).all(), f"{wl.name}: rows left unwritten (NaN) in the LSE"
    st, en, ct = (t.numpy() for t in wl.tables())
    if kw.get("model"):  # scores up to +-30: the oracle in fp64
        ref_out, ref_lse = oattn.flat_segmented_attention(
            to_np(q).astype(np.float64), to_np(slab_k).astype(np.float64), to_np(slab_v).astype(np.float64),
            st, en, ct, to_np(ck).astype(np.float64), to_np(wl.cur_v).astype(np.float64), 1.0,
            dtype=np.float64, workers=ORACLE_WORKERS)
    else:
        ref_out, ref_lse = oattn.flat_segmented_attention(
            to_np(wl.q), to_np(slab_k), to_np(slab_v), st, en, ct, to_np(wl.cur_k), to_np(wl.cur_v),
            wl.softmax_scale, workers=ORACLE_WORKERS)
    worst = (0.0, None)
    for b in range(B):
        for h in range(H):
            mx, _ = assert_attention_close(o[b, :, h * D:(h + 1) * D], l[b, h], ref_out[b, :, h * D:(h + 1) * D],
                                           ref_lse[b, h], what=f"{wl.name} budget={wl.budget} b={b} h={h}")
            worst = max(worst, (mx, (b, h)), key=lambda x: x[0])
    print(f"[full] {wl.name}: {B * H} (b, h) pairs within tolerance, worst max-abs {worst[0]:.3e} at {worst[1]}",
          flush=True)


def test_every_row_2b_final(device):
    check_every_row(W.config(2), device)


def test_every_row_2b_final_without_workspace(device):
    check_every_row(W.config(2), device, workspace=False)


_BASE4 = []


def _config4(budget):
    if not _BASE4:
        _BASE4.append(W.config(4, budget=1.0))
    return W.with_budget(_BASE4[0], budget)


@pytest.mark.parametrize("budget", [0.05, 0.1, 0.2, 1.0])
def test_every_row_8b_class(budget, device):
    check_every_row(_config4(budget), device)


def test_every_row_skewed_ragged(device):
    check_every_row(W.config(5), device)


# With the host work plan (its cut items and XCD grouping) instead of the
# kernel's own ordering.
def test_every_row_2b_final_planned(device):
    check_every_row(W.config(2), device, planned=True)


@pytest.mark.parametrize("budget", [0.1, 1.0])
def test_every_row_8b_class_planned(budget, device):
    check_every_row(_config4(budget), device, planned=True)


def test_every_row_skewed_ragged_planned(device):
    check_every_row(W.config(5), device, planned=True)


# The 2B final step at the model's precision: fp32 q/k through the staged
# kernel, and with K as split rows through the split-row kernel; with and
# without the host work plan (cut items merged through the workspace).
@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("split_rows", [False, True])
def test_every_row_2b_final_model_precision(planned, split_rows, device):
    check_every_row(W.config(2), device, planned=planned, model=True, split_rows=split_rows)


# The generation sweep's mid-scale steps, with the tables and the work plan
# its cache uses (SlabSchedule.device_work_plan at attention_item_shape):
# scale 9 (1024 queries: 256 items for 512 slots, every item cut in two) and
# scale 11 (2304 queries: 576 items), layers 0 and 31.
@pytest.mark.parametrize("layer", [0, 31])
@pytest.mark.parametrize("target", [9, 11])
def test_every_row_sweep_mid_scale_planned(target, layer, device):
    from heatkv_amd import attention_item_shape

    wl = W.sweep_step(layer, target)
    B, H, L, _ = wl.q.shape
    shape = attention_item_shape(wl.q.dtype, wl.cur_k.dtype, wl.cur_v.dtype, device=device)
    plan = wl.schedule.device_work_plan(wl.target, device, B, L, item_shape=shape)
    cuts = int((plan[:, 4].cpu() >= 0).sum())
    print(f"[full] sweep layer {layer} step {target}: {plan.shape[0]} units, {cuts} cut parts, slots {shape[1]}",
          flush=True)
    check_every_row(wl, device, planned=True, plan=plan)
