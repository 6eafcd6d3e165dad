"""The reference's dot-mode knobs change the arithmetic as they say.

REAL_PRUNING_FUSED_QK_DOT_MODE (real_pruning_fused_attention.py:141-153,
298-308) and REAL_PRUNING_FUSED_VALUE_DOT_MODE (:176-184, 286-295) select the
precision of S = Q K^T and of O = P V.  Each mode is run through the operator
on the GPU and compared with the fp64 oracle (oracle/segmented_attention.py)
at bounds that only that mode's precision meets, next to the default mode's
error on the same inputs:

* QK fp32/ieee on fp32 q/k at cosine-attention scores of +-100: the LSE
  (which does not involve the rounding of P) within 5e-5 (fp32 accumulation
  of scores of that size); the default
  2-piece split (~16 bits) is at least 4 times further off.
* value fp32: the output within 2e-5 for bf16, fp16 and fp32 V; the default
  mode rounds P to V's 16-bit type and is at least 10 times further off.
* fp32 V in the default value mode: P and V carry ~16 bits (the reference
  takes a TF32 dot there), output within 2e-4.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from heatkv_amd import fused_real_pruning_flat_segmented_attention
from oracle import segmented_attention as oattn
from support import to_np

pytestmark = pytest.mark.gpu


def _case(seed, dtype_qk, dtype_v, B=2, H=3, L=150, cap=500, S=5, cosine=False):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, H, L, 128), generator=g)
    ck = torch.randn((B, H, L, 128), generator=g)
    cv = torch.randn((B, H, L, 128), generator=g)
    sk = torch.randn((B, cap, 128), generator=g)
    sv = torch.randn((B, cap, 128), generator=g)
    if cosine:
        mul = torch.tensor([20.0, 55.0, 100.0][:H]).view(1, H, 1, 1)
        q = torch.nn.functional.normalize(q, dim=-1) * mul
        ck = torch.nn.functional.normalize(ck, dim=-1)
        sk = torch.nn.functional.normalize(sk, dim=-1)
    st = torch.zeros((H, S), dtype=torch.int32)
    en = torch.zeros((H, S), dtype=torch.int32)
    ct = torch.full((H,), S, dtype=torch.int32)
    for h in range(H):
        for i in range(S):
            a = int(torch.randint(0, cap - 80, (1,), generator=g))
            st[h, i] = a
            en[h, i] = a + int(torch.randint(1, 80, (1,), generator=g))
    return (q.to(dtype_qk), sk.to(dtype_qk), sv.to(dtype_v), (st, en, ct), ck.to(dtype_qk), cv.to(dtype_v))


def _errors(case, scale, device, monkeypatch, qk_mode="bf16", value_mode="bf16"):
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", qk_mode)
    monkeypatch.setenv("REAL_PRUNING_FUSED_VALUE_DOT_MODE", value_mode)
    q, sk, sv, (st, en, ct), ck, cv = case
    out, lse = fused_real_pruning_flat_segmented_attention(
        q=q.to(device), persisted_k=sk.to(device), persisted_v=sv.to(device), segment_starts=st.to(device),
        segment_ends=en.to(device), segment_counts=ct.to(device), current_k=ck.to(device),
        current_v=cv.to(device), softmax_scale=scale, return_lse=True, out_dtype=torch.float32)
    torch.cuda.synchronize(device)
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q).astype(np.float64), to_np(sk).astype(np.float64), to_np(sv).astype(np.float64),
        st.numpy(), en.numpy(), ct.numpy(), to_np(ck).astype(np.float64), to_np(cv).astype(np.float64),
        scale, dtype=np.float64)
    o = out.double().cpu().numpy()
    l = lse.double().cpu().numpy()
    assert np.isfinite(o).all() and np.isfinite(l).all()
    return float(np.abs(o - ref_out).max()), float(np.abs(l - ref_lse).max())


@pytest.mark.parametrize("mode", ["fp32", "ieee"])
def test_qk_fp32_mode_on_fp32_inputs(mode, device, monkeypatch):
    print(f"[dot] QK {mode}, fp32 q/k, cosine scores", flush=True)
    case = _case(81, torch.float32, torch.bfloat16, cosine=True)
    _, lse_default = _errors(case, 1.0, device, monkeypatch)
    _, lse_fp32 = _errors(case, 1.0, device, monkeypatch, qk_mode=mode)
    print(f"[dot] LSE max-abs: default {lse_default:.3e}, {mode} {lse_fp32:.3e}", flush=True)
    assert lse_fp32 <= 5e-5
    assert lse_default >= 4 * lse_fp32


@pytest.mark.parametrize("vdt", [torch.bfloat16, torch.float16, torch.float32])
def test_value_fp32_mode(vdt, device, monkeypatch):
    print(f"[dot] value fp32, v={vdt}", flush=True)
    case = _case(82, torch.bfloat16, vdt)
    scale = 0.125
    out_default, _ = _errors(case, scale, device, monkeypatch)
    out_fp32, lse_fp32 = _errors(case, scale, device, monkeypatch, value_mode="fp32")
    print(f"[dot] out max-abs: default {out_default:.3e}, fp32 {out_fp32:.3e}", flush=True)
    assert out_fp32 <= 2e-5
    assert lse_fp32 <= 2e-5
    if vdt != torch.float32:  # fp32 V already gets a 2-piece P in the default mode
        assert out_default >= 10 * out_fp32


def test_fp32_v_default_mode_beyond_tf32(device, monkeypatch):
    print("[dot] fp32 v, default value mode", flush=True)
    case = _case(83, torch.bfloat16, torch.float32)
    out_err, _ = _errors(case, 0.125, device, monkeypatch)
    print(f"[dot] out max-abs {out_err:.3e}", flush=True)
    assert out_err <= 2e-4


def test_all_fp32_modes_together(device, monkeypatch):
    """fp32 q, k and v with both knobs at fp32: every operand in 3 pieces."""
    print("[dot] fp32 everything", flush=True)
    case = _case(84, torch.float32, torch.float32, cosine=True)
    out_err, lse_err = _errors(case, 1.0, device, monkeypatch, qk_mode="ieee", value_mode="fp32")
    print(f"[dot] out max-abs {out_err:.3e} lse max-abs {lse_err:.3e}", flush=True)
    assert out_err <= 1e-4 and lse_err <= 5e-5


@pytest.mark.parametrize("mode", ["tf32", "fp32"])
@pytest.mark.parametrize("qdt,kdt", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                     (torch.float16, torch.bfloat16)])
def test_mixed_qk_dtypes(qdt, kdt, mode, device, monkeypatch):
    """q and k of different dtypes under the fp32-class QK modes, as the
    reference casts both to fp32 there (real_pruning_fused_attention.py:
    143-153): cosine-attention scores of +-100 against the fp64 oracle on the
    same (rounded) values; the fp32 mode's 3 pieces keep the LSE within 5e-5,
    the tf32 mode's 2 pieces within the contract.  The output keeps q's dtype."""
    print(f"[dot] mixed q {qdt} / k {kdt}, QK {mode}", flush=True)
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", mode)
    monkeypatch.setenv("REAL_PRUNING_FUSED_VALUE_DOT_MODE", "bf16")
    q, sk, sv, (st, en, ct), ck, cv = _case(85, torch.float32, torch.bfloat16, cosine=True)
    q, sk, ck = q.to(qdt), sk.to(kdt), ck.to(kdt)
    out, lse = fused_real_pruning_flat_segmented_attention(
        q=q.to(device), persisted_k=sk.to(device), persisted_v=sv.to(device), segment_starts=st.to(device),
        segment_ends=en.to(device), segment_counts=ct.to(device), current_k=ck.to(device),
        current_v=cv.to(device), softmax_scale=1.0, return_lse=True)
    torch.cuda.synchronize(device)
    assert out.dtype == qdt
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q).astype(np.float64), to_np(sk).astype(np.float64), to_np(sv).astype(np.float64),
        st.numpy(), en.numpy(), ct.numpy(), to_np(ck).astype(np.float64), to_np(cv).astype(np.float64),
        1.0, dtype=np.float64)
    o = out.double().cpu().numpy()
    l = lse.double().cpu().numpy()
    assert np.isfinite(o).all() and np.isfinite(l).all()
    oerr = np.abs(o - ref_out)
    lerr = float(np.abs(l - ref_lse).max())
    print(f"[dot] out max-abs {oerr.max():.3e} mean-abs {oerr.mean():.3e} lse max-abs {lerr:.3e}", flush=True)
    assert oerr.max() <= 2e-2 and oerr.mean() <= 2e-3
    assert lerr <= (5e-5 if mode == "fp32" else 1e-3)


def test_mixed_qk_dtypes_default_mode_raises(device, monkeypatch):
    """The default (bf16) QK mode takes one operand type, as the reference's
    Triton dot does."""
    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", "bf16")
    q, sk, sv, (st, en, ct), ck, cv = _case(86, torch.bfloat16, torch.bfloat16, L=64, cap=200, S=2)
    with pytest.raises(RuntimeError, match="one dtype"):
        fused_real_pruning_flat_segmented_attention(
            q=q.float().to(device), persisted_k=sk.to(device), persisted_v=sv.to(device),
            segment_starts=st.to(device), segment_ends=en.to(device), segment_counts=ct.to(device),
            current_k=ck.to(device), current_v=cv.to(device), softmax_scale=0.125)


@pytest.mark.parametrize("qk_mode,value_mode,qdt,kdt,vdt,per_cu,qpi", [
    ("bf16", "bf16", torch.bfloat16, torch.bfloat16, torch.bfloat16, 2, 128),  # 16-bit kernel
    ("tf32", "bf16", torch.float16, torch.float16, torch.float16, 2, 128),  # 16-bit kernel, exact products
    ("fp32", "bf16", torch.float32, torch.float32, torch.bfloat16, 1, 128),  # staged, 3-piece q/k
    ("bf16", "fp32", torch.bfloat16, torch.bfloat16, torch.bfloat16, 1, 128),  # staged, fp32 P V
    ("bf16", "bf16", torch.bfloat16, torch.bfloat16, torch.float32, 1, 128),  # staged, fp32 V
    ("tf32", "bf16", torch.bfloat16, torch.float32, torch.bfloat16, 1, 256),  # widened q: split-row kernel
])
def test_item_shape_slots_and_planned_calls(qk_mode, value_mode, qdt, kdt, vdt, per_cu, qpi, device, monkeypatch):
    """attention_item_shape reports the resident workgroups of the kernel
    that runs (1 per CU for the staged kernel's split modes and the split-row
    kernel, 2 for the others), and a plan built with them runs that kernel as
    accurately as the unplanned call: max-abs errors against the fp64 oracle
    within twice the unplanned call's (a cut item restarts its running max,
    which moves the rounding of P in the 16-bit value modes)."""
    from heatkv_amd import attention_item_shape, segmented_attention_plan

    monkeypatch.setenv("REAL_PRUNING_FUSED_QK_DOT_MODE", qk_mode)
    monkeypatch.setenv("REAL_PRUNING_FUSED_VALUE_DOT_MODE", value_mode)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    shape = attention_item_shape(qdt, kdt, vdt, device=device)
    print(f"[dot] item shape qk={qk_mode} value={value_mode} {qdt}/{kdt}/{vdt}: {shape}, {cus} CUs", flush=True)
    assert shape == (qpi, per_cu * cus)
    B, L, cap = 2, 700, 3000
    q, sk, sv, (st, en, ct), ck, cv = _case(87, torch.float32, torch.float32, B=B, H=3, L=L, cap=cap, S=12)
    q, sk, ck, sv, cv = q.to(qdt), sk.to(kdt), ck.to(kdt), sv.to(vdt), cv.to(vdt)
    plan = segmented_attention_plan(st, en, ct, batch_size=B, current_len=L, capacity=cap, device=device,
                                    queries_per_item=shape[0], slots=shape[1])
    ref_out, ref_lse = oattn.flat_segmented_attention(
        to_np(q).astype(np.float64), to_np(sk).astype(np.float64), to_np(sv).astype(np.float64),
        st.numpy(), en.numpy(), ct.numpy(), to_np(ck).astype(np.float64), to_np(cv).astype(np.float64),
        0.125, dtype=np.float64, workers=16)
    errs = []
    for wp in (None, plan):
        out, lse = fused_real_pruning_flat_segmented_attention(
            q=q.to(device), persisted_k=sk.to(device), persisted_v=sv.to(device), segment_starts=st.to(device),
            segment_ends=en.to(device), segment_counts=ct.to(device), current_k=ck.to(device),
            current_v=cv.to(device), softmax_scale=0.125, return_lse=True, out_dtype=torch.float32,
            work_plan=wp)
        torch.cuda.synchronize(device)
        o = out.double().cpu().numpy()
        l = lse.double().cpu().numpy()
        assert np.isfinite(o).all() and np.isfinite(l).all()
        errs.append((float(np.abs(o - ref_out).max()), float(np.abs(l - ref_lse).max())))
    print(f"[dot] max-abs (out, lse): unplanned {errs[0]}, planned {errs[1]}", flush=True)
    assert errs[1][0] <= 2 * errs[0][0] + 1e-6
    assert errs[1][1] <= 2 * errs[0][1] + 1e-6
