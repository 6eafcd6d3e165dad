"""The allocation-free attention entry point against the workspace one.

``hkv_segmented_attention_noalloc`` takes its round-split workspace from a
static device array of the library instead of the caller.  Two calls in a
row through the C ABI -- a 2304-query step (576 items: more than one round of
workgroup slots, so items are cut and merged through the array) and then a
smaller 1024-query step (256 items, cut as well) -- must give bit-identical
results to ``hkv_segmented_attention`` with a caller workspace on the same
inputs (same kernels, same split), with every output row written (NaN
prefill) and within the contract tolerances of the oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import _lib
from oracle import segmented_attention as oattn
from support import assert_attention_close, bits, to_np

pytestmark = pytest.mark.gpu


def _case(seed, B, H, L, cap, S):
    g = torch.Generator().manual_seed(seed)
    q, ck, cv = (torch.randn((B, H, L, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    sk, sv = (torch.randn((B, cap, 128), generator=g).to(torch.bfloat16) for _ in range(2))
    st = torch.zeros((H, S), dtype=torch.int32)
    en = torch.zeros((H, S), dtype=torch.int32)
    ct = torch.randint(0, S + 1, (H,), generator=g, dtype=torch.int32)
    for h in range(H):
        for i in range(S):
            a = int(torch.randint(0, cap - 300, (1,), generator=g))
            st[h, i] = a
            en[h, i] = a + int(torch.randint(1, 300, (1,), generator=g))
    return q, sk, sv, (st, en, ct), ck, cv


def _call(entry, case, device, workspace):
    q, sk, sv, tables, ck, cv = (x.to(device) if torch.is_tensor(x) else x for x in case)
    st, en, ct = (t.to(device) for t in tables)
    B, H, L, D = q.shape
    out = torch.full((B, L, H * D), float("nan"), dtype=q.dtype, device=device)
    lse = torch.full((B, H, L), float("nan"), dtype=torch.float32, device=device)
    args = [q.data_ptr(), sk.data_ptr(), sv.data_ptr(), st.data_ptr(), en.data_ptr(), ct.data_ptr(),
            ck.data_ptr(), cv.data_ptr(), out.data_ptr(), lse.data_ptr(), B, H, L, int(sk.shape[1]),
            int(st.shape[1]), D, 2, 2, 2, 0, 1.0 / math.sqrt(128), 0, 0, 0, None, 0]
    if workspace is not None:
        args += [workspace.data_ptr(), int(workspace.numel())]
    code = entry(*args, torch.cuda.current_stream(device).cuda_stream)
    _lib.check(code)
    return out, lse


def test_noalloc_matches_workspace_entry_twice(device):
    lib = _lib.load()
    ws = torch.zeros(int(lib.hkv_segmented_attention_workspace_bytes(device.index or 0)), dtype=torch.uint8,
                     device=device)
    for seed, L in ((91, 2304), (92, 1024)):  # the second call is smaller
        print(f"[noalloc] B=2 H=16 L={L}", flush=True)
        case = _case(seed, 2, 16, L, 3000, 8)
        got, got_lse = _call(lib.hkv_segmented_attention_noalloc, case, device, None)
        want, want_lse = _call(lib.hkv_segmented_attention, case, device, ws)
        torch.cuda.synchronize(device)
        assert torch.isfinite(got.float()).all() and torch.isfinite(got_lse).all()
        assert np.array_equal(bits(got), bits(want)) and np.array_equal(bits(got_lse), bits(want_lse))
        q, sk, sv, (st, en, ct), ck, cv = case
        ref_out, ref_lse = oattn.flat_segmented_attention(
            to_np(q), to_np(sk), to_np(sv), st.numpy(), en.numpy(), ct.numpy(), to_np(ck), to_np(cv),
            1.0 / math.sqrt(128), workers=16)
        assert_attention_close(to_np(got), to_np(got_lse), ref_out, ref_lse, what=f"noalloc L={L}")
