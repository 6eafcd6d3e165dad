"""Pins the attention oracle against checks independent of its own formula.

* brute force: pure-Python double loops in double precision on tiny shapes;
* library routine: torch's scaled_dot_product_attention (what the reference's
  CPU path calls, real_pruning_fused_attention.py:353-359) on each (b, h) over
  the explicitly gathered keys;
* closed forms: identical keys give the mean of the values with
  lse = scale q.k + ln(N); a single key gives that value;
* invariances: permuting a head's segment table entries, or relocating the
  segments to other slab offsets, leaves the output unchanged.
A planted mistake in the oracle (current keys dropped, scale applied twice)
fails these checks.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import segmented_attention as oattn


def _case(seed, B=2, H=3, L=7, cap=60, S=4, D=128):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, L, D)).astype(np.float32)
    ck = rng.standard_normal((B, H, L, D)).astype(np.float32)
    cv = rng.standard_normal((B, H, L, D)).astype(np.float32)
    sk = rng.standard_normal((B, cap, D)).astype(np.float32)
    sv = rng.standard_normal((B, cap, D)).astype(np.float32)
    st = np.zeros((H, S), np.int32)
    en = np.zeros((H, S), np.int32)
    ct = rng.integers(0, S + 1, size=H).astype(np.int32)
    for h in range(H):
        for i in range(S):
            a = int(rng.integers(0, cap))
            n = int(rng.integers(-2, 12))
            st[h, i] = a
            en[h, i] = min(cap, a + n)
    return q, sk, sv, st, en, ct, ck, cv


def _gathered(q, sk, sv, st, en, ct, ck, cv, b, h):
    idx = []
    for i in range(int(ct[h])):
        if st[h, i] < en[h, i]:
            idx.extend(range(int(st[h, i]), int(en[h, i])))
    keys = np.concatenate([sk[b, idx], ck[b, h]], 0)
    vals = np.concatenate([sv[b, idx], cv[b, h]], 0)
    return keys, vals


def test_brute_force_tiny():
    q, sk, sv, st, en, ct, ck, cv = _case(0, B=1, H=2, L=3, cap=12, S=3, D=8)
    scale = 0.37
    out, lse = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale, dtype=np.float64)
    D = q.shape[-1]
    for h in range(2):
        keys, vals = _gathered(q, sk, sv, st, en, ct, ck, cv, 0, h)
        bo, bl = oattn.brute_force_attention(q[0, h].tolist(), keys.tolist(), vals.tolist(), scale)
        np.testing.assert_allclose(out[0, :, h * D:(h + 1) * D], np.array(bo), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse[0, h], np.array(bl), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_matches_torch_sdpa(seed):
    q, sk, sv, st, en, ct, ck, cv = _case(seed)
    scale = 1 / math.sqrt(128)
    out, lse = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale)
    D = q.shape[-1]
    for b in range(q.shape[0]):
        for h in range(q.shape[1]):
            keys, vals = _gathered(q, sk, sv, st, en, ct, ck, cv, b, h)
            tq = torch.from_numpy(q[b, h]).double()[None, None]
            tk = torch.from_numpy(keys).double()[None, None]
            tv = torch.from_numpy(vals).double()[None, None]
            ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, scale=scale)[0, 0]
            np.testing.assert_allclose(out[b, :, h * D:(h + 1) * D], ref.numpy(), atol=2e-6, rtol=1e-5)
            ref_lse = torch.logsumexp(scale * tq[0, 0] @ tk[0, 0].T, dim=-1)
            np.testing.assert_allclose(lse[b, h], ref_lse.numpy(), atol=2e-5)


def test_identical_keys_give_mean_of_values():
    rng = np.random.default_rng(4)
    B, H, L, D, cap = 1, 2, 5, 128, 30
    q = rng.standard_normal((B, H, L, D)).astype(np.float32)
    key = rng.standard_normal(D).astype(np.float32)
    ck = np.broadcast_to(key, (B, H, L, D)).copy()
    sk = np.broadcast_to(key, (B, cap, D)).copy()
    cv = rng.standard_normal((B, H, L, D)).astype(np.float32)
    sv = rng.standard_normal((B, cap, D)).astype(np.float32)
    st = np.array([[0, 20], [5, 0]], np.int32)
    en = np.array([[10, 30], [15, 0]], np.int32)
    ct = np.array([2, 1], np.int32)
    scale = 0.2
    out, lse = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale, dtype=np.float64)
    for h, rows in ((0, list(range(0, 10)) + list(range(20, 30))), (1, list(range(5, 15)))):
        vals = np.concatenate([sv[0, rows], cv[0, h]], 0).astype(np.float64)
        n = vals.shape[0]
        np.testing.assert_allclose(out[0, :, h * D:(h + 1) * D], np.broadcast_to(vals.mean(0), (L, D)),
                                   atol=1e-12)
        np.testing.assert_allclose(lse[0, h], scale * (q[0, h].astype(np.float64) @ key) + math.log(n),
                                   atol=1e-9)


def test_single_key_returns_its_value():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 1, 1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 1, 1, 128)).astype(np.float32)
    v = rng.standard_normal((1, 1, 1, 128)).astype(np.float32)
    z = np.zeros((1, 0), np.int32)
    out, lse = oattn.flat_segmented_attention(q, None, None, z, z, np.zeros(1, np.int32), k, v, 0.5,
                                              dtype=np.float64)
    np.testing.assert_allclose(out[0, 0], v[0, 0, 0], atol=1e-15)
    np.testing.assert_allclose(lse[0, 0, 0], 0.5 * float(q[0, 0, 0].astype(np.float64) @ k[0, 0, 0]),
                               atol=1e-12)


def test_segment_permutation_and_relocation_invariance():
    q, sk, sv, st, en, ct, ck, cv = _case(6, cap=80, S=5)
    scale = 0.09
    base, base_lse = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale, dtype=np.float64)
    # permute each head's live entries
    st2, en2 = st.copy(), en.copy()
    for h in range(st.shape[0]):
        n = int(ct[h])
        perm = np.random.default_rng(h).permutation(n)
        st2[h, :n] = st[h, :n][perm]
        en2[h, :n] = en[h, :n][perm]
    out, lse = oattn.flat_segmented_attention(q, sk, sv, st2, en2, ct, ck, cv, scale, dtype=np.float64)
    np.testing.assert_allclose(out, base, atol=1e-12)
    np.testing.assert_allclose(lse, base_lse, atol=1e-12)
    # relocate every live segment to a fresh region of a larger slab
    B, cap, D = sk.shape
    cap2 = cap * 10
    sk2 = np.zeros((B, cap2, D), np.float32)
    sv2 = np.zeros((B, cap2, D), np.float32)
    st3, en3 = st.copy(), en.copy()
    cursor = 7
    for h in range(st.shape[0]):
        for i in range(int(ct[h])):
            a, e = int(st[h, i]), int(en[h, i])
            n = max(e - a, 0)
            sk2[:, cursor:cursor + n] = sk[:, a:a + n]
            sv2[:, cursor:cursor + n] = sv[:, a:a + n]
            st3[h, i] = cursor
            en3[h, i] = cursor + n if n > 0 else cursor - 1
            cursor += n + 3
    out, lse = oattn.flat_segmented_attention(q, sk2, sv2, st3, en3, ct, ck, cv, scale, dtype=np.float64)
    np.testing.assert_allclose(out, base, atol=1e-12)
    np.testing.assert_allclose(lse, base_lse, atol=1e-12)


def test_planted_mistakes_are_caught(monkeypatch):
    """A wrong oracle (current keys dropped / scale twice) fails the SDPA check."""
    q, sk, sv, st, en, ct, ck, cv = _case(8, B=1, H=1)
    ct[:] = 2
    st[0, :2] = [0, 10]
    en[0, :2] = [8, 20]
    scale = 0.1
    keys, vals = _gathered(q, sk, sv, st, en, ct, ck, cv, 0, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q[0, 0])[None, None], torch.from_numpy(keys)[None, None],
        torch.from_numpy(vals)[None, None], scale=scale)[0, 0].numpy()
    good, _ = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale)
    assert np.abs(good[0] - ref).max() < 1e-5
    no_cur, _ = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck * 0 - 1e9, cv, scale)
    assert np.abs(no_cur[0] - ref).max() > 1e-2
    twice, _ = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, scale * scale)
    assert np.abs(twice[0] - ref).max() > 1e-2


def test_attention_flops_closed_form():
    st = np.array([[0, 5], [3, 0]], np.int32)
    en = np.array([[4, 9], [2, 0]], np.int32)  # head 1: start >= end, skipped
    ct = np.array([2, 1], np.int32)
    assert oattn.attention_flops(ct, st, en, batch=2, cur_len=10, head_dim=128) == \
        2 * (4 * 10 * (8 + 10) * 128 + 4 * 10 * (0 + 10) * 128)


@pytest.mark.parametrize("seed", [4, 5])
def test_thread_pool_gives_the_same_result(seed):
    q, sk, sv, st, en, ct, ck, cv = _case(seed, B=3, H=4)
    one = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, 0.1)
    many = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, 0.1, workers=5)
    assert np.array_equal(one[0], many[0]) and np.array_equal(one[1], many[1])


@pytest.mark.parametrize("seed", [6, 7])
def test_sdpa_restatement_matches_brute_force_and_numpy(seed):
    """The torch restatement (timed as the CPU baseline) against the pure-Python
    brute force on a small case and the numpy oracle on a larger one; a planted
    mistake (current keys dropped) fails the comparison."""
    q, sk, sv, st, en, ct, ck, cv = _case(seed, B=1, H=2, L=3, cap=12, S=3, D=8)
    got = oattn.flat_segmented_attention_sdpa(*(torch.from_numpy(x) for x in (q, sk, sv)), st, en, ct,
                                              torch.from_numpy(ck), torch.from_numpy(cv), 0.29).numpy()
    D = q.shape[-1]
    for h in range(2):
        keys, vals = _gathered(q, sk, sv, st, en, ct, ck, cv, 0, h)
        bo, _ = oattn.brute_force_attention(q[0, h].tolist(), keys.tolist(), vals.tolist(), 0.29)
        np.testing.assert_allclose(got[0, :, h * D:(h + 1) * D], np.array(bo), rtol=1e-5, atol=1e-6)
    q, sk, sv, st, en, ct, ck, cv = _case(seed, B=2, H=3, L=20, cap=80, S=5)
    t = lambda x: torch.from_numpy(x)  # noqa: E731
    got = oattn.flat_segmented_attention_sdpa(t(q), t(sk), t(sv), st, en, ct, t(ck), t(cv), 0.088).numpy()
    ref, _ = oattn.flat_segmented_attention(q, sk, sv, st, en, ct, ck, cv, 0.088)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)
    bad = oattn.flat_segmented_attention_sdpa(t(q), t(sk), t(sv), st, en, ct, t(ck[:, :, :1]), t(cv[:, :, :1]),
                                              0.088).numpy()
    assert np.abs(bad - ref).max() > 1e-2
