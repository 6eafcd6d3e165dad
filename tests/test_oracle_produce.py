"""Pins of the QKV-prologue oracle (oracle/produce.py) and of the host RoPE tables.

Each check is fixed by something other than the oracle's own formula: hand
values of the index rounding, closed-form angles, complex multiplication,
norm preservation, the relative-position property of RoPE and torch's own
bf16 conversion.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from heatkv_amd import produce as P
from heatkv_amd.slab_schedule import SIDES_1M
from oracle import produce as O

SCHED_1M = [(1, s, s) for s in SIDES_1M]


def test_star_indices_hand_values():
    # round(i * 64 / side): 64/3 = 21.33, 42.67; 64/5 = 12.8, 25.6, 38.4, 51.2
    assert O.star_indices(3, 64).tolist() == [0, 21, 43]
    assert O.star_indices(5, 64).tolist() == [0, 13, 26, 38, 51]
    assert O.star_indices(1, 64).tolist() == [0]
    assert O.star_indices(64, 64).tolist() == list(range(64))
    assert O.star_indices(2, 64).tolist() == [0, 32]


def test_grid_angles_closed_form():
    ang = O.grid_angles(128)
    # 32 row entries then 32 column entries; inv_freq[j] = 10000^(-j/32)
    assert ang.shape == (128, 128, 64)
    assert ang[1, 0, 0] == 1.0 and ang[0, 1, 32] == 1.0
    assert ang[0, 1, 0] == 0.0 and ang[1, 0, 32] == 0.0
    assert math.isclose(ang[3, 0, 1], 3 * 10000 ** (-1 / 32), rel_tol=1e-15)
    assert math.isclose(ang[0, 5, 33], 5 * 10000 ** (-1 / 32), rel_tol=1e-15)
    assert math.isclose(ang[127, 0, 31], 127 * 10000 ** (-31 / 32), rel_tol=1e-15)


def test_table_position_zero_is_identity_and_known_rows():
    t = O.rope_table(128, SCHED_1M, mode=2, pad_to_multiplier=128)
    assert t.shape == (2, 10624, 64)
    assert np.all(t[0, 0] == 1.0) and np.all(t[1, 0] == 0.0)
    assert np.all(t[:, 10521:] == 0.0)
    # scale 1 is 2x2 at grid rows/cols {0, 32}: table rows 1..4 are
    # (0, 0), (0, 32), (32, 0), (32, 32)
    assert np.all(t[0, 1] == 1.0)
    assert math.isclose(t[0, 2, 32], math.cos(32.0)) and math.isclose(t[1, 2, 32], math.sin(32.0))
    assert t[0, 2, 0] == 1.0 and t[0, 3, 32] == 1.0
    assert math.isclose(t[1, 3, 0], math.sin(32.0)) and t[1, 4, 32] == t[1, 4, 0] == t[1, 3, 0]


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_host_table_matches_oracle(mode):
    got = P.rope2d_freqs_table(128, SCHED_1M, rope2d_normalized_by_hw=mode, pad_to_multiplier=128)
    want = O.rope_table(128, SCHED_1M, mode=mode, pad_to_multiplier=128)
    assert tuple(got.shape) == want.shape and got.dtype == torch.float32
    # fp32 angles of up to 127 rad (the product) against float64 ones
    np.testing.assert_allclose(got.numpy(), want, rtol=0, atol=2e-5)


def test_grid_dict_keys_and_layout():
    drhw = {1.0: {"1M": {"scales": SCHED_1M}, "0.06M": {"scales": SCHED_1M[:7]}}}
    grid = P.precompute_rope2d_freqs_grid(128, drhw, 2, pad_to_multiplier=128)
    assert set(grid) == {P.schedule_key(SCHED_1M), P.schedule_key(SCHED_1M[:7])}
    g = grid[P.schedule_key(SCHED_1M[:7])]
    assert tuple(g.shape) == (2, 1, 1, 1, 10624, 64)
    assert P.rope_start(SCHED_1M, 0) == 0 and P.rope_start(SCHED_1M, 3) == 1 + 4 + 16
    assert P.rope_start(SCHED_1M, 12) == 10521 - 4096


def test_rotation_is_complex_multiplication_and_invertible():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 7, 128)).astype(np.float32)
    a = rng.uniform(-40, 40, (7, 64))
    got = O.rotate_pairs(x, np.cos(a), np.sin(a))
    z = (x[..., 0::2].astype(np.float64) + 1j * x[..., 1::2]) * np.exp(1j * a)
    np.testing.assert_allclose(got[..., 0::2], z.real, atol=2e-6)
    np.testing.assert_allclose(got[..., 1::2], z.imag, atol=2e-6)
    back = O.rotate_pairs(got, np.cos(-a), np.sin(-a))
    np.testing.assert_allclose(back, x, atol=4e-6)
    np.testing.assert_allclose(np.hypot(got[..., 0::2], got[..., 1::2]),
                               np.hypot(x[..., 0::2], x[..., 1::2]), rtol=2e-6)


def test_relative_position_property_mode0():
    # <R(p1) q, R(p2) k> depends on p2 - p1 only: shift both positions
    t = O.rope_table(128, [(1, 16, 16)], mode=0)
    rng = np.random.default_rng(1)
    q = rng.standard_normal((1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 128)).astype(np.float32)

    def dot(p1, p2):
        r1 = O.rotate_pairs(q, t[0, [p1]], t[1, [p1]])
        r2 = O.rotate_pairs(k, t[0, [p2]], t[1, [p2]])
        return float(np.sum(r1.astype(np.float64) * r2))

    tok = lambda r, c: r * 16 + c  # noqa: E731
    assert math.isclose(dot(tok(1, 2), tok(4, 7)), dot(tok(6, 3), tok(9, 8)), abs_tol=1e-4)
    assert math.isclose(dot(tok(0, 0), tok(3, 3)), dot(tok(5, 9), tok(8, 12)), abs_tol=1e-4)
    assert not math.isclose(dot(tok(0, 0), tok(3, 3)), dot(tok(0, 0), tok(3, 4)), abs_tol=1e-3)


def test_produce_norms_identity_and_bias():
    rng = np.random.default_rng(2)
    B, L, H, D = 2, 5, 3, 128
    qkv = O.bf16_round(rng.standard_normal((B, L, 3, H, D)).astype(np.float32) * 3)
    sm = np.array([4.0, 17.5, 100.0], np.float32)
    table = O.rope_table(D, [(1, 1, 1), (1, 2, 2), (1, 4, 4)], mode=2).astype(np.float32)
    q, k, v = O.produce(qkv, scale_mul=sm, table=table, start=5)
    np.testing.assert_allclose(np.linalg.norm(q, axis=-1), np.broadcast_to(sm[None, :, None], (B, H, L)),
                               rtol=2e-6)
    np.testing.assert_allclose(np.linalg.norm(k, axis=-1), 1.0, rtol=2e-6)
    assert np.array_equal(v, qkv[:, :, 2].transpose(0, 2, 1, 3))
    # token 0 of the table: identity rotation
    q0, k0, _ = O.produce(qkv[:, :1], scale_mul=sm, table=table, start=0)
    q1, k1, _ = O.produce(qkv[:, :1], scale_mul=sm)
    assert np.array_equal(q0, q1) and np.array_equal(k0, k1)
    # biases: q bias enters before the normalization, v bias is rounded to bf16
    qb = rng.standard_normal(H * D).astype(np.float32)
    vb = rng.standard_normal(H * D).astype(np.float32)
    qq, _, vv = O.produce(qkv, q_bias=qb, v_bias=vb, normalize=False)
    np.testing.assert_array_equal(qq, (qkv[:, :, 0] + qb.reshape(H, D)).transpose(0, 2, 1, 3))
    vt = torch.from_numpy((qkv[:, :, 2] + vb.reshape(H, D)).transpose(0, 2, 1, 3).copy())
    np.testing.assert_array_equal(vv, vt.to(torch.bfloat16).float().numpy())


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10,
                        np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -0.0, 65504.0, 1e-40], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(O.bf16_round(x), want)
    assert O.bf16_round(np.array([1 + 2 ** -8], np.float32))[0] == 1.0
    assert O.bf16_round(np.array([1 + 3 * 2 ** -8], np.float32))[0] == 1 + 2 ** -6


def test_torch_composition_matches_oracle():
    """The reference's torch op sequence (fp32 on the CPU) against the oracle."""
    rng = np.random.default_rng(4)
    B, L, H, D = 2, 16, 4, 128
    qkv = O.bf16_round(rng.standard_normal((B, L, 3, H, D)).astype(np.float32))
    sm = np.array([4.0, 8.0, 30.0, 100.0], np.float32)
    table = P.rope2d_freqs_table(D, SCHED_1M, 2, 128)
    start = P.rope_start(SCHED_1M, 4)
    from tests.support import torch_qkv_prologue

    tq, tk, tv = torch_qkv_prologue(torch.from_numpy(qkv), torch.from_numpy(sm), table, start)
    q, k, v = O.produce(qkv, scale_mul=sm, table=table.numpy(), start=start)
    np.testing.assert_allclose(tq.numpy(), q, rtol=0, atol=4e-6 * 100)
    np.testing.assert_allclose(tk.numpy(), k, rtol=0, atol=4e-6)
    np.testing.assert_array_equal(tv.numpy(), v)
