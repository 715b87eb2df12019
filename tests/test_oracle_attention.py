"""Pins of oracle/attention.py: closed forms, invariants and the agreement of
the reference's two delta-net paths (the float32 Numba loop of
engine/numba_kernels.py:11-45 and the NumPy fallback of
engine/qwen35.py:248-252), chosen so that a dropped term, a wrong index or a
wrong scale fails one of them."""
import math

import numpy as np
import pytest

from oracle import attention as oatt


def rand_cache(rng, max_seq, nkv, hd):
    return (rng.standard_normal((max_seq, nkv, hd)).astype(np.float32),
            rng.standard_normal((max_seq, nkv, hd)).astype(np.float32))


# ---------------------------------------------------------------- attention

def test_single_position_returns_v():
    rng = np.random.default_rng(1)
    nh, nkv, hd = 8, 2, 64
    kc, vc = rand_cache(rng, 16, nkv, hd)
    q = rng.standard_normal(nh * hd)
    kn, vn = rng.standard_normal(nkv * hd), rng.standard_normal(nkv * hd)
    out, kc2, vc2 = oatt.gqa_decode(q, kc, vc, 0, nh, nkv, hd, k_new=kn, v_new=vn)
    g = nh // nkv
    want = np.repeat(vn.reshape(nkv, hd).astype(np.float32), g, axis=0).reshape(-1)
    np.testing.assert_allclose(out, want, rtol=0, atol=1e-12)
    np.testing.assert_array_equal(kc2[0], kn.reshape(nkv, hd).astype(np.float32))
    np.testing.assert_array_equal(kc2[1:], kc[1:])


def test_equal_keys_average_the_values():
    rng = np.random.default_rng(2)
    nh, nkv, hd, pos = 4, 4, 64, 9
    kc, vc = rand_cache(rng, 16, nkv, hd)
    kc[:] = kc[0]
    out, _, _ = oatt.gqa_decode(rng.standard_normal(nh * hd), kc, vc, pos, nh, nkv, hd)
    np.testing.assert_allclose(out, vc[:pos + 1].astype(np.float64).mean(axis=0).reshape(-1), rtol=1e-12,
                               atol=1e-12)


def test_two_positions_logistic_weights_pin_the_scale():
    # keys 0 and a q-parallel key: the weight of position 1 is the logistic of
    # (q . k1) / sqrt(head_dim)
    rng = np.random.default_rng(3)
    hd = 128
    q = rng.standard_normal(hd)
    kc = np.zeros((2, 1, hd), np.float32)
    kc[1, 0] = (0.05 * q).astype(np.float32)
    vc = rng.standard_normal((2, 1, hd)).astype(np.float32)
    out, _, _ = oatt.gqa_decode(q, kc, vc, 1, 1, 1, hd)
    a = float(np.dot(q, kc[1, 0].astype(np.float64))) / math.sqrt(hd)
    w1 = 1.0 / (1.0 + math.exp(-a))
    v64 = vc.astype(np.float64)
    np.testing.assert_allclose(out, (1 - w1) * v64[0, 0] + w1 * v64[1, 0], rtol=1e-12, atol=1e-12)


def test_query_head_reads_kv_head_h_div_g():
    rng = np.random.default_rng(4)
    nh, nkv, hd = 12, 3, 64
    kc, vc = rand_cache(rng, 8, nkv, hd)
    for j in range(nkv):
        vc[:, j, :] = 10.0 * (j + 1)
    out, _, _ = oatt.gqa_decode(rng.standard_normal(nh * hd), kc, vc, 5, nh, nkv, hd)
    heads = out.reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_allclose(heads[h], 10.0 * (h // (nh // nkv) + 1), rtol=1e-12)


def test_window_hides_older_positions():
    rng = np.random.default_rng(5)
    nh, nkv, hd, pos, win = 4, 2, 64, 20, 6
    kc, vc = rand_cache(rng, 32, nkv, hd)
    q = rng.standard_normal(nh * hd)
    a, _, _ = oatt.gqa_decode(q, kc, vc, pos, nh, nkv, hd, window=win)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:pos + 1 - win] = 100.0
    vc2[:pos + 1 - win] = -7.0
    b, _, _ = oatt.gqa_decode(q, kc2, vc2, pos, nh, nkv, hd, window=win)
    np.testing.assert_array_equal(a, b)
    c, _, _ = oatt.gqa_decode(q, kc2, vc2, pos, nh, nkv, hd)
    assert np.abs(c - a).max() > 1.0


def test_gate_closed_forms():
    rng = np.random.default_rng(6)
    nh, nkv, hd = 2, 1, 64
    kc, vc = rand_cache(rng, 4, nkv, hd)
    q = rng.standard_normal(nh * hd)
    base, _, _ = oatt.gqa_decode(q, kc, vc, 3, nh, nkv, hd)
    half, _, _ = oatt.gqa_decode(q, kc, vc, 3, nh, nkv, hd, gate=np.zeros(nh * hd))
    np.testing.assert_allclose(half, 0.5 * base, rtol=1e-15)
    big, _, _ = oatt.gqa_decode(q, kc, vc, 3, nh, nkv, hd, gate=np.full(nh * hd, 1000.0))
    np.testing.assert_allclose(big, base / (1.0 + math.exp(-80.0)), rtol=1e-15)


def test_float32_form_agrees_with_fp64():
    rng = np.random.default_rng(13)
    nh, nkv, hd, pos = 16, 4, 128, 300
    kc, vc = rand_cache(rng, 512, nkv, hd)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    a, _, _ = oatt.gqa_decode(q, kc, vc, pos, nh, nkv, hd, window=200)
    b = oatt.gqa_decode_f32(q, kc, vc, pos, nh, nkv, hd, window=200)
    assert b.dtype == np.float32
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()


# ---------------------------------------------------------------- delta net

def rand_step(rng, heads=4, kd=32, vd=24):
    state = rng.standard_normal((heads, kd, vd)).astype(np.float32)
    q = rng.standard_normal((heads, kd)).astype(np.float32)
    k = rng.standard_normal((heads, kd)).astype(np.float32)
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    v = rng.standard_normal((heads, vd)).astype(np.float32)
    decay = -rng.uniform(0.01, 2.0, heads).astype(np.float32)
    beta = rng.uniform(0.05, 0.95, heads).astype(np.float32)
    return state, q, k, v, decay, beta


def test_float32_loop_matches_the_fp64_fallback():
    rng = np.random.default_rng(7)
    args = rand_step(rng)
    S, core = oatt.delta_net_step(*args)
    S64, core64 = oatt.delta_net_step_f64(*args)
    assert np.abs(S - S64).max() <= 1e-5 * np.abs(S64).max()
    assert np.abs(core - core64).max() <= 1e-5 * np.abs(core64).max()


def test_zero_beta_is_pure_decay():
    rng = np.random.default_rng(8)
    state, q, k, v, decay, _ = rand_step(rng)
    S, core = oatt.delta_net_step(state, q, k, v, decay, np.zeros(4, np.float32))
    f = np.exp(decay.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(S, state * f[:, None, None])
    np.testing.assert_allclose(core, np.einsum('hkv,hk->hv', S.astype(np.float64), q.astype(np.float64)),
                               rtol=1e-5, atol=1e-5)


def test_one_hot_key_with_unit_beta_replaces_the_row():
    rng = np.random.default_rng(9)
    state, q, _, v, _, _ = rand_step(rng)
    j = 5
    k = np.zeros_like(q)
    k[:, j] = 1.0
    S, _ = oatt.delta_net_step(state, q, k, v, np.zeros(4, np.float32), np.ones(4, np.float32))
    # row j = S_j + fl(v - S_j): v up to the rounding of that difference
    np.testing.assert_allclose(S[:, j, :], v, rtol=0, atol=2.0 ** -22 * np.abs(state).max())
    assert np.abs(S[:, j, :] - v).max() < np.abs(state[:, j, :] - v).max() * 1e-5
    rest = [i for i in range(state.shape[1]) if i != j]
    np.testing.assert_array_equal(S[:, rest, :], state[:, rest, :])


def test_predicted_value_gives_no_update():
    rng = np.random.default_rng(10)
    state, q, k, _, _, beta = rand_step(rng)
    # decay 0 and v = S^T k computed in the loop's own order: delta is exactly 0
    k = np.zeros_like(k)
    k[:, 3] = 1.0
    v = state[:, 3, :].copy()
    S, core = oatt.delta_net_step(state, q, k, v, np.zeros(4, np.float32), beta)
    np.testing.assert_array_equal(S, state)


@pytest.mark.parametrize('seed', [11, 12])
def test_update_is_rank_one(seed):
    rng = np.random.default_rng(seed)
    args = rand_step(rng)
    S64, _ = oatt.delta_net_step_f64(*args)
    state, _, k, _, decay, _ = args
    diff = S64 - np.exp(decay.astype(np.float64))[:, None, None] * state.astype(np.float64)
    for h in range(diff.shape[0]):
        s = np.linalg.svd(diff[h], compute_uv=False)
        assert s[1] <= 1e-10 * s[0]
