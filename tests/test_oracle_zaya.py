"""Pins of the ZAYA MoE block oracle (oracle/zaya_moe.py) on the CPU: the
reference's GELU test values (tests/test_zaya.py:117-122), closed forms for
GELU, RMSNorm and softmax, the skip route, EDA and the expert path against a
direct computation."""
import math

import numpy as np
from scipy.special import erf

from oracle import zaya_moe as zm


def test_gelu_reference_test_values():
    r = zm.gelu(np.array([-4.0, 0.0, 4.0], dtype=np.float32))
    assert np.isfinite(r).all()
    assert float(r[1]) == 0.0
    assert float(r[0]) < 0.0 and float(r[2]) > 3.9


def test_gelu_closed_form():
    x = np.linspace(-6, 6, 1001).astype(np.float32)
    want = x.astype(np.float64) * 0.5 * (1.0 + erf(x.astype(np.float64) / math.sqrt(2.0)))
    got = zm.gelu(x).astype(np.float64)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 2.5e-7


def test_rmsnorm_constant_vector():
    x = np.full(256, -3.0, np.float32)
    w = np.linspace(0.5, 2.0, 256).astype(np.float32)
    got = zm.rmsnorm(x, w, 1e-5)
    np.testing.assert_allclose(got, -w / math.sqrt(1.0 + 1e-5 / 9.0), rtol=1e-6)


def _tensors(rng, E=4, H=64, I=32, R=16):
    t = {'inp': rng.standard_normal((R, H)).astype(np.float32), 'inp_b': None,
         'eda': rng.standard_normal(R).astype(np.float32), 'norm': rng.uniform(0.5, 1.5, R).astype(np.float32),
         'gate': rng.standard_normal((R, R)).astype(np.float32) / 4, 'gate_b': None,
         'mlp2': rng.standard_normal((R, R)).astype(np.float32) / 4, 'mlp2_b': None,
         'mlp4': rng.standard_normal((E + 1, R)).astype(np.float32), 'mlp4_b': None,
         'route_bias': np.zeros(E + 1, np.float32),
         'gate_up': rng.standard_normal((E, 2 * I, H)).astype(np.float32) / 8,
         'down': rng.standard_normal((E, H, I)).astype(np.float32) / 8}
    return t


def test_softmax_sums_to_one_and_expert_path():
    rng = np.random.default_rng(1)
    t = _tensors(rng)
    h = rng.standard_normal(64).astype(np.float32)
    moe, state, probs, e, margin = zm.moe_block(t, 4, 1e-5, h, None)
    assert abs(float(probs.sum()) - 1.0) < 1e-6
    assert e == int(np.argmax(probs)) and margin >= 0
    np.testing.assert_allclose(state, t['inp'].astype(np.float64) @ h, rtol=1e-5)
    g = t['gate_up'][e].astype(np.float64) @ h
    gate, up = g[:32], g[32:]
    want = (t['down'][e].astype(np.float64) @ (gate / (1 + np.exp(-gate)) * up)) * probs[e]
    np.testing.assert_allclose(moe, want, rtol=1e-4, atol=1e-6)


def test_skip_route_and_forced_expert():
    rng = np.random.default_rng(2)
    t = _tensors(rng)
    h = rng.standard_normal(64).astype(np.float32)
    t['route_bias'][4] = 10.0
    moe, _, probs, e, _ = zm.moe_block(t, 4, 1e-5, h, None)
    assert e == 4
    np.testing.assert_array_equal(moe, h * probs[4])
    t['route_bias'][4] = 0.0
    t['route_bias'][2] = 10.0
    assert zm.moe_block(t, 4, 1e-5, h, None)[3] == 2


def test_eda_adds_prev_times_eda():
    rng = np.random.default_rng(3)
    t = _tensors(rng)
    h = rng.standard_normal(64).astype(np.float32)
    prev = rng.standard_normal(16).astype(np.float32)
    _, s0, _, _, _ = zm.moe_block(t, 4, 1e-5, h, None)
    _, s1, _, _, _ = zm.moe_block(t, 4, 1e-5, h, prev)
    np.testing.assert_array_equal(s1, s0 + prev * t['eda'])
    t['eda'] = None
    _, s2, _, _, _ = zm.moe_block(t, 4, 1e-5, h, prev)
    np.testing.assert_array_equal(s2, s0)


def test_softmax_pinned_by_scipy_on_known_logits():
    """With W_mlp4 zero the logits are exactly its bias b (0 + b in fp32), so
    the oracle's probabilities must be scipy.special.softmax(b) whatever the
    router MLP computed: a softmax of 2 * logits, a missing max shift that
    overflows, or a dropped term all fail here."""
    from scipy.special import softmax
    rng = np.random.default_rng(4)
    t = _tensors(rng)
    h = rng.standard_normal(64).astype(np.float32)
    t['mlp4'] = np.zeros_like(t['mlp4'])
    for scale in (0.1, 1.0, 8.0, 60.0, 200.0):
        b = (rng.standard_normal(5) * scale).astype(np.float32)
        t['mlp4_b'] = b
        _, _, probs, e, _ = zm.moe_block(t, 4, 1e-5, h, None)
        want = softmax(b.astype(np.float64))
        big = want > 1e-30
        # fp32 evaluation: the shifted logit b - max(b) carries its own
        # rounding, which exp turns into a relative error of |b - max| * 2^-24
        tol = (np.abs(b.astype(np.float64) - b.max()) + 8.0) * 2.0 ** -23
        assert np.all(np.abs(probs[big] - want[big]) / want[big] <= tol[big])
        assert np.all(np.abs(probs[~big]) < 1e-30)
        assert e == int(np.argmax(b))


def test_two_route_softmax_is_the_logistic():
    """Two routes (one expert + the skip route): probs[1] = expit(b1 - b0)
    exactly in closed form; the skip route wins when its logit is larger."""
    from scipy.special import expit
    rng = np.random.default_rng(5)
    t = _tensors(rng, E=1)
    h = rng.standard_normal(64).astype(np.float32)
    t['mlp4'] = np.zeros_like(t['mlp4'])
    for d in (-30.0, -5.0, -0.5, 0.25, 3.0, 20.0):
        t['mlp4_b'] = np.array([0.0, d], np.float32)
        _, _, probs, e, _ = zm.moe_block(t, 1, 1e-5, h, None)
        assert abs(float(probs[1]) - expit(d)) <= 1e-6 * expit(d) + 1e-12
        assert abs(float(probs[0]) - expit(-d)) <= 1e-6 * expit(-d) + 1e-12
        assert e == (1 if d > 0 else 0)
