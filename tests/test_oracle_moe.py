"""Pins the MoE composition oracle (oracle/moe.py). The reference has no top-k
MoE and no MoE test, so these are invariants and reductions to pinned pieces."""
import math

import numpy as np

from oracle import moe, quant


def test_router_logit_is_correctly_rounded_sum():
    rng = np.random.default_rng(0)
    h = rng.standard_normal((3, 2048)).astype(np.float32)
    w = (rng.standard_normal((16, 2048)) * 0.02).astype(np.float32)
    got = moe.router_logits(h, w)
    for t in range(3):
        for e in range(16):
            exact = math.fsum(float(a) * float(b) for a, b in zip(h[t], w[e]))   # exact sum
            # the fixed-order fp64 sum is within a few fp64 ulps of exact, so the
            # fp32 rounding agrees except when exact sits on a rounding boundary
            assert abs(float(got[t, e]) - exact) <= np.spacing(np.float32(abs(exact))) * 0.5000001 + 1e-30


def test_router_handles_width_not_multiple_of_64():
    rng = np.random.default_rng(1)
    h = rng.standard_normal((2, 100)).astype(np.float32)
    w = rng.standard_normal((5, 100)).astype(np.float32)
    np.testing.assert_allclose(moe.router_logits(h, w), h.astype(np.float64) @ w.T.astype(np.float64), rtol=1e-6)


def test_topk_ties_go_to_lower_index():
    logits = np.array([[0.5, 2.0, 2.0, 1.0, 2.0]], dtype=np.float32)
    idx, sel = moe.topk(logits, 3)
    assert idx.tolist() == [[1, 2, 4]]
    idx1, _ = moe.topk(logits, 1)
    assert idx1[0, 0] == int(np.argmax(logits[0]))      # np.argmax rule, engine/zaya.py:296


def test_gates_are_a_distribution_over_selected():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((50, 16)).astype(np.float32)
    idx, sel = moe.topk(logits, 2)
    g = moe.gates(sel)
    np.testing.assert_allclose(g.sum(axis=1), 1.0, rtol=1e-12)
    full = np.exp(logits - logits.max(axis=1, keepdims=True))
    full /= full.sum(axis=1, keepdims=True)
    picked = np.take_along_axis(full, idx, axis=1)
    np.testing.assert_allclose(g, picked / picked.sum(axis=1, keepdims=True), rtol=1e-6)


def test_permutation_is_stable_expert_major():
    rng = np.random.default_rng(3)
    idx = rng.integers(0, 7, size=(40, 3))
    counts, offsets, perm = moe.permutation(idx, 7)
    flat = idx.reshape(-1)
    assert counts.sum() == flat.size and sorted(perm.tolist()) == list(range(flat.size))
    assert np.all(np.diff(flat[perm]) >= 0)
    for e in range(7):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(flat[seg] == e) and np.all(np.diff(seg) > 0)


def test_one_expert_layer_is_the_dense_swiglu():
    from localai_amd import synth
    rng = np.random.default_rng(4)
    H, I = 256, 256
    gu = synth.quant_tensor(rng, 14, 2 * I, H, batch=1)
    dn = synth.quant_tensor(rng, 14, H, I, batch=1)
    h = rng.standard_normal((2, H)).astype(np.float32)
    rw = rng.standard_normal((1, H)).astype(np.float32)
    out, idx, g, _ = moe.moe_forward(h, rw, gu, dn, 14, 1, 1, I)
    assert np.all(idx == 0) and np.allclose(g, 1.0)
    wgu = quant.dequantize(gu, 14, (2 * I, H)).astype(np.float64)
    wd = quant.dequantize(dn, 14, (H, I)).astype(np.float64)
    for t in range(2):
        v = wgu @ h[t]
        a = v[:I] / (1 + np.exp(-np.clip(v[:I], -80, 80))) * v[I:]
        np.testing.assert_allclose(out[t], wd @ a, rtol=1e-12, atol=1e-12)


def test_expert_slices_follow_zaya_byte_offsets():
    from localai_amd import synth
    rng = np.random.default_rng(5)
    raw = synth.quant_tensor(rng, 12, 64, 256, batch=3)
    per = len(raw) // 3
    for e in range(3):
        np.testing.assert_array_equal(moe.expert_matrix(raw, 12, e, 64, 256),
                                      quant.dequantize(raw[e * per:(e + 1) * per], 12, (64, 256)))


def _dense_swiglu(gu_raw, dn_raw, t, H, I, x):
    """One expert's FFN from pieces pinned elsewhere: quant.matvec_exact (pinned
    against the reference library) and SiLU as x * expit(x) (SciPy's logistic
    function, engine/zaya.py:305 without the clip, which changes nothing
    below |x| = 80)."""
    from scipy.special import expit
    v = quant.matvec_exact(gu_raw, t, 2 * I, H, x)
    a = v[:I] * expit(v[:I]) * v[I:]
    return quant.matvec_exact(dn_raw, t, H, I, a)


def test_identical_experts_give_the_dense_ffn_for_any_k():
    """All experts byte-identical: the gates sum to one, so for every k the
    layer is the dense SwiGLU FFN whatever the gates are. A dropped gate
    factor (k x dense) or one applied twice (sum g^2 x dense) fails."""
    from localai_amd import synth
    rng = np.random.default_rng(6)
    H, I, E = 256, 512, 6
    gu1 = synth.quant_tensor(rng, 12, 2 * I, H)
    dn1 = synth.quant_tensor(rng, 12, H, I)
    h = rng.standard_normal((4, H)).astype(np.float32)
    rw = rng.standard_normal((E, H)).astype(np.float32) * 0.1
    dense = np.stack([_dense_swiglu(gu1, dn1, 12, H, I, h[t]) for t in range(4)])
    for k in (1, 2, 3, 6):
        out, idx, g, _ = moe.moe_forward(h, rw, gu1 * E, dn1 * E, 12, E, k, I)
        if k > 1:
            assert g.min() < 0.9 / k < 1.1 / k < g.max()      # gates far from uniform
        np.testing.assert_allclose(out, dense, rtol=1e-10, atol=1e-12 * np.abs(dense).max())


def test_doubling_one_experts_down_weights_doubles_only_its_gated_term():
    """Q6_K weights are linear in d (w = d * sc * q), so adding one to the
    exponent of every d of expert e's down slice doubles that expert's
    output exactly. The layer output must then grow by gate[t, slot(e)] * y_e
    for the tokens routed to e (y_e from a one-expert layer on e's bytes,
    whose gate is 1), and stay the same for every other token."""
    from localai_amd import synth
    rng = np.random.default_rng(7)
    H, I, E, k, T = 256, 256, 5, 2, 12
    gu = synth.quant_tensor(rng, 14, 2 * I, H, batch=E)
    dn = synth.quant_tensor(rng, 14, H, I, batch=E)
    h = rng.standard_normal((T, H)).astype(np.float32)
    rw = rng.standard_normal((E, H)).astype(np.float32) * 0.2
    out, idx, g, _ = moe.moe_forward(h, rw, gu, dn, 14, E, k, I)
    e = int(np.bincount(idx.reshape(-1), minlength=E).argmax())
    per_gu, per_dn = moe.expert_bytes(14, 2 * I, H), moe.expert_bytes(14, H, I)
    blocks = np.frombuffer(dn, np.uint8).reshape(-1, 210).copy()
    nb = per_dn // 210
    d = blocks[e * nb:(e + 1) * nb, 208:210].copy().view(np.uint16)
    assert np.all(((d >> 10) & 31) > 0) and np.all(((d >> 10) & 31) < 30)   # normal, room to double
    blocks[e * nb:(e + 1) * nb, 208:210] = (d + np.uint16(0x400)).view(np.uint8)
    out2, idx2, g2, _ = moe.moe_forward(h, rw, gu, blocks.tobytes(), 14, E, k, I)
    np.testing.assert_array_equal(idx2, idx)
    y_e, _, g1, _ = moe.moe_forward(h, np.zeros((1, H), np.float32), gu[e * per_gu:(e + 1) * per_gu],
                                    dn[e * per_dn:(e + 1) * per_dn], 14, 1, 1, I)
    assert np.all(g1 == 1.0)
    routed = 0
    for t in range(T):
        slots = np.nonzero(idx[t] == e)[0]
        want = g[t, slots[0]] * y_e[t] if slots.size else np.zeros(H)
        routed += slots.size
        np.testing.assert_allclose(out2[t] - out[t], want, rtol=1e-9, atol=1e-12 * np.abs(out).max())
    assert 0 < routed < T


def test_silu_matches_the_logistic_function_and_its_limits():
    """engine/zaya.py:305: g / (1 + exp(-clip(g, -80, 80))) against g * expit(g)
    and its limits: silu(0) = 0, silu(g) -> g for large g, -> 0 for very
    negative g, silu(-g) = silu(g) - g."""
    from scipy.special import expit
    g = np.concatenate([np.linspace(-90, 90, 3601), [-1e4, -80.5, 80.5, 1e4, 0.0]])
    s = moe.silu(g)
    np.testing.assert_allclose(s, g * expit(g), rtol=1e-13, atol=1e-30)
    assert moe.silu(np.array([0.0]))[0] == 0.0
    np.testing.assert_allclose(moe.silu(np.array([40.0, 1e4])), [40.0, 1e4], rtol=1e-15)
    assert abs(moe.silu(np.array([-1e4]))[0]) < 1e-30
    np.testing.assert_allclose(moe.silu(-g[:3601]), moe.silu(g[:3601]) - g[:3601], rtol=1e-12, atol=1e-12)
