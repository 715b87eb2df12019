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
