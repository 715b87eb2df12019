"""CPU restatement of ZAYA's MoE block (engine/zaya.py:274-307). TEST
INFRASTRUCTURE ONLY.

    router = W_inp h (+ bias)                            zaya.py:281, model.py:72-79
    router = router + prev_router * eda   (when both)    zaya.py:282-286
    state  = router.copy()                               zaya.py:287
    router = norm(router, w_norm, eps)                   zaya.py:288, model.py:82
    router = gelu(W_gate router (+ bias))                zaya.py:289
    router = gelu(W_mlp2 router (+ bias))                zaya.py:290
    logits = W_mlp4 router (+ bias)                      zaya.py:291
    probs  = softmax(logits)                             zaya.py:292
    expert = argmax(probs + route_bias)                  zaya.py:296-297
    skip (expert == E): moe = h * probs[E]               zaya.py:297-301
    else: gate, up = split(W_gate_up[e] h); silu = gate / (1 + exp(-clip(gate)));
          moe = (W_down[e] (silu * up)) * probs[e]       zaya.py:303-306

The matrix products are exact (fp64 over exactly decoded weights, rounded to
fp32 once: the reference's own products go through its GGUF matvec, whose
summation order is not fixed); every elementwise step is the reference's
fp32 NumPy expression, and GELU is its math.erf loop (zaya.py:180-186).
Pinned by: the GELU known values of the reference's test
(tests/test_zaya.py:117-122) and the closed forms checked in
tests/test_oracle_zaya.py (RMSNorm, softmax, skip route, EDA); the choice of
expert is compared with the GPU only where the best two routes are apart
by more than a few fp32 ulps (np.exp's rounding is not restated: parity
unpinned there).
"""
from __future__ import annotations

import math

import numpy as np


def gelu(x):
    """engine/zaya.py:180-186: exact GELU through math.erf, one value at a time."""
    flat = np.asarray(x, dtype=np.float32).reshape(-1)
    return np.fromiter((v * (1.0 + math.erf(float(v) / math.sqrt(2.0))) * 0.5 for v in flat),
                       dtype=np.float32, count=flat.size).reshape(np.shape(x))


def rmsnorm(x, w, eps):
    """engine/model.py:82."""
    return x * (1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)) * w


def mat(w, x, bias=None):
    """W @ x exactly (fp64), rounded to fp32, plus the GGUF bias in fp32 (model.py:72-79)."""
    y = (np.asarray(w, np.float64) @ np.asarray(x, np.float64)).astype(np.float32)
    return y + bias if bias is not None else y


def moe_block(t, n_experts, eps, h, prev_router):
    """t: dict of fp32 numpy tensors (decoded) with the short names inp, inp_b,
    eda, norm, gate, gate_b, mlp2, mlp2_b, mlp4, mlp4_b, route_bias, gate_up
    [E, 2I, H], down [E, H, I] (biases and eda may be None).
    Returns (moe, state, probs, expert, margin): margin = gap between the best
    and the second-best route value."""
    h = np.asarray(h, np.float32)
    router = mat(t['inp'], h, t.get('inp_b'))
    if t.get('eda') is not None and prev_router is not None:
        router = router + np.asarray(prev_router, np.float32) * t['eda']
    state = router.copy()
    router = rmsnorm(router, t['norm'], eps)
    router = gelu(mat(t['gate'], router, t.get('gate_b')))
    router = gelu(mat(t['mlp2'], router, t.get('mlp2_b')))
    logits = mat(t['mlp4'], router, t.get('mlp4_b'))
    logits = logits - logits.max()
    probs = np.exp(logits)
    probs = probs / probs.sum()
    route = probs + t['route_bias']
    expert = int(np.argmax(route))
    order = np.sort(route)
    margin = float(order[-1] - order[-2]) if route.size > 1 else math.inf
    if expert == n_experts:
        moe = h.copy() * probs[expert]
    else:
        packed = mat(t['gate_up'][expert], h)
        gate, up = np.split(packed, 2)
        silu = gate / (1.0 + np.exp(-np.clip(gate, -80, 80)))
        moe = mat(t['down'][expert], silu * up) * probs[expert]
    return moe, state, probs, expert, margin
