"""Oracle of the decode-step attention mixers. TEST INFRASTRUCTURE ONLY.

gqa_decode restates in fp64 the decode step's attention of
engine/model.py:222-227 (cache write, window, np.repeat head grouping, scaled
scores, max-shifted softmax, weighted values) with the output gate of
engine/qwen35.py:158-182 (sigmoid as engine/qwen35.py:17-19).

delta_net_step restates engine/numba_kernels.py:11-45 in float32 in the
reference loop's operation order: the state scaled by exp(decay) (by
default the fp64 exponential rounded once to float32, which is what the GPU
kernel computes; NumPy's float32 exponential, the reference's own, on
request), pred accumulated over ki ascending with
each product and each sum rounded on its own, delta = (v - pred) * beta, then
the rank-one update and core in the same order. NumPy's float32 elementwise
operations round exactly as the scalar loop does, so the loop over ki is
vectorised over heads and value columns. delta_net_step_f64 restates the
reference's NumPy fallback (engine/qwen35.py:248-252) in fp64.

Pins (tests/test_oracle_attention.py): the float32 step against the fp64
fallback (two reference paths), the closed forms of beta = 0 (pure decay), a
one-hot key with beta = 1 (row replaced by v), and v = S^T k (delta = 0);
attention by a single position (out = v), equal keys (out = mean of V), a
two-position logistic closed form (pins the 1/sqrt(head_dim) scale), the
head-to-kv-head map h // G, the window, and the gate's closed forms.
"""
from __future__ import annotations

import math

import numpy as np


def sigmoid(x):
    """engine/qwen35.py:17-19 in fp64: 1 / (1 + exp(-clip(x, -80, 80)))."""
    x = np.asarray(x, dtype=np.float64)
    return 1.0 / (1.0 + np.exp(-np.clip(x, -80.0, 80.0)))


def gqa_decode(q, k_cache, v_cache, position, n_heads, n_kv_heads, head_dim, window=0, gate=None,
               k_new=None, v_new=None):
    """Returns (out [n_heads * head_dim] fp64, k_cache', v_cache') with the
    token's k_new / v_new written at `position` (engine/model.py:222).
    Caches: [max_seq, n_kv_heads, head_dim]."""
    kc = np.array(k_cache, dtype=np.float32, copy=True)
    vc = np.array(v_cache, dtype=np.float32, copy=True)
    if k_new is not None:
        kc[position] = np.asarray(k_new, np.float32).reshape(n_kv_heads, head_dim)
        vc[position] = np.asarray(v_new, np.float32).reshape(n_kv_heads, head_dim)
    start = max(0, position + 1 - window) if window > 0 else 0            # :223
    ks = kc[start:position + 1].astype(np.float64)
    vs = vc[start:position + 1].astype(np.float64)
    groups = n_heads // n_kv_heads
    kh = np.repeat(ks, groups, axis=1).transpose(1, 0, 2)                 # :225
    vh = np.repeat(vs, groups, axis=1).transpose(1, 0, 2)
    qh = np.asarray(q, np.float64).reshape(n_heads, head_dim)
    scores = np.einsum('hd,hld->hl', qh, kh) / math.sqrt(head_dim)        # :226
    scores -= scores.max(axis=-1, keepdims=True)
    probs = np.exp(scores)
    probs /= probs.sum(axis=-1, keepdims=True)
    out = np.einsum('hl,hld->hd', probs, vh).reshape(-1)                 # :227
    if gate is not None:
        out = out * sigmoid(np.asarray(gate, np.float64).reshape(-1))     # engine/qwen35.py:181
    return out, kc, vc


def gqa_decode_f32(q, k_cache, v_cache, position, n_heads, n_kv_heads, head_dim, window=0):
    """The reference's own float32 NumPy form of the same attention
    (engine/model.py:223-227, np.repeat + einsum), reading the caches in
    place (the token's row already written): the CPU baseline's workload."""
    start = max(0, position + 1 - window) if window > 0 else 0
    ks, vs = k_cache[start:position + 1], v_cache[start:position + 1]
    groups = n_heads // n_kv_heads
    kh = np.repeat(ks, groups, axis=1).transpose(1, 0, 2)
    vh = np.repeat(vs, groups, axis=1).transpose(1, 0, 2)
    scores = np.einsum('hd,hld->hl', np.asarray(q, np.float32).reshape(n_heads, head_dim), kh,
                       optimize=True) / math.sqrt(head_dim)
    scores -= scores.max(axis=-1, keepdims=True)
    probs = np.exp(scores)
    probs /= probs.sum(axis=-1, keepdims=True)
    return np.einsum('hl,hld->hd', probs, vh, optimize=True).reshape(-1)


def delta_net_step(state, q, k, v, decay, beta, factor_exp='rounded'):
    """engine/numba_kernels.py:11-45 in float32, the loop's rounding order.
    Returns (state', core) without changing `state`.

    factor_exp: 'rounded' takes exp(decay) as the fp64 exponential rounded
    once to float32 (what the GPU kernel computes); 'numpy_f32' takes NumPy's
    float32 exponential of the float32 decay, as the reference evaluates
    np.exp on float32 values (engine/numba_kernels.py:25,
    engine/qwen35.py:242). The two factors can differ in the last bit."""
    S = np.array(state, dtype=np.float32, copy=True)
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    beta = np.asarray(beta, np.float32)
    heads, kd, vd = S.shape
    if factor_exp == 'numpy_f32':
        factor = np.exp(np.asarray(decay, np.float32))                      # :25
    else:
        factor = np.exp(np.asarray(decay, np.float64)).astype(np.float32)
    pred = np.zeros((heads, vd), np.float32)
    for ki in range(kd):                                                   # :29-34
        S[:, ki, :] = S[:, ki, :] * factor[:, None]
        pred = pred + S[:, ki, :] * k[:, ki, None]
    delta = (v - pred) * beta[:, None]                                     # :36
    core = np.zeros((heads, vd), np.float32)
    for ki in range(kd):                                                   # :38-44
        S[:, ki, :] = S[:, ki, :] + k[:, ki, None] * delta
        core = core + S[:, ki, :] * q[:, ki, None]
    return S, core


def delta_net_step_f64(state, q, k, v, decay, beta):
    """The reference's NumPy fallback (engine/qwen35.py:248-252) in fp64."""
    S = np.array(state, dtype=np.float64, copy=True)
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    S *= np.exp(np.asarray(decay, np.float64))[:, None, None]
    pred = np.einsum('hkv,hk->hv', S, k)
    delta = (v - pred) * np.asarray(beta, np.float64)[:, None]
    S += k[:, :, None] * delta[:, None, :]
    core = np.einsum('hkv,hk->hv', S, q)
    return S, core
