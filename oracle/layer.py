"""Oracle of the decode-layer matvec chain. TEST INFRASTRUCTURE ONLY.

Restates, in fp64 over exactly decoded weights, the part of the reference's
decode step between the attention output of layer L and the attention inputs
of layer L+1 (engine/model.py:215-240 of layer L, then :181-213 of L+1):

    x1  = pre + W_o att                                  (:229)
    u   = norm(x1, w_ffn)                                (:231, norm :82)
    act = silu(W_gate u) * (W_up u)                      (:232)
    x2  = x1 + W_down act                                (:233)
    v'  = norm(x2, w_attn)                               (:181 of L+1)
    q, k, v = W_q v', W_k v', W_v v'                     (:182-185)
    q, k = rope(q), rope(k)  (adjacent pairs, Llama)     (:203-210)

norm(x, w) = x / sqrt(mean(x^2) + eps) * w and silu(g) = g / (1 + exp(-clip(g,
-80, 80))) as the reference writes them; the matvecs are quant.matvec_exact.
Pins (tests/test_oracle_layer.py): the matvecs are pinned against the
reference library elsewhere; norm by unit RMS and scale invariance; RoPE
against complex multiplication by exp(i*angle); SiLU through oracle.moe.silu.
"""
from __future__ import annotations

import numpy as np

from .moe import silu
from .quant import matvec_exact

ORDER = ('attn_output', 'ffn_gate', 'ffn_up', 'ffn_down', 'attn_q', 'attn_k', 'attn_v')


def norm(x, w, eps):
    """engine/model.py:82: x * (1 / sqrt(mean(x * x) + eps)) * w, in fp64."""
    x = np.asarray(x, dtype=np.float64)
    return x * (1.0 / np.sqrt(np.mean(x * x) + eps)) * np.asarray(w, dtype=np.float64)


def rope_pairs(a, cos, sin, head_dim):
    """Adjacent-pair RoPE of engine/model.py:205-210 on a flat [heads * head_dim]
    vector: in each head, pair (2j, 2j + 1) for j < len(cos) is rotated by the
    angle whose cosine and sine are cos[j], sin[j]; later dimensions unchanged."""
    a = np.asarray(a, dtype=np.float64).reshape(-1, head_dim)
    out = a.copy()
    half = len(cos)
    even, odd = a[:, 0:2 * half:2], a[:, 1:2 * half:2]
    c, s = np.asarray(cos, np.float64)[None, :], np.asarray(sin, np.float64)[None, :]
    out[:, 0:2 * half:2] = even * c - odd * s
    out[:, 1:2 * half:2] = even * s + odd * c
    return out.reshape(-1)


def chain(mats, pre, att, w_ffn, w_attn, eps, rope=None, head_dim=None):
    """mats: name -> (raw GGML bytes, ggml type, rows, cols) for the names of
    ORDER. Returns (x_out, q, k, v) in fp64 and the intermediates (o, act, d)."""
    def mv(name, x):
        raw, t, rows, cols = mats[name]
        return matvec_exact(raw, t, rows, cols, x)
    o = mv('attn_output', att)
    x1 = np.asarray(pre, np.float64) + o
    u = norm(x1, w_ffn, eps)
    act = silu(mv('ffn_gate', u)) * mv('ffn_up', u)
    d = mv('ffn_down', act)
    x2 = x1 + d
    v_in = norm(x2, w_attn, eps)
    q, k, v = mv('attn_q', v_in), mv('attn_k', v_in), mv('attn_v', v_in)
    if rope is not None:
        cos, sin = rope
        q, k = rope_pairs(q, cos, sin, head_dim), rope_pairs(k, cos, sin, head_dim)
    return (x2, q, k, v), (o, act, d)
