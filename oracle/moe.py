"""Composition oracle for the top-k MoE expert layer. TEST INFRASTRUCTURE ONLY.

The reference has only a top-1 MoE (engine/zaya.py:274-307): router matvec,
softmax, argmax with the lowest index winning ties (np.argmax,
engine/zaya.py:296), then for the chosen expert
    packed = W_gate_up[e] @ h ; gate, up = split(packed, 2)      (zaya.py:303-304)
    silu   = gate / (1 + exp(-clip(gate, -80, 80)))               (zaya.py:305)
    out    = (W_down[e] @ (silu * up)) * p_e                      (zaya.py:306)
where W[e] is the byte slice [e*B, (e+1)*B) of the 3-D expert tensor
(zaya.py:139-175). This module generalises it to top-k with softmax gates
renormalised over the selected experts (softmax over the k selected logits),
and a gate-weighted sum over the k experts.

Routing is made bit-reproducible by a canonical router: each logit is a sum of
exact fp64 products h*w in a fixed order (64 lane sums over interleaved
4-element chunks, then a pairwise tree over the lanes), rounded once to fp32. The ranking key is
(logit descending, expert index ascending).

The reference has no top-k>1 MoE and no MoE test, so no reference output pins
this module; tests/test_oracle_moe.py pins it through checks that a dropped,
doubled or misplaced term fails: permutation round trip, histogram totals,
gates summing to one, forced ties, the router logit against math.fsum, the
one-expert layer and the all-experts-identical layer (any k) against a dense
FFN built from quant.matvec_exact and SciPy's expit, an exact doubling of
one expert's down weights that must move the output by exactly that
expert's gated term, and SiLU against x * expit(x) and its limits.
"""
from __future__ import annotations

import numpy as np

from .quant import block_layout, dequantize

LANES = 64


def router_logits(h, w):
    """Canonical fp32 router logits [T, E] for h [T, H] and w [E, H] (both fp32).

    Sum order: lane l (0..63) accumulates, for j = 0, 1, ..., the exact fp64
    products of elements 256 j + 4 l + c, c = 0, 1, 2, 3, in that order (one
    16-byte load per lane and step); the 64 lane sums are then added pairwise
    s[l] += s[l + off] for off = 32, 16, 8, 4, 2, 1; the result is rounded to
    fp32 once.
    """
    h = np.asarray(h, dtype=np.float32)
    w = np.asarray(w, dtype=np.float32)
    T, H = h.shape
    E = w.shape[0]
    pad = (-H) % (4 * LANES)
    hp = np.pad(h.astype(np.float64), ((0, 0), (0, pad)))
    wp = np.pad(w.astype(np.float64), ((0, 0), (0, pad)))
    steps = hp.shape[1] // (4 * LANES)
    out = np.empty((T, E), dtype=np.float32)
    for t0 in range(0, T, 16):                                   # bound the fp64 temporaries
        prod = hp[t0:t0 + 16, None, :] * wp[None, :, :]          # exact products
        prod = prod.reshape(prod.shape[0], E, steps, LANES, 4)
        acc = np.zeros((prod.shape[0], E, LANES), dtype=np.float64)
        for i in range(steps):                                   # sequential per lane
            for c in range(4):
                acc = acc + prod[:, :, i, :, c]
        off = LANES // 2
        while off:
            acc = acc[:, :, :off] + acc[:, :, off:2 * off]
            off //= 2
        out[t0:t0 + 16] = acc[:, :, 0].astype(np.float32)
    return out


def topk(logits, k):
    """Indices [T, k] ranked by (value desc, index asc) and their logits."""
    logits = np.asarray(logits, dtype=np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), dtype=np.int32)
    for t in range(T):
        order = np.lexsort((np.arange(E), -logits[t].astype(np.float64)))
        idx[t] = order[:k]
    return idx, np.take_along_axis(logits, idx, axis=1)


def gates(selected_logits):
    """Softmax over the k selected logits (= full softmax renormalised over top-k)."""
    s = np.asarray(selected_logits, dtype=np.float64)
    e = np.exp(s - s.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def silu(g):
    """engine/zaya.py:305 (clip to +-80 before exp)."""
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-np.clip(g, -80.0, 80.0)))


def expert_bytes(t, rows, cols):
    """Bytes of one expert's [rows, cols] slice (engine/zaya.py:144-148)."""
    block, bpb = block_layout(t)
    return (rows * cols // block) * bpb


def expert_matrix(raw, t, e, rows, cols):
    """fp64 decode of expert e's slice of a [E, rows, cols] tensor (zaya.py:149-150)."""
    b = expert_bytes(t, rows, cols)
    view = memoryview(raw)[e * b:(e + 1) * b]
    return dequantize(view, t, (rows, cols)).astype(np.float64)


def moe_forward(h, router_w, gu_raw, down_raw, t, n_experts, k, inter, router_bias=None):
    """Full MoE layer: returns (out [T,H] fp64, idx [T,k], gates [T,k] fp64, logits [T,E]).

    gu_raw: GGML bytes of [E, 2*inter, H] (rows 0..inter-1 gate, inter.. up).
    down_raw: GGML bytes of [E, H, inter].
    router_bias (optional, [E] fp32) is added to the fp32 logits before ranking
    and gating, as LlamaModel._mat_impl adds a stored bias (engine/model.py:74-79).
    """
    h = np.asarray(h, dtype=np.float32)
    T, H = h.shape
    logits = router_logits(h, router_w)
    if router_bias is not None:
        logits = (logits + np.asarray(router_bias, dtype=np.float32)[None, :]).astype(np.float32)
    idx, sel = topk(logits, k)
    g = gates(sel)
    cache = {}
    out = np.zeros((T, H), dtype=np.float64)
    for ti in range(T):
        for s in range(k):
            e = int(idx[ti, s])
            if e not in cache:
                cache[e] = (expert_matrix(gu_raw, t, e, 2 * inter, H),
                            expert_matrix(down_raw, t, e, H, inter))
            wgu, wd = cache[e]
            gu = wgu @ h[ti].astype(np.float64)
            act = silu(gu[:inter]) * gu[inter:]
            out[ti] += g[ti, s] * (wd @ act)
    return out, idx, g, logits


def permutation(idx, n_experts):
    """Expert-major order of the T*k assignments a = t*k + slot.

    Returns (counts [E], offsets [E+1], perm [T*k]) where perm lists the
    assignments sorted by (expert, a).
    """
    flat = np.asarray(idx, dtype=np.int64).reshape(-1)
    counts = np.bincount(flat, minlength=n_experts)
    offsets = np.concatenate([[0], np.cumsum(counts)])
    perm = np.lexsort((np.arange(flat.size), flat))
    return counts.astype(np.int32), offsets.astype(np.int32), perm.astype(np.int32)
