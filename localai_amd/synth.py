"""Seeded synthetic GGML tensors and activations for the benchmark workloads.

All generators take a numpy Generator so tests and the benchmark share
byte-identical inputs. Distributions:

  Q4_K : qs bytes U(0..255) (4-bit quants U(0..15)); 12 scale bytes U(0..255)
         (the 16 six-bit scales/mins U(0..63)); d, dmin = fp16(U(1e-4, 2e-3))
  Q6_K : ql/qh bytes U(0..255) (6-bit quants); int8 scales U(-128..127);
         d = fp16(U(1e-4, 2e-3))
  Q8_0 : int8 quants U(-127..127); d = fp16(U(1e-4, 1e-2))
  Q4_0 / Q5_K : like Q4_K (d = fp16(U(1e-4, 2e-3)))
"""
from __future__ import annotations

import numpy as np

_LAYOUT = {2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}


def _f16_bytes(vals):
    return np.asarray(vals, dtype=np.float16).view(np.uint8).reshape(-1, 2)


def quant_tensor(rng, ggml_type, rows, cols, batch=1, d_range=None):
    """GGML bytes of a [batch, rows, cols] tensor (as `bytes`)."""
    block, bpb = _LAYOUT[ggml_type]
    assert cols % block == 0
    nblk = batch * rows * (cols // block)
    buf = rng.integers(0, 256, size=(nblk, bpb), dtype=np.uint8)
    if ggml_type == 8:
        lo, hi = d_range or (1e-4, 1e-2)
        buf[:, 0:2] = _f16_bytes(rng.uniform(lo, hi, nblk))
        buf[:, 2:34] = rng.integers(-127, 128, size=(nblk, 32), dtype=np.int8).view(np.uint8)
    elif ggml_type in (12, 13):
        lo, hi = d_range or (1e-4, 2e-3)
        buf[:, 0:2] = _f16_bytes(rng.uniform(lo, hi, nblk))
        buf[:, 2:4] = _f16_bytes(rng.uniform(lo, hi, nblk))
    elif ggml_type == 14:
        lo, hi = d_range or (1e-4, 2e-3)
        buf[:, 208:210] = _f16_bytes(rng.uniform(lo, hi, nblk))
    elif ggml_type == 2:
        lo, hi = d_range or (1e-4, 2e-3)
        buf[:, 0:2] = _f16_bytes(rng.uniform(lo, hi, nblk))
    return buf.tobytes()


def activations(rng, *shape):
    return rng.standard_normal(shape, dtype=np.float64).astype(np.float32)


# Llama-3-8B decode layer at batch 1 with the Q4_K_M mix (attn_v and ffn_down in Q6_K).
LLAMA3_8B_LAYER = [
    # name, type, rows, cols, input
    ('attn_q', 12, 4096, 4096, 'h'),
    ('attn_k', 12, 1024, 4096, 'h'),
    ('attn_v', 14, 1024, 4096, 'h'),
    ('attn_output', 12, 4096, 4096, 'attn'),
    ('ffn_gate', 12, 14336, 4096, 'h2'),
    ('ffn_up', 12, 14336, 4096, 'h2'),
    ('ffn_down', 14, 4096, 14336, 'act'),
]


def layer_weight_bytes(layer=LLAMA3_8B_LAYER):
    total = 0
    for _, t, rows, cols, _ in layer:
        block, bpb = _LAYOUT[t]
        total += rows * (cols // block) * bpb
    return total


def layer_algorithmic_bytes(layer=LLAMA3_8B_LAYER):
    """Weights + fp32 input vector + fp32 output vector per matvec."""
    total = 0
    for _, t, rows, cols, _ in layer:
        block, bpb = _LAYOUT[t]
        total += rows * (cols // block) * bpb + 4 * cols + 4 * rows
    return total


def zipf_bias(n_experts, s=1.1):
    """Logit bias b_e = ln(p_e), p_e proportional to (e+1)^-s (normalised)."""
    p = (np.arange(1, n_experts + 1, dtype=np.float64)) ** (-s)
    p /= p.sum()
    return np.log(p).astype(np.float32)
