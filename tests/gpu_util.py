"""Shared helpers for the GPU tests (random GGML tensors with finite scales)."""
import numpy as np

from oracle import quant

# byte offsets of the fp16 scale fields per GGML type
SCALE_FIELDS = {2: (0,), 3: (0, 2), 6: (0,), 7: (0, 2), 8: (0,), 12: (0, 2), 13: (0, 2), 14: (208,)}


def random_ggml(rng, t, n_values, scale_lo=1e-4, scale_hi=2e-2, scales=None):
    """GGML bytes for n_values of type t: random quants, finite fp16 scales."""
    block, bpb = quant.block_layout(t)
    assert n_values % block == 0
    if t == 0:
        return rng.standard_normal(n_values).astype(np.float32).tobytes()
    if t == 1:
        return rng.standard_normal(n_values).astype(np.float16).tobytes()
    nb = n_values // block
    buf = rng.integers(0, 256, size=(nb, bpb), dtype=np.uint8)
    for off in SCALE_FIELDS[t]:
        if scales is None:
            v = rng.uniform(scale_lo, scale_hi, nb) * rng.choice([-1.0, 1.0], nb)
        else:
            v = rng.choice(np.asarray(scales, dtype=np.float64), nb)
        buf[:, off:off + 2] = np.asarray(v, dtype=np.float16).view(np.uint8).reshape(nb, 2)
    return buf.tobytes()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
