"""GGML block decoders and exact products. TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Every decoder below is a restatement of engine/dequant.py (and of the
per-row decoders engine/native_quant.cpp:543-618), written as one closed-form
index formula per element and evaluated for all blocks at once:

  value index e inside a block  ->  (byte offset, bit shift, scale index)

The arithmetic is done in float32 in the same association the reference uses,
so results are bit-identical to the reference on finite inputs: every product
is exact in fp32 (fp16 scale <= 11 significant bits, 6-bit scale, <= 7-bit
quant), and the affine types (Q4_1, Q5_1, Q4_K, Q5_K) round exactly once at
the final add/subtract.
"""
from __future__ import annotations

import numpy as np

# GGML type id -> (values per block, bytes per block); engine/dequant.py:8-11.
LAYOUT = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
    8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210),
}
TYPE_NAMES = {0: 'F32', 1: 'F16', 2: 'Q4_0', 3: 'Q4_1', 6: 'Q5_0', 7: 'Q5_1',
              8: 'Q8_0', 12: 'Q4_K', 13: 'Q5_K', 14: 'Q6_K'}


def block_layout(t):
    """engine/dequant.py:12-17: unknown types raise NotImplementedError."""
    if t not in LAYOUT:
        raise NotImplementedError(f'unsupported tensor type {t}')
    return LAYOUT[t]


def _blocks(raw, t):
    bpb = LAYOUT[t][1]
    buf = np.frombuffer(raw, dtype=np.uint8)
    if buf.size % bpb:
        raise ValueError('raw size is not a whole number of blocks')
    return buf.reshape(-1, bpb)


def _f16_at(blocks, off):
    """fp16 little-endian field at byte `off` of every block, widened exactly."""
    lo = blocks[:, off].astype(np.uint16)
    hi = blocks[:, off + 1].astype(np.uint16)
    return (lo | (hi << 8)).view(np.float16).astype(np.float32)


def kquant_scale_min(scales12):
    """6-bit (scale, min) pairs of the K-quant 12-byte table, per group g=0..7.

    engine/native_quant.cpp:117-124 (q4_scale/q4_min), engine/dequant.py:265-270.
    g<4 : sc = s[g] & 63,                 mn = s[g+4] & 63
    g>=4: sc = (s[g+4] & 15) | (s[g-4] >> 6) << 4,  mn = (s[g+4] >> 4) | (s[g] >> 6) << 4
    Returns two uint8 arrays [nblocks, 8].
    """
    s = scales12.astype(np.uint8)
    sc = np.empty((s.shape[0], 8), np.uint8)
    mn = np.empty((s.shape[0], 8), np.uint8)
    sc[:, :4] = s[:, 0:4] & 63
    mn[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, mn


def _dequant_blocks(blk, t):
    n = blk.shape[0]
    if t == 8:      # Q8_0: d f16 @0, int8 q[32] @2; w = q*d  (engine/dequant.py:75-78)
        d = _f16_at(blk, 0)
        q = blk[:, 2:34].view(np.int8).astype(np.float32)
        return q * d[:, None]
    if t == 2:      # Q4_0: d @0, qs[16] @2; e<16 low nibble of qs[e], else high nibble of qs[e-16]
        d = _f16_at(blk, 0)
        qs = blk[:, 2:18]
        e = np.arange(32)
        q = (qs[:, e % 16] >> (4 * (e // 16))) & 15
        return (q.astype(np.float32) - 8.0) * d[:, None]
    if t == 3:      # Q4_1: d @0, m @2, qs[16] @4; w = q*d + m
        d, m = _f16_at(blk, 0), _f16_at(blk, 2)
        qs = blk[:, 4:20]
        e = np.arange(32)
        q = (qs[:, e % 16] >> (4 * (e // 16))) & 15
        return q.astype(np.float32) * d[:, None] + m[:, None]
    if t in (6, 7):  # Q5_0 (d @0, qh[4] @2, qs @6) / Q5_1 (d @0, m @2, qh @4, qs @8)
        d = _f16_at(blk, 0)
        qh_off = 2 if t == 6 else 4
        qh = blk[:, qh_off:qh_off + 4]
        qs = blk[:, qh_off + 4:qh_off + 20]
        e = np.arange(32)
        low = (qs[:, e % 16] >> (4 * (e // 16))) & 15
        high = (qh[:, e // 8] >> (e % 8)) & 1
        q = (low | (high << 4)).astype(np.float32)
        if t == 6:
            return (q - 16.0) * d[:, None]
        m = _f16_at(blk, 2)
        return q * d[:, None] + m[:, None]
    if t in (12, 13):  # Q4_K / Q5_K
        d, dmin = _f16_at(blk, 0), _f16_at(blk, 2)
        sc, mn = kquant_scale_min(blk[:, 4:16])
        qs = blk[:, 16:144] if t == 12 else blk[:, 48:176]
        e = np.arange(256)
        g, j = e // 32, e % 32
        q = (qs[:, 32 * (g // 2) + j] >> (4 * (g & 1))) & 15
        if t == 13:
            qh = blk[:, 16:48]
            q = q | (((qh[:, j] >> g) & 1) << 4)
        scale = d[:, None] * sc.astype(np.float32)          # exact
        minimum = dmin[:, None] * mn.astype(np.float32)     # exact
        return q.astype(np.float32) * scale[:, g] - minimum[:, g]
    if t == 14:     # Q6_K: ql[128] @0, qh[64] @128, int8 sc[16] @192, d @208
        d = _f16_at(blk, 208)
        ql, qh = blk[:, 0:128], blk[:, 128:192]
        sc = blk[:, 192:208].view(np.int8).astype(np.float32)
        e = np.arange(256)
        h, c, j = e // 128, (e % 128) // 32, e % 32
        lo = (ql[:, 64 * h + 32 * (c & 1) + j] >> (4 * (c >= 2))) & 15
        hi = (qh[:, 32 * h + j] >> (2 * c)) & 3
        q = (lo | (hi << 4)).astype(np.float32) - 32.0
        return (d[:, None] * sc[:, 8 * h + 2 * c + j // 16]) * q
    raise NotImplementedError(f'unsupported tensor type {t}')


def dequantize(raw, t, shape):
    """Decode GGML bytes to float32 of `shape` (engine/dequant.py:27-167)."""
    block, bpb = block_layout(t)
    n = int(np.prod(shape, dtype=np.int64))
    if n % block:
        raise ValueError(f'{n} elements is not divisible by block size {block}')
    if t == 0:
        return np.frombuffer(raw, dtype='<f4', count=n).astype(np.float32).reshape(shape)
    if t == 1:
        return np.frombuffer(raw, dtype='<f2', count=n).astype(np.float32).reshape(shape)
    blk = _blocks(raw, t)[: n // block]
    return _dequant_blocks(blk, t).reshape(shape)


def row_bytes(t, cols):
    block, bpb = block_layout(t)
    if cols % block:
        raise ValueError('cols not a multiple of the block size')
    return (cols // block) * bpb


def matvec_exact(raw, t, rows, cols, x):
    """fp64 W @ x with W decoded exactly; engine/gguf_parser.py:273-278 semantics."""
    w = dequantize(raw, t, (rows, cols)).astype(np.float64)
    return w @ np.asarray(x, dtype=np.float64)


def matmul_exact(raw, t, rows, cols, xs):
    """fp64 X @ W^T, shape [tokens, rows] (engine/native_quant.py:130-156 convention)."""
    w = dequantize(raw, t, (rows, cols)).astype(np.float64)
    return np.asarray(xs, dtype=np.float64) @ w.T


def q8_activation_matvec(raw, t, rows, cols, x):
    """Model of the AVX2 Q4_K/Q5_K matvec (engine/native_quant.cpp:84-109, :183-278).

    The reference quantises x to int8 per 32 values (scale = max|x|/127,
    round-to-nearest, clamp +-127) for the scale term but keeps the exact fp32
    32-sums for the minimum term. Equivalently: W_exact @ x_q plus the minimum
    correction  sum_g dmin*mn_g * (sum(x_g) - sum(x_q,g)).
    Same model as the reference's own test helper tests/test_dequant.py:5-33.
    """
    assert t in (12, 13)
    x = np.asarray(x, dtype=np.float32)
    groups = cols // 32
    xg = x.reshape(groups, 32)
    mx = np.abs(xg).max(axis=1)
    scale = np.where(mx > 1e-20, mx / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(xg / scale[:, None]), -127, 127)
    xq = (q * scale[:, None]).astype(np.float64)
    w = dequantize(raw, t, (rows, cols)).astype(np.float64)
    out = w @ xq.reshape(-1)
    delta = xg.astype(np.float64).sum(axis=1) - xq.sum(axis=1)            # [groups]
    blk = _blocks(raw, t)
    dmin = _f16_at(blk, 2).astype(np.float64)
    _, mn = kquant_scale_min(blk[:, 4:16])
    minw = (dmin[:, None] * mn).reshape(rows, groups)                      # [rows, groups]
    return out - minw @ delta
