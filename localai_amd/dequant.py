"""GPU drop-in for engine/dequant.py.

    LAYOUT, block_layout(t)       engine/dequant.py:6-17 (host-side table, same errors)
    dequantize(raw, t, shape)     engine/dequant.py:27-167 -> float32 numpy array

dequantize() runs the decode on the GPU (liblocalai_hip.so) and is
bit-identical to the reference decoders for every type. dequantize_device()
keeps the result on the device as a torch tensor.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, device

LAYOUT = {
    0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
    8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210),
}


def block_layout(t):
    if t not in LAYOUT:
        raise NotImplementedError(
            f'unsupported tensor type {t}; supported: F32(0), F16(1), Q4_0(2), Q4_1(3), Q5_0(6), '
            f'Q5_1(7), Q8_0(8), Q4_K(12), Q5_K(13), Q6_K(14)')
    return LAYOUT[t]


def dequantize_device(raw, t, shape, stream=None):
    """Decode GGML bytes (host bytes-like or uint8 device tensor) to a float32 device tensor."""
    tt = device.torch()
    block, bpb = block_layout(t)
    n = int(np.prod(shape, dtype=np.int64))
    if n % block:
        raise ValueError(f'{n} elements is not divisible by block size {block}')
    need = (n // block) * bpb
    if isinstance(raw, tt.Tensor):
        src = raw if raw.is_cuda else raw.to(device.device())
        if src.numel() < need:
            raise ValueError('raw tensor is smaller than the requested shape')
    else:
        view = np.frombuffer(raw, dtype=np.uint8)
        if view.size < need:
            raise ValueError('raw buffer is smaller than the requested shape')
        src = device.bytes_to_device(view[:need])
    out = tt.empty(tuple(int(s) for s in shape), dtype=tt.float32, device=device.device())
    _lib.check(_lib.load().localai_hip_dequant(int(t), device.ptr(src), n, device.ptr(out),
                                               ctypes.c_void_p(device.stream_ptr(stream))))
    return out


def dequantize(raw, t, shape):
    """Decode packed GGML blocks to a float32 NumPy tensor (computed on the GPU)."""
    return dequantize_device(raw, t, shape).cpu().numpy()
