"""GPU drop-in for engine/native_quant.py: same functions, signatures and errors.

    get_native()                                            engine/native_quant.py:66-99
    matvec(raw, x, rows, cols, ggml_type, threads=4)        engine/native_quant.py:102-126
    matmul(raw, vectors, rows, cols, ggml_type, threads=4)  engine/native_quant.py:130-156

Behaviour kept from the reference:
  * unsupported type, rows < 1 or cols not a positive multiple of the block
    size -> None (the caller falls back), engine/native_quant.py:104-111;
  * wrong raw / vector size -> ValueError, engine/native_quant.py:115-116, :141-147;
  * matvec returns float32 [rows]; matmul returns float32 [tokens, rows];
  * `threads` is accepted and ignored (the work runs on the GPU).

get_native() returns the loaded HIP library, or None when this process sees
no HIP device (the reference's "native kernel unavailable" contract). With a
device present and the library missing it raises instead of returning None.

Weights: `raw` is GGML bytes in host memory (a GGUF mmap slice in the
reference). Immutable buffers -- `bytes`, read-only memoryviews such as mmap
slices -- are uploaded once and kept as device handles, keyed by address,
size, type and shape. A cache entry references the object that owns the
memory (the bytes object, or the mmap behind a slice), so the address cannot
be reused while the entry lives, but holds no exported buffer: the owner's
mmap.close() (GGUFFile.close, engine/gguf_parser.py:77-80) still succeeds,
and entries whose mmap has closed are dropped. Writable buffers are uploaded
on every call. The cache is bounded by LOCALAI_HIP_WEIGHT_CACHE_GB (default
64).
"""
from __future__ import annotations

import os
from collections import OrderedDict

import numpy as np

from . import _lib, device

_NATIVE_TYPES = (2, 8, 12, 13, 14)
_BYTES_PER_BLOCK = {2: 18, 8: 34, 12: 144, 13: 176, 14: 210}

_cache: 'OrderedDict[tuple, tuple]' = OrderedDict()
_cache_bytes = [0]


def get_native():
    if not device.gpu_available():
        return None
    lib = _lib.load()
    return lib


def _block_size(t):
    return 32 if t in (2, 8) else 256


def _immutable(raw) -> bool:
    if isinstance(raw, bytes):
        return True
    try:
        return bool(memoryview(raw).readonly)
    except TypeError:
        return False


def _cache_limit() -> int:
    return int(float(os.environ.get('LOCALAI_HIP_WEIGHT_CACHE_GB', '64')) * (1 << 30))


def _owner(raw):
    """The object owning raw's memory, found without keeping a buffer export."""
    try:
        view = memoryview(raw)
    except TypeError:
        return raw
    owner = view.obj
    view.release()
    return owner


def _stale(owner) -> bool:
    return bool(getattr(owner, 'closed', False))


def _drop(key):
    q, _, nbytes = _cache.pop(key)
    _cache_bytes[0] -= nbytes   # as counted on insertion (a handle can grow later)
    q.close()


def weights(raw, rows, cols, ggml_type, batch=1):
    """Device handle for GGML bytes `raw` [batch, rows, cols] (cached when immutable)."""
    for key in [k for k, (_, o, _n) in _cache.items() if _stale(o)]:
        _drop(key)
    addr, nbytes = device.host_address(raw)
    key = (addr, nbytes, int(ggml_type), int(batch), int(rows), int(cols))
    hit = _cache.get(key)
    if hit is not None:
        _cache.move_to_end(key)
        return hit[0]
    q = device.QMat.from_ggml(raw, ggml_type, rows, cols, batch)
    if _immutable(raw):
        nbytes = q.device_bytes
        _cache[key] = (q, _owner(raw), nbytes)
        _cache_bytes[0] += nbytes
        while _cache_bytes[0] > _cache_limit() and len(_cache) > 1:
            _drop(next(iter(_cache)))
    return q


def clear_cache():
    while _cache:
        _, (q, _, _n) = _cache.popitem()
        q.close()
    _cache_bytes[0] = 0


def _validate(raw, rows, cols, ggml_type):
    if ggml_type not in _NATIVE_TYPES or rows < 1:
        return None
    block = _block_size(ggml_type)
    if cols < block or cols % block:
        return None
    return rows * (cols // block) * _BYTES_PER_BLOCK[ggml_type]


def matvec(raw, x, rows: int, cols: int, ggml_type: int, threads: int = 4):
    """W @ x for GGML bytes W [rows, cols]; float32 [rows], or None if unsupported."""
    expected = _validate(raw, rows, cols, ggml_type)
    if expected is None:
        return None
    if get_native() is None:
        return None
    raw_view = np.frombuffer(raw, dtype=np.uint8)
    if raw_view.size != expected or np.asarray(x).size != cols:
        raise ValueError('native quantized matvec received an invalid tensor or vector size')
    q = weights(raw, rows, cols, ggml_type)
    xd = device.to_device_f32(np.asarray(x).reshape(-1))
    y = q.matvec(xd)
    return y.cpu().numpy()


# Token count from which matmul() runs the MFMA GEMM instead of the fp32 matvec.
GEMM_TOKENS = 32


def matmul(raw, vectors, rows: int, cols: int, ggml_type: int, threads: int = 4):
    """X @ W^T for GGML bytes W [rows, cols]; float32 [tokens, rows], or None."""
    expected = _validate(raw, rows, cols, ggml_type)
    if expected is None:
        return None
    if get_native() is None:
        return None
    x = np.ascontiguousarray(vectors, dtype=np.float32)
    if x.ndim != 2 or x.shape[1] != cols or x.shape[0] < 1:
        raise ValueError('native quantized matmul received an invalid input matrix')
    raw_view = np.frombuffer(raw, dtype=np.uint8)
    if raw_view.size != expected:
        raise ValueError('native quantized matmul received an invalid tensor size')
    q = weights(raw, rows, cols, ggml_type)
    xd = device.to_device_f32(x)
    # many tokens: MFMA GEMM (f16 operands, fp32 accumulation); few: fp32 matvec
    y = q.matmul(xd) if x.shape[0] >= GEMM_TOKENS else q.matvec(xd)
    return y.cpu().numpy()
