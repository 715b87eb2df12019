"""Device buffers and weight handles on top of PyTorch-ROCm.

torch only owns device memory and streams here; all arithmetic runs in the
HIP kernels of liblocalai_hip.so.
"""
from __future__ import annotations

import atexit
import ctypes
import os

import numpy as np

from . import _lib

_TORCH = None
_EXITING = [False]
# Device frees are skipped once the interpreter is shutting down: the HIP
# runtime may already be torn down, and the process exit releases the memory.
atexit.register(lambda: _EXITING.__setitem__(0, True))


def torch():
    global _TORCH
    if _TORCH is None:
        import torch as t
        _TORCH = t
    return _TORCH


def gpu_available() -> bool:
    t = torch()
    return bool(t.cuda.is_available())


def device():
    t = torch()
    if not t.cuda.is_available():
        raise RuntimeError('no HIP device visible to PyTorch')
    return t.device('cuda', int(os.environ.get('LOCALAI_HIP_DEVICE', '0')))


def stream_ptr(stream=None) -> int:
    t = torch()
    s = stream if stream is not None else t.cuda.current_stream()
    return int(s.cuda_stream)


def ptr(tensor) -> int:
    return int(tensor.data_ptr())


def host_address(raw) -> tuple[int, int]:
    """(address, nbytes) of a bytes-like object."""
    view = np.frombuffer(raw, dtype=np.uint8)
    return int(view.ctypes.data), int(view.size)


def to_device_f32(x, shape=None):
    """numpy/array-like -> contiguous fp32 device tensor (16-byte aligned)."""
    t = torch()
    arr = np.ascontiguousarray(x, dtype=np.float32)
    if shape is not None:
        arr = arr.reshape(shape)
    return t.from_numpy(arr).to(device())


def bytes_to_device(raw):
    t = torch()
    view = np.frombuffer(raw, dtype=np.uint8)
    return t.from_numpy(view.copy()).to(device())


class QMat:
    """A device-resident (repacked) GGML weight tensor [batch, rows, cols]."""

    def __init__(self, handle, ggml_type, rows, cols, batch):
        self.handle = handle
        self.ggml_type = int(ggml_type)
        self.rows, self.cols, self.batch = int(rows), int(cols), int(batch)

    @classmethod
    def from_ggml(cls, raw, ggml_type, rows, cols, batch=1, stream=None):
        """raw: host bytes-like or a uint8 device tensor of GGML bytes."""
        lib = _lib.load()
        h = ctypes.c_void_p()
        t = torch()
        from .dequant import block_layout
        block, bpb = block_layout(int(ggml_type))
        if int(cols) % block:
            raise ValueError(f'cols {cols} is not a multiple of the block size {block}')
        need = int(batch) * int(rows) * (int(cols) // block) * bpb
        if isinstance(raw, t.Tensor):
            if not raw.is_cuda:
                raw = raw.to(device())
            if raw.numel() * raw.element_size() < need:
                raise ValueError('GGML tensor is smaller than batch*rows*cols requires')
            src, on_dev = ptr(raw), 1
        else:
            src, size = host_address(raw)
            if size < need:
                raise ValueError('GGML buffer is smaller than batch*rows*cols requires')
            on_dev = 0
        _lib.check(lib.localai_hip_qmat_create(int(ggml_type), int(rows), int(cols), int(batch),
                                               ctypes.c_void_p(src), on_dev,
                                               ctypes.c_void_p(stream_ptr(stream)), ctypes.byref(h)))
        return cls(h, ggml_type, rows, cols, batch)

    @property
    def device_bytes(self) -> int:
        return int(_lib.load().localai_hip_qmat_device_bytes(self.handle))

    def matvec(self, x, expert=0, out=None, stream=None):
        """x: [cols] or [ntok, cols] fp32 device tensor -> [rows] / [ntok, rows]."""
        t = torch()
        squeeze = x.dim() == 1
        x2 = x.reshape(1, -1) if squeeze else x
        if x2.dtype != t.float32 or not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.to(t.float32).contiguous().clone()
        if x2.shape[1] != self.cols:
            raise ValueError(f'x has {x2.shape[1]} columns, matrix has {self.cols}')
        ntok = x2.shape[0]
        if out is None:
            out = t.empty((ntok, self.rows), dtype=t.float32, device=x2.device)
        _lib.check(_lib.load().localai_hip_matvec(self.handle, int(expert), ptr(x2), ptr(out), int(ntok),
                                                  ctypes.c_void_p(stream_ptr(stream))))
        return out.reshape(-1) if squeeze else out

    def matmul(self, x, expert=0, out=None, rows_major=False, stream=None):
        """Prefill product on MFMA: x [tokens, cols] fp32 device tensor ->
        [tokens, rows] (or [rows, tokens] with rows_major=True, the layout of
        the reference's localai_*_matmul)."""
        t = torch()
        x2 = x
        if x2.dtype != t.float32 or not x2.is_contiguous():
            x2 = x2.to(t.float32).contiguous()
        if x2.dim() != 2 or x2.shape[1] != self.cols:
            raise ValueError(f'x must be [tokens, {self.cols}]')
        ntok = x2.shape[0]
        lib = _lib.load()
        ws_bytes = int(lib.localai_hip_matmul_workspace_size(self.handle, int(ntok)))
        ws = t.empty(max(ws_bytes, 1), dtype=t.uint8, device=x2.device)
        shape = (self.rows, ntok) if rows_major else (ntok, self.rows)
        if out is None:
            out = t.empty(shape, dtype=t.float32, device=x2.device)
        elif tuple(out.shape) != shape or not out.is_contiguous():
            raise ValueError(f'out must be a contiguous {shape} tensor')
        _lib.check(lib.localai_hip_matmul(self.handle, int(expert), ptr(x2), int(ntok), ptr(out),
                                          1 if rows_major else 0, ptr(ws), ws_bytes,
                                          ctypes.c_void_p(stream_ptr(stream))))
        return out

    def dequant(self, expert=0, stream=None):
        t = torch()
        out = t.empty((self.rows, self.cols), dtype=t.float32, device=device())
        _lib.check(_lib.load().localai_hip_qmat_dequant(self.handle, int(expert), ptr(out),
                                                        ctypes.c_void_p(stream_ptr(stream))))
        return out

    def unpack(self, stream=None):
        """GGML bytes of the whole tensor, reconstructed on the device (uint8 tensor)."""
        t = torch()
        from .dequant import block_layout
        block, bpb = block_layout(self.ggml_type)
        n = self.batch * self.rows * (self.cols // block) * bpb
        out = t.empty(n, dtype=t.uint8, device=device())
        _lib.check(_lib.load().localai_hip_qmat_unpack(self.handle, ptr(out),
                                                       ctypes.c_void_p(stream_ptr(stream))))
        return out

    def close(self):
        if _EXITING[0]:
            return
        if self.handle is not None and self.handle.value:
            _lib.load().localai_hip_qmat_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def matvec_many(mats, x, outs=None, experts=None, stream=None):
    """y_j = W_j @ x for several matrices sharing x (same cols), as one launch
    for the Q4_K / Q6_K matrices: q/k/v or gate/up of a decode step.
    Returns the list of [rows_j] outputs."""
    t = torch()
    if not mats or len(mats) > 8:
        raise ValueError('matvec_many takes 1..8 matrices')
    x2 = x.reshape(-1)
    if x2.dtype != t.float32 or not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.to(t.float32).contiguous().clone()
    for m in mats:
        if m.cols != x2.shape[0]:
            raise ValueError(f'x has {x2.shape[0]} values, matrix has {m.cols} columns')
    if outs is None:
        outs = [t.empty(m.rows, dtype=t.float32, device=x2.device) for m in mats]
    n = len(mats)
    handles = (ctypes.c_void_p * n)(*[m.handle.value for m in mats])
    ex = (ctypes.c_int64 * n)(*([0] * n if experts is None else [int(e) for e in experts]))
    ys = (ctypes.c_void_p * n)(*[ptr(o) for o in outs])
    _lib.check(_lib.load().localai_hip_matvec_many(n, handles, ex, ptr(x2), ys,
                                                   ctypes.c_void_p(stream_ptr(stream))))
    return outs
