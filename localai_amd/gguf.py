"""GPU drop-in for engine/gguf_parser.py: the GGUF v2/v3 reader, with every
matrix uploaded to the device once and kept there until close().

    GGUFFile(path)                          engine/gguf_parser.py:48-84
      .version .alignment .metadata .tensors .path ._map
      .tensor_bytes(info) .raw_tensor(name)   :141-149
      .tensor(name)                           :150-155 (decoded on the GPU)
      .tensor_row(name, row)                  :157-173 (decoded on the GPU)
      .matvec(name, x, row_chunk=1024)        :175-289
      .matmul(name, X, row_chunk=1024)        :291-367
      .find(*suffixes) .close() with-block    :368-378
    _native_thread_count(rows, type, batched)  :13-42 (thread policy; the GPU ignores it)
    TensorInfo                                 :44-46

Parsing, validation and error types follow the reference: the magic and
version (2 or 3), count limits, string and array bounds, one to eight
positive dimensions, unique names, offsets aligned to `general.alignment`
(32 unless 1..4096), tensor ranges inside the file and not overlapping;
tensors of an unknown type stay listed and fail on access. Shapes are the
GGUF dimensions reversed ([out, in] for a matrix).

Device residency replaces the reference's host caches (decoded fp16/fp32
copies, :55-74): matvec / matmul on a matrix upload its bytes on first use --
the packed types (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K) as a device weight handle
that the quantized kernels read directly, every other type decoded once by
the GPU dequant kernels to an fp32 device matrix -- and later calls reuse it.
device_matrix(name) hands that object to code that keeps its vectors on the
device. Uploads stop being cached past LOCALAI_HIP_WEIGHT_CACHE_GB (default
64) per file; close() frees them. The reference's Numba and chunked-decode
fallbacks are not needed: every type has a device path.
"""
from __future__ import annotations

import ctypes
import mmap
import os
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import _lib, device
from .dequant import block_layout

MAGIC = b'GGUF'
# GGUF metadata value types
(UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64,
 FLOAT64) = range(13)
_SCALAR = {UINT8: '<B', INT8: '<b', UINT16: '<H', INT16: '<h', UINT32: '<I', INT32: '<i',
           FLOAT32: '<f', BOOL: '<?', UINT64: '<Q', INT64: '<q', FLOAT64: '<d'}
_PACKED = (2, 8, 12, 13, 14)     # types with a device weight handle (the reference's native types)
_MAX_TENSORS, _MAX_KV, _MAX_ARRAY = 10_000_000, 1_000_000, 100_000_000


def _native_thread_count(rows, ggml_type, *, batched=False):
    """Worker count the reference's AVX2 pool would use (engine/gguf_parser.py:13-42).
    The GPU kernels ignore it; it is kept for callers that pass `threads`."""
    if not batched:
        env = os.environ.get('LOCALAI_NATIVE_DECODE_THREADS', '').strip()
        if env:
            try:
                want = int(env)
            except ValueError:
                want = 0
            if want > 0:
                return min(want, os.cpu_count() or 1)
    if rows >= 65536 and ggml_type != 8:
        want = 8
    elif not batched and ggml_type == 12 and rows >= 4096:
        want = 8
    elif not batched and ggml_type == 14 and rows >= 4096:
        want = 7
    elif ggml_type == 8 or ggml_type in (12, 13, 14):
        want = 6
    else:
        want = 4
    return min(want, os.cpu_count() or 1)


@dataclass
class TensorInfo:
    name: str
    shape: tuple
    ggml_type: int
    offset: int
    nbytes: int = 0


class DenseMatrix:
    """fp32 device matrix [batch, rows, cols] with the QMat product interface
    (localai_hip_f32_matvec): GGUF matrices outside the packed types."""

    def __init__(self, values, batch, rows, cols):
        self.values = values
        self.batch, self.rows, self.cols = int(batch), int(rows), int(cols)

    @property
    def device_bytes(self) -> int:
        return self.values.numel() * 4

    def matvec(self, x, expert=0, out=None, stream=None):
        t = device.torch()
        squeeze = x.dim() == 1
        x2 = x.reshape(1, -1) if squeeze else x
        if x2.dtype != t.float32 or not x2.is_contiguous():
            x2 = x2.to(t.float32).contiguous()
        if x2.shape[1] != self.cols:
            raise ValueError(f'x has {x2.shape[1]} columns, matrix has {self.cols}')
        if not 0 <= int(expert) < self.batch:
            raise IndexError(f'expert {expert} outside [0, {self.batch})')
        ntok = x2.shape[0]
        if out is None:
            out = t.empty((ntok, self.rows), dtype=t.float32, device=x2.device)
        w = self.values.reshape(self.batch, self.rows, self.cols)[int(expert)]
        _lib.check(_lib.load().localai_hip_f32_matvec(device.ptr(w), self.rows, self.cols, device.ptr(x2),
                                                      ntok, device.ptr(out),
                                                      ctypes.c_void_p(device.stream_ptr(stream))))
        return out.reshape(-1) if squeeze else out

    def matmul(self, x, expert=0, out=None, stream=None):
        return self.matvec(x, expert=expert, out=out, stream=stream)

    def close(self):
        self.values = None


class GgmlMatrix:
    """GGML bytes of a [batch, rows, cols] matrix kept on the device as they are
    in the file, with the QMat product interface (localai_hip_ggml_matvec:
    blocks decoded in registers): F16, Q4_1, Q5_0 and Q5_1 matrices, which the
    reference keeps as fp32 or fp16 caches (engine/gguf_parser.py:65-69)."""

    def __init__(self, raw, ggml_type, batch, rows, cols):
        t = device.torch()
        block, bpb = block_layout(ggml_type)
        self.ggml_type = int(ggml_type)
        self.batch, self.rows, self.cols = int(batch), int(rows), int(cols)
        self.matrix_bytes = self.rows * (self.cols // block) * bpb
        host = np.frombuffer(raw, dtype=np.uint8)
        if host.size != self.batch * self.matrix_bytes:
            raise ValueError('tensor bytes do not match [batch, rows, cols]')
        # each matrix starts 256-byte aligned (F16 rows need 16-byte alignment)
        self.stride = -(-self.matrix_bytes // 256) * 256
        self.bytes = t.empty(self.batch * self.stride, dtype=t.uint8, device=device.device())
        for e in range(self.batch):
            self.bytes[e * self.stride:e * self.stride + self.matrix_bytes].copy_(
                t.from_numpy(host[e * self.matrix_bytes:(e + 1) * self.matrix_bytes].copy()))

    @property
    def device_bytes(self) -> int:
        return self.bytes.numel()

    def matvec(self, x, expert=0, out=None, stream=None):
        t = device.torch()
        squeeze = x.dim() == 1
        x2 = x.reshape(1, -1) if squeeze else x
        if x2.dtype != t.float32 or not x2.is_contiguous() or x2.data_ptr() % 16:
            x2 = x2.to(t.float32).contiguous().clone()
        if x2.shape[1] != self.cols:
            raise ValueError(f'x has {x2.shape[1]} columns, matrix has {self.cols}')
        if not 0 <= int(expert) < self.batch:
            raise IndexError(f'expert {expert} outside [0, {self.batch})')
        ntok = x2.shape[0]
        if out is None:
            out = t.empty((ntok, self.rows), dtype=t.float32, device=x2.device)
        w = device.ptr(self.bytes) + int(expert) * self.stride
        _lib.check(_lib.load().localai_hip_ggml_matvec(self.ggml_type, w, self.rows, self.cols, device.ptr(x2),
                                                       ntok, device.ptr(out),
                                                       ctypes.c_void_p(device.stream_ptr(stream))))
        return out.reshape(-1) if squeeze else out

    def matmul(self, x, expert=0, out=None, stream=None):
        return self.matvec(x, expert=expert, out=out, stream=stream)

    def close(self):
        self.bytes = None


# kept on the device as GGML bytes (GgmlMatrix) when rows are whole 8-value groups
_RAW = (1, 3, 6, 7)


class GGUFFile:
    def __init__(self, path):
        self.path = Path(path)
        self._file = self.path.open('rb')
        self._map = None
        try:
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
            self.metadata, self.tensors, self.version, self.alignment = {}, {}, 0, 32
            self._dev, self._dev_bytes = {}, 0
            self._dev_limit = int(float(os.environ.get('LOCALAI_HIP_WEIGHT_CACHE_GB', '64')) * (1 << 30))
            self._parse()
        except Exception:
            if self._map is not None:
                self._map.close()
            self._file.close()
            raise

    # ---- parsing ----------------------------------------------------------

    def _take(self, fmt):
        n = struct.calcsize(fmt)
        if self._pos + n > len(self._map):
            raise ValueError(f'{self.path}: truncated GGUF at byte {self._pos}')
        v = struct.unpack_from(fmt, self._map, self._pos)[0]
        self._pos += n
        return v

    def _string(self):
        n = self._take('<Q')
        if n > len(self._map):
            raise ValueError('Invalid GGUF string length')
        if self._pos + n > len(self._map):
            raise ValueError('Truncated GGUF string')
        b = self._map[self._pos:self._pos + n]
        self._pos += n
        return b.decode('utf-8', errors='replace')

    def _value(self, typ):
        if typ == STRING:
            return self._string()
        if typ == ARRAY:
            et, n = self._take('<I'), self._take('<Q')
            if n > _MAX_ARRAY:
                raise ValueError('Unreasonable GGUF array length')
            return [self._value(et) for _ in range(n)]
        fmt = _SCALAR.get(typ)
        if fmt is None:
            raise ValueError(f'Unsupported GGUF metadata value type {typ}')
        return self._take(fmt)

    def _parse(self):
        self._pos = 0
        if bytes(self._map[0:4]) != MAGIC:
            raise ValueError(f'{self.path} is not a GGUF file')
        self._pos = 4
        self.version = self._take('<I')
        if self.version not in (2, 3):
            raise ValueError(f'GGUF version {self.version} unsupported; expected v2/v3')
        n_tensors, n_kv = self._take('<Q'), self._take('<Q')
        if n_tensors > _MAX_TENSORS or n_kv > _MAX_KV:
            raise ValueError('Invalid GGUF counts')
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._take('<I'))
        align = int(self.metadata.get('general.alignment', 32))
        self.alignment = align if 0 < align <= 4096 else 32
        infos, seen = [], set()
        for _ in range(n_tensors):
            name = self._string()
            nd = self._take('<I')
            if not 1 <= nd <= 8:
                raise ValueError(f'Tensor {name}: invalid dimension count {nd}')
            dims = tuple(self._take('<Q') for _ in range(nd))
            typ, off = self._take('<I'), self._take('<Q')
            if name in seen:
                raise ValueError(f'Duplicate tensor name in GGUF: {name!r}')
            if 0 in dims:
                raise ValueError(f'Tensor {name}: dimensions must be positive')
            if off % self.alignment:
                raise ValueError(f'Tensor {name}: data offset {off} is not aligned to {self.alignment} bytes')
            seen.add(name)
            infos.append(TensorInfo(name, tuple(reversed(dims)), typ, off))
        data_start = -(-self._pos // self.alignment) * self.alignment
        spans = []
        for info in infos:
            info.offset += data_start
            try:
                info.nbytes = self.tensor_bytes(info)
            except NotImplementedError:   # unknown type: listed, fails on access
                info.nbytes = 0
            else:
                end = info.offset + info.nbytes
                if end > len(self._map):
                    raise ValueError(f'Tensor {info.name} extends past end of GGUF '
                                     f'(end={end}, file_size={len(self._map)})')
                spans.append((info.offset, end, info.name))
            self.tensors[info.name] = info
        spans.sort()
        for (_, end0, a), (start1, _, b) in zip(spans, spans[1:]):
            if start1 < end0:
                raise ValueError(f'Tensor data ranges overlap: {a!r} and {b!r}')

    # ---- bytes and decoded values -----------------------------------------

    def tensor_bytes(self, info):
        block, bpb = block_layout(info.ggml_type)
        n = int(np.prod(info.shape, dtype=np.int64))
        if n % block:
            raise ValueError(f'Tensor {info.name} has {n} values, not divisible by block size {block}')
        return (n // block) * bpb

    def raw_tensor(self, name):
        info = self.tensors[name]
        end = info.offset + self.tensor_bytes(info)
        if end > len(self._map):
            raise ValueError(f'Tensor {name} extends past end of GGUF')
        return memoryview(self._map)[info.offset:end]

    def tensor(self, name):
        from .dequant import dequantize
        info = self.tensors[name]
        try:
            return dequantize(self.raw_tensor(name), info.ggml_type, info.shape)
        except Exception as e:
            raise type(e)(f'tensor "{name}" (GGML type {info.ggml_type}): {e}') from e

    def tensor_row(self, name, row):
        """One row of a 2-D tensor, decoded on the GPU from that row's bytes only."""
        from .dequant import dequantize
        info = self.tensors[name]
        if len(info.shape) != 2:
            raise ValueError(f'{name}: tensor_row requires a 2-D tensor, got {info.shape}')
        rows, cols = info.shape
        if not 0 <= int(row) < rows:
            raise IndexError(f'{name}: row {row} outside [0, {rows})')
        block, bpb = block_layout(info.ggml_type)
        if cols % block:
            raise ValueError(f'{name}: row length {cols} is not divisible by quantization block {block}')
        row_bytes = (cols // block) * bpb
        start = info.offset + int(row) * row_bytes
        return dequantize(memoryview(self._map)[start:start + row_bytes], info.ggml_type, (cols,))

    # ---- device residency ---------------------------------------------------

    def device_matrix(self, name):
        """The device copy of matrix `name` ([out, in], or [experts, out, in]):
        a QMat for the packed types, the GGML bytes (GgmlMatrix) for F16,
        Q4_1, Q5_0 and Q5_1, an fp32 DenseMatrix for F32 (and rows that are
        not whole 8-value groups); uploaded on first use."""
        hit = self._dev.get(name)
        if hit is not None:
            return hit
        info = self.tensors[name]
        if len(info.shape) not in (2, 3):
            raise ValueError(f'{name}: a device matrix needs 2 or 3 dimensions, got {info.shape}')
        batch = info.shape[0] if len(info.shape) == 3 else 1
        rows, cols = info.shape[-2], info.shape[-1]
        block, _ = block_layout(info.ggml_type)
        if cols % block:
            raise ValueError(f'{name}: row length {cols} is not divisible by quantization block {block}')
        raw = self.raw_tensor(name)
        try:
            if info.ggml_type in _PACKED:
                m = device.QMat.from_ggml(raw, info.ggml_type, rows, cols, batch)
            elif info.ggml_type in _RAW and cols % 8 == 0:
                m = GgmlMatrix(raw, info.ggml_type, batch, rows, cols)
            else:
                from .dequant import dequantize_device
                m = DenseMatrix(dequantize_device(raw, info.ggml_type, (batch * rows, cols)), batch, rows, cols)
        finally:
            raw.release()
        if self._dev_bytes + m.device_bytes <= self._dev_limit:
            self._dev[name] = m
            self._dev_bytes += m.device_bytes
        return m

    def _matrix_args(self, name, row_chunk):
        info = self.tensors[name]
        if row_chunk < 1:
            raise ValueError('row_chunk must be positive')
        rows, cols = info.shape
        block, _ = block_layout(info.ggml_type)
        if cols % block:
            raise ValueError(f'{name}: row length {cols} is not divisible by quantization block {block}')
        return rows, cols

    def matvec(self, name, vector, *, row_chunk=1024):
        """W @ x for the GGUF matrix W [out, in] (float32 [out]), on the GPU.
        row_chunk is validated as in the reference; the device product has no chunks."""
        info = self.tensors[name]
        if len(info.shape) != 2:
            raise ValueError(f'{name}: matvec requires a 2-D tensor, got {info.shape}')
        x = np.asarray(vector, dtype=np.float32)
        if x.ndim != 1 or x.size != info.shape[1]:
            raise ValueError(f'{name}: expected vector shape ({info.shape[1]},), got {x.shape}')
        self._matrix_args(name, row_chunk)
        m = self.device_matrix(name)
        return m.matvec(device.to_device_f32(x)).cpu().numpy()

    def matmul(self, name, vectors, *, row_chunk=1024):
        """X @ W^T for X [tokens, in] (float32 [tokens, out]), on the GPU: the MFMA
        GEMM from native_quant.GEMM_TOKENS tokens on for the packed types."""
        from .native_quant import GEMM_TOKENS
        info = self.tensors[name]
        if len(info.shape) != 2:
            raise ValueError(f'{name}: matmul requires a 2-D tensor, got {info.shape}')
        x = np.asarray(vectors, dtype=np.float32)
        if x.ndim != 2 or x.shape[1] != info.shape[1]:
            raise ValueError(f'{name}: expected batch shape (tokens, {info.shape[1]}), got {x.shape}')
        self._matrix_args(name, row_chunk)
        if x.shape[0] == 0:
            return np.empty((0, info.shape[0]), dtype=np.float32)
        m = self.device_matrix(name)
        xd = device.to_device_f32(x)
        if isinstance(m, device.QMat) and x.shape[0] >= GEMM_TOKENS:
            return m.matmul(xd).cpu().numpy()
        return m.matvec(xd).reshape(x.shape[0], -1).cpu().numpy()

    def find(self, *suffixes):
        # exact names first, so `output.weight` is not `blk.N.attn_output.weight`
        for s in suffixes:
            if s in self.tensors:
                return s
        for s in suffixes:
            for name in self.tensors:
                if name.endswith('.' + s):
                    return name
        return None

    def close(self):
        for m in self._dev.values():
            m.close()
        self._dev.clear()
        self._dev_bytes = 0
        self._map.close()
        self._file.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
