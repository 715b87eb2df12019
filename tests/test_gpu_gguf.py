"""GGUFFile device paths against the fp64 oracle: every tensor type through
matvec / matmul / tensor / tensor_row, device residency, close(), the ZAYA
expert mixin on a 3-D tensor, and the mmap-close regression of the
native_quant weight cache.

Tolerances: the packed-type matvec and the fp32 matrix path sum exact
products in fp32 (normwise error ~1e-6, gate 1e-5); the MFMA GEMM rounds the
activations to f16 (gate 1e-3, as test_gpu_gemm.py); decodes are bit-exact.
"""
import mmap

import numpy as np
import pytest

from oracle import quant
from tests.conftest import normwise_rel
from tests.gguf_writer import build
from tests.gpu_util import bits, random_ggml

pytestmark = pytest.mark.gpu

ROWS, COLS = 96, 512
TYPES = (0, 1, 2, 3, 6, 7, 8, 12, 13, 14)


@pytest.fixture(scope='module')
def model(tmp_path_factory):
    rng = np.random.default_rng(7)
    tensors, raws = [], {}
    for t in TYPES:
        raw = random_ggml(rng, t, ROWS * COLS)
        raws[t] = raw
        tensors.append((f'blk.0.w{t}.weight', (ROWS, COLS), t, raw))
    experts = random_ggml(rng, 14, 3 * 64 * 256)
    tensors.append(('blk.0.ffn_down_exps.weight', (3, 64, 256), 14, experts))
    tensors.append(('output_norm.weight', (COLS,), 0, rng.standard_normal(COLS).astype(np.float32).tobytes()))
    path = tmp_path_factory.mktemp('gguf') / 'model.gguf'
    path.write_bytes(build(tensors, metadata=[('general.architecture', 8, 'llama')], alignment=32))
    return path, raws, experts


def test_tensor_and_rows_are_bit_exact(model):
    from localai_amd.gguf import GGUFFile
    path, raws, _ = model
    with GGUFFile(path) as g:
        for t in TYPES:
            name = f'blk.0.w{t}.weight'
            want = quant.dequantize(raws[t], t, (ROWS, COLS))
            got = g.tensor(name)
            assert got.shape == (ROWS, COLS)
            np.testing.assert_array_equal(bits(got), bits(want))
            for r in (0, 37, ROWS - 1):
                np.testing.assert_array_equal(bits(g.tensor_row(name, r)), bits(want[r]))
        norm = g.tensor('output_norm.weight')
        assert norm.shape == (COLS,)


@pytest.mark.parametrize('t', TYPES)
def test_matvec_every_type(model, t):
    from localai_amd.gguf import GGUFFile
    path, raws, _ = model
    x = np.random.default_rng(t).standard_normal(COLS).astype(np.float32)
    want = quant.matvec_exact(raws[t], t, ROWS, COLS, x)
    with GGUFFile(path) as g:
        y = g.matvec(f'blk.0.w{t}.weight', x)
        assert y.dtype == np.float32 and y.shape == (ROWS,)
        assert normwise_rel(y, want) < 1e-5
        # the second call reuses the device copy
        m = g.device_matrix(f'blk.0.w{t}.weight')
        assert g.device_matrix(f'blk.0.w{t}.weight') is m
        np.testing.assert_array_equal(g.matvec(f'blk.0.w{t}.weight', x), y)


@pytest.mark.parametrize('t', TYPES)
@pytest.mark.parametrize('tokens', [3, 40])
def test_matmul_every_type(model, t, tokens):
    from localai_amd.gguf import GGUFFile
    from localai_amd.native_quant import GEMM_TOKENS
    path, raws, _ = model
    X = np.random.default_rng(100 + t).standard_normal((tokens, COLS)).astype(np.float32)
    want = quant.matmul_exact(raws[t], t, ROWS, COLS, X)
    with GGUFFile(path) as g:
        Y = g.matmul(f'blk.0.w{t}.weight', X)
    assert Y.shape == (tokens, ROWS)
    gemm = t in (2, 8, 12, 13, 14) and tokens >= GEMM_TOKENS
    assert normwise_rel(Y, want) < (1e-3 if gemm else 1e-5)


def test_zaya_expert_mixin_uses_the_file_device_copy(model):
    from localai_amd.gguf import GGUFFile
    from localai_amd.moe import ZayaExpertsMixin
    path, _, experts = model
    name = 'blk.0.ffn_down_exps.weight'

    class Zaya(ZayaExpertsMixin):
        n_experts = 3

        def __init__(self, gguf):
            self.gguf = gguf

    x = np.random.default_rng(5).standard_normal(256).astype(np.float32)
    per = 64 * (256 // 256) * 210
    with GGUFFile(path) as g:
        z = Zaya(g)
        for e in range(3):
            want = quant.matvec_exact(experts[e * per:(e + 1) * per], 14, 64, 256, x)
            assert normwise_rel(z._expert_matvec(name, e, x), want) < 1e-5
        assert name in g._dev
        with pytest.raises(IndexError):
            z._expert_matvec(name, 3, x)


def test_close_frees_device_copies_and_unmaps(model):
    from localai_amd.gguf import GGUFFile
    path, raws, _ = model
    g = GGUFFile(path)
    g.matvec('blk.0.w12.weight', np.ones(COLS, np.float32))
    g.matvec('blk.0.w1.weight', np.ones(COLS, np.float32))
    assert len(g._dev) == 2 and g._dev_bytes > 0
    g.close()
    assert g._map.closed and not g._dev and g._dev_bytes == 0


def test_native_quant_cache_does_not_pin_the_mmap(model):
    """engine/gguf_parser.py:175-193 passes mmap slices to native_quant.matvec and
    closes the map in close(); a cached device copy must not hold the export."""
    from localai_amd import native_quant
    path, raws, _ = model
    from localai_amd.gguf import GGUFFile
    with GGUFFile(path) as g:
        info = g.tensors['blk.0.w14.weight']
    with open(path, 'rb') as f:
        m = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        raw = memoryview(m)[info.offset:info.offset + info.nbytes]
        x = np.random.default_rng(9).standard_normal(COLS).astype(np.float32)
        y = native_quant.matvec(raw, x, ROWS, COLS, 14)
        y2 = native_quant.matvec(memoryview(m)[info.offset:info.offset + info.nbytes], x, ROWS, COLS, 14)
        np.testing.assert_array_equal(y, y2)
        n_cached = len(native_quant._cache)
        del raw
        m.close()                      # raises BufferError if an export is still held
    assert normwise_rel(y, quant.matvec_exact(raws[14], 14, ROWS, COLS, x)) < 1e-5
    # the entry of the closed map is dropped on the next use of the cache
    native_quant.matvec(raws[12], np.ones(COLS, np.float32), ROWS, COLS, 12)
    assert len(native_quant._cache) <= n_cached


@pytest.mark.parametrize('t', (1, 3, 6, 7, 0, 2, 8))
@pytest.mark.parametrize('rows,cols,tokens', [(1, 32 * 8, 1), (77, 512, 1), (257, 4096, 3), (33, 2048, 5)])
def test_ggml_matvec_from_file_bytes(t, rows, cols, tokens):
    """localai_hip_ggml_matvec on the GGML bytes as they are (F16, Q4_1,
    Q5_0, Q5_1, and F32, Q4_0, Q8_0): against the fp64 product of the exact
    decode, normwise 1e-5 (fp32 sums of exact products); repeated calls are
    bit-identical."""
    import ctypes
    import torch
    from localai_amd import _lib, device
    if cols % 32 and t not in (0, 1):
        pytest.skip('block types need cols % 32 == 0')
    rng = np.random.default_rng(1000 * t + rows + tokens)
    raw = random_ggml(rng, t, rows * cols)
    x = rng.standard_normal((tokens, cols)).astype(np.float32)
    w = torch.from_numpy(np.frombuffer(raw, np.uint8).copy()).to(device.device())
    xd = device.to_device_f32(x)
    lib = _lib.load()
    outs = []
    for _ in range(2):
        y = torch.empty((tokens, rows), dtype=torch.float32, device=device.device())
        _lib.check(lib.localai_hip_ggml_matvec(t, device.ptr(w), rows, cols, device.ptr(xd), tokens, device.ptr(y),
                                               ctypes.c_void_p(device.stream_ptr())))
        outs.append(y.cpu().numpy())
    np.testing.assert_array_equal(bits(outs[0]), bits(outs[1]))
    want = x.astype(np.float64) @ quant.dequantize(raw, t, (rows, cols)).astype(np.float64).T
    assert normwise_rel(outs[0], want) < 1e-5


def test_ggml_matvec_rejects_what_it_cannot_read():
    import ctypes
    import torch
    from localai_amd import _lib, device
    lib = _lib.load()
    w = torch.zeros(4096, dtype=torch.uint8, device=device.device())
    x = torch.zeros(64, dtype=torch.float32, device=device.device())
    y = torch.empty(64, dtype=torch.float32, device=device.device())
    p = device.ptr
    assert lib.localai_hip_ggml_matvec(12, p(w), 1, 256, p(x), 1, p(y), None) == 2   # Q4_K: its own kernels
    assert lib.localai_hip_ggml_matvec(3, p(w), 1, 48, p(x), 1, p(y), None) == 1     # not whole blocks
    assert lib.localai_hip_ggml_matvec(1, p(w), 1, 12, p(x), 1, p(y), None) == 1     # not whole 8-value groups
    assert lib.localai_hip_ggml_matvec(1, p(w) + 2, 1, 16, p(x), 1, p(y), None) == 1   # F16 rows unaligned


def test_reader_keeps_f16_and_5bit_types_as_file_bytes(model):
    """F16, Q4_1, Q5_0 and Q5_1 matrices stay on the device as their GGML
    bytes (0.6 to 2 bytes per value instead of fp32's 4)."""
    from localai_amd.gguf import GGUFFile, GgmlMatrix
    path, raws, _ = model
    with GGUFFile(path) as g:
        for t in (1, 3, 6, 7):
            m = g.device_matrix(f'blk.0.w{t}.weight')
            assert isinstance(m, GgmlMatrix)
            assert len(raws[t]) <= m.device_bytes < len(raws[t]) + 256
