"""GGUF reader (localai_amd.gguf): parsing, validation and lookup on the CPU.

Mirrors the reference's tests/test_gguf_parser.py (thread policy table,
suffix lookup, v3 metadata and offsets) and adds the validation rules of
engine/gguf_parser.py:104-140 one by one. The device products are in
test_gpu_gguf.py.
"""
import struct

import numpy as np
import pytest

from localai_amd.gguf import GGUFFile, _native_thread_count
from tests.gguf_writer import build, gguf_string


def write(tmp_path, blob, name='t.gguf'):
    p = tmp_path / name
    p.write_bytes(blob)
    return p


# ---- thread policy (reference tests/test_gguf_parser.py:19-42) -------------

def test_decode_thread_override_is_opt_in_and_does_not_change_prefill(monkeypatch):
    import os
    monkeypatch.setenv('LOCALAI_NATIVE_DECODE_THREADS', '8')
    assert _native_thread_count(4096, 14) == min(8, os.cpu_count() or 1)
    assert _native_thread_count(4096, 14, batched=True) == min(6, os.cpu_count() or 1)


def test_invalid_decode_thread_override_falls_back_to_policy(monkeypatch):
    import os
    monkeypatch.setenv('LOCALAI_NATIVE_DECODE_THREADS', 'not-a-number')
    assert _native_thread_count(4096, 14) == min(7, os.cpu_count() or 1)


def test_thread_policy_table(monkeypatch):
    import os
    monkeypatch.delenv('LOCALAI_NATIVE_DECODE_THREADS', raising=False)
    c = os.cpu_count() or 1
    for rows, t, batched, want in [(128256, 12, False, 8), (128256, 14, False, 8), (14336, 12, False, 8),
                                   (4096, 12, False, 8), (4096, 14, False, 7), (2048, 14, False, 6),
                                   (128256, 8, False, 6), (14336, 12, True, 6), (4096, 14, True, 6),
                                   (128256, 14, True, 8), (1024, 2, False, 4), (1024, 0, False, 4)]:
        assert _native_thread_count(rows, t, batched=batched) == min(want, c), (rows, t, batched)


# ---- lookup -----------------------------------------------------------------

def test_suffix_lookup_does_not_confuse_attention_output_with_output_head():
    g = GGUFFile.__new__(GGUFFile)
    g.tensors = {'blk.0.attn_output.weight': object()}
    assert g.find('output.weight') is None
    g.tensors = {'blk.0.attn_output.weight': object(), 'output.weight': object()}
    assert g.find('output.weight') == 'output.weight'
    g.tensors = {'blk.3.ffn_down.weight': object()}
    assert g.find('missing', 'ffn_down.weight') == 'blk.3.ffn_down.weight'


# ---- parsing ----------------------------------------------------------------

def test_v3_metadata_tensor_offsets_and_raw_bytes(tmp_path):
    # one Q8_0 block, the reference test's file (tests/test_gguf_parser.py:50-65)
    q = np.arange(-16, 16, dtype=np.int8)
    blk = np.float16(.25).tobytes() + q.tobytes()
    p = write(tmp_path, build([('test.weight', (32,), 8, blk)], alignment=32))
    with GGUFFile(p) as g:
        assert g.version == 3
        assert g.metadata['general.alignment'] == 32
        info = g.tensors['test.weight']
        assert info.shape == (32,) and info.ggml_type == 8 and info.nbytes == 34
        assert info.offset % 32 == 0
        assert bytes(g.raw_tensor('test.weight')) == blk


def test_metadata_value_types_and_shapes(tmp_path):
    meta = [('u8', 0, 200), ('i8', 1, -5), ('u16', 2, 60000), ('i16', 3, -300), ('u32', 4, 4000000000),
            ('i32', 5, -7), ('f32', 6, 1.5), ('flag', 7, True), ('name', 8, 'llama ✓'),
            ('ids', 9, (5, [1, -2, 3])), ('words', 9, (8, ['a', 'bc'])), ('u64', 10, 2 ** 40),
            ('i64', 11, -2 ** 40), ('f64', 12, 0.1)]
    w = np.zeros((3, 64), np.float32).tobytes()
    h = np.zeros((2, 4, 32), np.float16).tobytes()
    p = write(tmp_path, build([('w', (3, 64), 0, w), ('e', (2, 4, 32), 1, h)], metadata=meta, version=2,
                              alignment=64))
    with GGUFFile(p) as g:
        assert g.version == 2 and g.alignment == 64
        for k, _, v in meta:
            if isinstance(v, tuple):
                v = v[1]
            got = g.metadata[k]
            assert got == pytest.approx(v) if isinstance(v, float) else got == v, k
        assert g.tensors['w'].shape == (3, 64) and g.tensors['e'].shape == (2, 4, 32)
        assert g.tensors['w'].offset % 64 == 0 and g.tensors['e'].offset % 64 == 0
        assert bytes(g.raw_tensor('e')) == h


@pytest.mark.parametrize('align', [0, 8192])
def test_out_of_range_alignment_means_32(tmp_path, align):
    blk = np.float16(1.0).tobytes() + bytes(32)
    p = write(tmp_path, build([('a', (32,), 8, blk), ('b', (32,), 8, blk)], alignment=align))
    with GGUFFile(p) as g:
        assert g.alignment == 32
        assert g.tensors['b'].offset - g.tensors['a'].offset == 64


def test_unknown_tensor_type_is_listed_and_fails_on_access(tmp_path):
    p = write(tmp_path, build([('odd', (32,), 99, bytes(64))]))
    with GGUFFile(p) as g:
        assert g.tensors['odd'].ggml_type == 99
        with pytest.raises(NotImplementedError):
            g.raw_tensor('odd')


def test_close_succeeds_after_raw_views_are_dropped(tmp_path):
    blk = np.float16(1.0).tobytes() + bytes(32)
    p = write(tmp_path, build([('a', (32,), 8, blk)]))
    g = GGUFFile(p)
    assert bytes(g.raw_tensor('a')) == blk
    g.close()
    assert g._map.closed


# ---- rejected files -----------------------------------------------------------

def _header(version=3, n_tensors=0, n_kv=0):
    return b'GGUF' + struct.pack('<IQQ', version, n_tensors, n_kv)


def _tensor_info(name, dims, typ, off):
    return gguf_string(name) + struct.pack('<I', len(dims)) + struct.pack(f'<{len(dims)}Q', *dims) + \
        struct.pack('<IQ', typ, off)


def _pad(b, align=32):
    return b + bytes((-len(b)) % align)


BLK = np.float16(1.0).tobytes() + bytes(32)   # one Q8_0 block


@pytest.mark.parametrize('blob,match', [
    (b'GGUX' + bytes(60), 'not a GGUF file'),
    (_header(version=1), 'unsupported'),
    (_header(version=4), 'unsupported'),
    (_header(n_tensors=10_000_001), 'Invalid GGUF counts'),
    (_header(n_kv=1_000_001), 'Invalid GGUF counts'),
    (_header(n_kv=1)[:-3], 'truncated'),
    (_header(n_kv=1) + struct.pack('<Q', 1 << 40), 'string length'),
    (_header(n_kv=1) + gguf_string('k') + struct.pack('<I', 13) + bytes(8), 'value type 13'),
    (_header(n_kv=1) + gguf_string('k') + struct.pack('<IIQ', 9, 4, 100_000_001), 'array length'),
    (_pad(_header(n_tensors=1) + _tensor_info('t', (), 8, 0)), 'dimension count 0'),
    (_pad(_header(n_tensors=1) + _tensor_info('t', (1,) * 9, 8, 0)), 'dimension count 9'),
    (_pad(_header(n_tensors=1) + _tensor_info('t', (32, 0), 8, 0)), 'dimensions must be positive'),
    (_pad(_header(n_tensors=1) + _tensor_info('t', (32,), 8, 16)) + BLK, 'not aligned'),
    (_pad(_header(n_tensors=2) + _tensor_info('t', (32,), 8, 0) + _tensor_info('t', (32,), 8, 64)) + BLK * 3,
     'Duplicate tensor name'),
    (_pad(_header(n_tensors=1) + _tensor_info('t', (64,), 8, 0)) + BLK, 'extends past end'),
    (_pad(_header(n_tensors=2) + _tensor_info('a', (64,), 8, 0) + _tensor_info('b', (32,), 8, 32)) + BLK * 2,
     'overlap'),
])
def test_rejected_files(tmp_path, blob, match):
    with pytest.raises(ValueError, match=match):
        GGUFFile(write(tmp_path, blob))


def test_rejected_file_closes_its_handles(tmp_path):
    p = write(tmp_path, b'GGUX' + bytes(60))
    opened = []
    real_open = type(p).open

    def spy(self, *a, **k):
        f = real_open(self, *a, **k)
        opened.append(f)
        return f
    import pathlib
    pathlib.Path.open = spy
    try:
        with pytest.raises(ValueError):
            GGUFFile(p)
    finally:
        pathlib.Path.open = real_open
    assert opened and opened[0].closed


def test_matrix_entry_points_validate_before_device_use(tmp_path):
    w = np.zeros((4, 32), np.float32).tobytes()
    p = write(tmp_path, build([('w', (4, 32), 0, w), ('v', (32,), 0, bytes(128))]))
    with GGUFFile(p) as g:
        with pytest.raises(ValueError, match='requires a 2-D tensor'):
            g.matvec('v', np.zeros(32, np.float32))
        with pytest.raises(ValueError, match='expected vector shape'):
            g.matvec('w', np.zeros(31, np.float32))
        with pytest.raises(ValueError, match='row_chunk must be positive'):
            g.matvec('w', np.zeros(32, np.float32), row_chunk=0)
        with pytest.raises(ValueError, match='expected batch shape'):
            g.matmul('w', np.zeros((2, 31), np.float32))
        with pytest.raises(ValueError, match='tensor_row requires a 2-D tensor'):
            g.tensor_row('v', 0)
        with pytest.raises(IndexError):
            g.tensor_row('w', 4)
        assert g.matmul('w', np.zeros((0, 32), np.float32)).shape == (0, 4)
