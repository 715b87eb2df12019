"""C-ABI checks that need no GPU: the library loads, exports every symbol that
include/localai_hip.h declares, and rejects bad arguments before touching a
device."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from localai_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / 'include' / 'localai_hip.h'


def declared():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(localai_\w+)\s*\(', text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_mirrors_header():
    assert sorted(_lib.SIGNATURES) == declared()


def test_legacy_symbols_present():
    lib = _lib.load()
    for n in ('q8_0', 'q4_0', 'q4k', 'q5k', 'q6k'):
        assert hasattr(lib, f'localai_{n}_matvec') and hasattr(lib, f'localai_{n}_matmul')


def test_block_layout_matches_reference_table():
    lib = _lib.load()
    table = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
             8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}
    for t, lay in table.items():
        v, b = ctypes.c_int(), ctypes.c_int()
        assert lib.localai_hip_block_layout(t, ctypes.byref(v), ctypes.byref(b)) == 0
        assert (v.value, b.value) == lay
    assert lib.localai_hip_block_layout(99, None, None) == 2   # LOCALAI_ETYPE
    assert lib.localai_hip_last_error()


def test_argument_errors_before_device_use():
    lib = _lib.load()
    assert lib.localai_hip_dequant(99, None, 0, None, None) == 2
    assert lib.localai_hip_dequant(12, None, 100, None, None) == 1      # not a multiple of 256
    h = ctypes.c_void_p()
    assert lib.localai_hip_qmat_create(3, 4, 32, 1, ctypes.c_void_p(1), 0, None, ctypes.byref(h)) == 2
    assert lib.localai_hip_qmat_create(12, 4, 100, 1, ctypes.c_void_p(1), 0, None, ctypes.byref(h)) == 1
    assert lib.localai_hip_matvec(None, 0, None, None, 1, None) == 1
    assert lib.localai_hip_f32_matvec(None, 4, 4, None, 1, None, None) == 1
    one = ctypes.c_void_p(16)
    assert lib.localai_hip_f32_matvec(one, 0, 4, one, 1, one, None) == 1
    assert lib.localai_hip_zaya_router(*([None] * 5), ctypes.c_float(1e-5), 256, None, None, 256, None, None, 256,
                                       None, None, 17, None, None, None, None, None, None) == 1
    assert lib.localai_hip_zaya_scale(None, None, 4, None, None, None) == 1
    assert lib.localai_hip_moe_experts1(None, 64, None, None, 1, None, None, -1, None, None, 0, None) == 1
    # attention: null buffers, heads not a multiple of kv heads, position past
    # the cache, k without v, misaligned buffers
    att = lambda q, kn, vn, pos, nh, nkv, hd: lib.localai_hip_attention_decode(
        q, kn, vn, one, one, pos, 16, nh, nkv, hd, 0, None, one, None, 0, None)
    assert att(None, None, None, 0, 8, 2, 128) == 1
    assert att(one, None, None, 0, 6, 4, 128) == 1
    assert att(one, None, None, 16, 8, 2, 128) == 1
    assert att(one, one, None, 0, 8, 2, 128) == 1
    assert att(ctypes.c_void_p(20), None, None, 0, 8, 2, 128) == 1
    assert lib.localai_hip_attention_workspace_size(4096, 32, 8, 128) == 8 * 64 * 4 * 130 * 4
    assert lib.localai_hip_attention_workspace_size(4096, 32, 8, 96) == 0
    assert lib.localai_hip_attention_workspace_size(4096, 6, 4, 128) == -1
    assert lib.localai_hip_delta_net_step(*([None] * 7), 32, 128, 128, None) == 1
    assert lib.localai_hip_delta_net_step(*([one] * 7), 0, 128, 128, None) == 1
    with pytest.raises(_lib.HipError):
        _lib.check(lib.localai_hip_dequant(99, None, 0, None, None))


def test_legacy_rejects_misaligned_cols_with_nan_and_status():
    lib = _lib.load()
    raw = np.zeros(1024, np.uint8)
    x = np.ones(100, np.float32)
    out = np.zeros(4, np.float32)
    lib.localai_q4k_matvec(raw.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                           x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                           out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 4, 100, 4)
    assert lib.localai_hip_last_status() == 1
    assert np.isnan(out).all()


@pytest.mark.parametrize('T,E,k,H,I', [(1, 16, 2, 2048, 4096), (31, 16, 4, 512, 256), (32, 128, 8, 2048, 768),
                                       (512, 128, 8, 2048, 768)])
def test_moe_table_offsets_lie_inside_the_workspace(T, E, k, H, I):
    """localai_hip_moe_table_offsets (host arithmetic only): every table is
    256-byte aligned, the tables do not overlap and end inside the workspace
    that localai_hip_moe_workspace_size asks for; the expert GEMM tile list
    exists from 32 tokens on, with its capacity and tile width."""
    lib = _lib.load()
    offs = (ctypes.c_int64 * 12)()
    assert lib.localai_hip_moe_table_offsets(T, E, k, H, I, offs) == 0
    ws = lib.localai_hip_moe_workspace_size(T, E, k, H, I)
    N = T * k
    sizes = [4 * E, 4 * (E + 1), 4 * E, 4, 4 * N, 4 * N]
    gemm = T >= 32
    assert (offs[6] >= 0) == gemm and (offs[11] > 0) == gemm
    if gemm:
        sizes += [4 * offs[10]] * 3 + [4]
    spans = sorted((offs[i], offs[i] + n) for i, n in enumerate(sizes))
    assert all(o % 256 == 0 for o, _ in spans)
    assert all(a_end <= b for (_, a_end), (b, _) in zip(spans, spans[1:]))
    assert spans[-1][1] <= ws
    assert lib.localai_hip_moe_table_offsets(0, E, k, H, I, offs) == 1
    assert lib.localai_hip_moe_table_offsets(T, E, k, H, I, None) == 1
