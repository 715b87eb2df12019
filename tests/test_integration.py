"""The reference-side binding in the maintainers' integration notes at the
repository root, run as written.

The two residency blocks (register the GGUF map in GGUFFile.__init__,
unregister it in close()) are read out of those notes (the fenced python
blocks marked `<!-- snippet: NAME -->`) and executed against
an object that opens a GGUF file exactly as engine/gguf_parser.py:50-53 does
(`open('rb')`, `mmap.mmap(fileno, 0, access=mmap.ACCESS_READ)`). The CPU test
checks that registration works on that read-only map and that the map can
still be closed; the GPU test drives the legacy export localai_q4k_matvec
twice on a tensor slice of the map, as engine/native_quant.py:102-126 does,
and checks that the second call reuses the device copy."""
import ctypes
import mmap
import re
import types
from pathlib import Path

import numpy as np
import pytest

from oracle import quant
from tests import gguf_writer
from tests.conftest import normwise_rel

ROOT = Path(__file__).resolve().parents[1]


def snippet(name):
    text = (ROOT / 'INTEGRATION.md').read_text()
    m = re.search(r'<!-- snippet: ' + re.escape(name) + r' -->\s*```python\n(.*?)```', text, re.S)
    assert m, f'snippet {name} not found in the integration notes'
    lines = m.group(1).splitlines()
    indent = min(len(s) - len(s.lstrip()) for s in lines if s.strip())
    return '\n'.join(s[indent:] for s in lines)


class ReadOnlyGGUF:
    """The file handling of engine/gguf_parser.py:48-53 and :83-86, nothing else."""

    def __init__(self, path):
        self.path = Path(path)
        self._file = self.path.open('rb')
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)

    def close(self):
        self._map.close()
        self._file.close()


def run_block(name, obj, lib):
    env = {'self': obj, 'ctypes': ctypes, 'np': np,
           'native_quant': types.SimpleNamespace(get_native=lambda: lib)}
    exec(compile(snippet(name), f'INTEGRATION.md:{name}', 'exec'), env)


def _file(tmp_path, rows=256, cols=1024, seed=5):
    from localai_amd import synth
    rng = np.random.default_rng(seed)
    raw = synth.quant_tensor(rng, 12, rows, cols)
    path = tmp_path / 'm.gguf'
    path.write_bytes(gguf_writer.build([('blk.0.ffn_gate.weight', (rows, cols), 12, raw)]))
    return path, raw


def _tensor_offset(path, raw):
    data = path.read_bytes()
    off = data.rfind(raw)
    assert off > 0
    return off


def test_writable_export_fails_on_the_reference_map(tmp_path):
    """Why the snippet takes a NumPy view: ctypes' from_buffer needs a
    writable buffer, and the reference's map is ACCESS_READ."""
    path, _ = _file(tmp_path)
    g = ReadOnlyGGUF(path)
    try:
        with pytest.raises(TypeError):
            (ctypes.c_char * len(g._map)).from_buffer(g._map)
    finally:
        g.close()


def test_register_snippet_on_read_only_map_then_close(tmp_path):
    from localai_amd import _lib
    lib = _lib.load()
    path, _ = _file(tmp_path)
    g = ReadOnlyGGUF(path)
    run_block('gguf-register', g, lib)
    assert g._hip_base is not None and g._hip_base != 0
    run_block('gguf-unregister', g, lib)
    assert g._hip_base is None
    g.close()                     # no buffer export was left behind
    assert g._map.closed
    # unregistering twice is an argument error, not a crash
    assert lib.localai_hip_unregister_host(ctypes.c_void_p(12345)) == 1


@pytest.mark.gpu
def test_legacy_matvec_reuses_device_copy_of_registered_map(tmp_path):
    from localai_amd import _lib
    lib = _lib.load()
    rows, cols = 256, 1024
    path, raw = _file(tmp_path, rows, cols)
    off = _tensor_offset(path, raw)
    x = np.random.default_rng(9).standard_normal(cols).astype(np.float32)
    want = quant.matvec_exact(raw, 12, rows, cols, x)
    lib.localai_hip_cache_clear()
    g = ReadOnlyGGUF(path)
    run_block('gguf-register', g, lib)
    n0 = int(lib.localai_hip_cache_entries())
    outs = []
    for call in range(2):
        # engine/native_quant.py:112-125: a zero-copy view of the map slice
        view = np.frombuffer(memoryview(g._map)[off:off + len(raw)], dtype=np.uint8)
        out = np.empty(rows, np.float32)
        lib.localai_q4k_matvec(view.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)),
                               x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                               out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), rows, cols, 8)
        del view
        assert lib.localai_hip_last_status() == 0, lib.localai_hip_last_error()
        outs.append(out)
        assert int(lib.localai_hip_cache_entries()) == n0 + 1   # the second call adds no copy
    np.testing.assert_array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    assert normwise_rel(outs[0], want) < 1e-5
    run_block('gguf-unregister', g, lib)
    assert int(lib.localai_hip_cache_entries()) == n0
    g.close()
    assert g._map.closed
