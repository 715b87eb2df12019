"""A small GGUF v2/v3 writer for the reader tests (the format of
engine/gguf_parser.py:104-140: header, metadata, tensor infos, aligned data)."""
import struct

import numpy as np

_FMT = {0: '<B', 1: '<b', 2: '<H', 3: '<h', 4: '<I', 5: '<i', 6: '<f', 7: '<?', 10: '<Q', 11: '<q', 12: '<d'}


def gguf_string(s):
    raw = s.encode('utf-8')
    return struct.pack('<Q', len(raw)) + raw


def value(typ, v):
    if typ == 8:
        return gguf_string(v)
    if typ == 9:
        et, items = v
        return struct.pack('<IQ', et, len(items)) + b''.join(value(et, x) for x in items)
    return struct.pack(_FMT[typ], v)


def build(tensors, metadata=(), version=3, alignment=None, offsets=None):
    """tensors: [(name, shape [out, in] order, ggml_type, raw bytes)];
    metadata: [(key, type, value)]. Returns the file bytes."""
    meta = list(metadata)
    if alignment is not None:
        meta.insert(0, ('general.alignment', 4, alignment))
    align = alignment if alignment and 0 < alignment <= 4096 else 32
    head = bytearray(b'GGUF' + struct.pack('<IQQ', version, len(tensors), len(meta)))
    for key, typ, v in meta:
        head += gguf_string(key) + struct.pack('<I', typ) + value(typ, v)
    rel, data = [], bytearray()
    for _, _, _, raw in tensors:
        data += bytes((-len(data)) % align)
        rel.append(len(data))
        data += raw
    if offsets is not None:
        rel = list(offsets)
    for (name, shape, typ, _), off in zip(tensors, rel):
        dims = tuple(reversed(shape))
        head += gguf_string(name) + struct.pack('<I', len(dims)) + struct.pack(f'<{len(dims)}Q', *dims)
        head += struct.pack('<IQ', typ, off)
    head += bytes((-len(head)) % align)
    return bytes(head) + bytes(data)


def f16_matrix(rows, cols, seed=0):
    return np.random.default_rng(seed).standard_normal((rows, cols)).astype(np.float16)
