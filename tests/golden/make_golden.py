"""Write tests/golden/ref_native_quant.npz from the reference's own kernels.

Run in a container that has /root/reference (builds oracle/_ref first):

    make -C oracle && python tests/golden/make_golden.py

The reference library is engine/native_quant.cpp compiled from source by
oracle/Makefile. The cases are the reference test suite's own randomised
cases (tests/test_dequant.py:119-230): same seeds, shapes, fixed fp16 scales
and byte generation. Stored per GGML type t:

  raw_t, x_t        inputs of the matvec case (seed/shape of the reference test)
  matvec_t          localai_*_matvec output (threads=4)
  decode_t          exact decode of the first 4 rows, read back through the
                    reference's batched matmul with one-hot vectors
  raw_mm_t          64-row matrix for the batched case (seed 53, :160-177)
  matmul_t          localai_*_matmul output for `vectors` (5 tokens), [5, 64]
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from oracle import ref  # noqa: E402

OUT = Path(__file__).resolve().parent / 'ref_native_quant.npz'

# type -> (seed, bytes/block, block, scale offset, d, dmin)   tests/test_dequant.py:119-230
CASES = {
    8: (50, 34, 32, 0, 0.03125, None),
    2: (55, 18, 32, 0, 0.03125, None),
    13: (54, 176, 256, 0, 0.0005, 0.00025),
    12: (51, 144, 256, 0, 0.0005, 0.00025),
    14: (52, 210, 256, 208, 0.0005, None),
}


def make_raw(rng, rows, cols, bpb, block, off, d, dmin):
    blocks = cols // block
    raw = bytearray(rng.integers(0, 256, size=rows * blocks * bpb, dtype=np.uint8).tobytes())
    for r in range(rows):
        for b in range(blocks):
            o = (r * blocks + b) * bpb + off
            raw[o:o + 2] = np.float16(d).tobytes()
            if dmin is not None:
                raw[o + 2:o + 4] = np.float16(dmin).tobytes()
    return bytes(raw)


def main():
    if not ref.available():
        raise SystemExit('oracle/_ref is not built: run `make -C oracle` first')
    out = {}
    rows, cols = 300, 512
    for t, (seed, bpb, block, off, d, dmin) in CASES.items():
        rng = np.random.default_rng(seed)
        raw = make_raw(rng, rows, cols, bpb, block, off, d, dmin)
        x = rng.normal(size=cols).astype(np.float32)
        out[f'raw_{t}'] = np.frombuffer(raw, dtype=np.uint8)
        out[f'x_{t}'] = x
        out[f'matvec_{t}'] = ref.matvec(raw, x, rows, cols, t, threads=4)
        out[f'decode_{t}'] = ref.decode_rows(raw[:4 * (cols // block) * bpb], t, 4, cols)
    rng = np.random.default_rng(53)
    vectors = rng.normal(size=(5, cols)).astype(np.float32)
    out['vectors'] = vectors
    for t, (_, bpb, block, off, _, _) in CASES.items():
        raw = make_raw(rng, 64, cols, bpb, block, off, 0.03125, 0.015625 if t in (12, 13) else None)
        out[f'raw_mm_{t}'] = np.frombuffer(raw, dtype=np.uint8)
        out[f'matmul_{t}'] = ref.matmul(raw, vectors, 64, cols, t, threads=4)
    np.savez_compressed(OUT, **out)
    print(f'wrote {OUT} ({OUT.stat().st_size} bytes)')


if __name__ == '__main__':
    main()
