"""Build liblocalai_hip.so (gfx950) from localai_amd/csrc with hipcc.

    python -m localai_amd.build            # compile every source, link the .so

Every source is compiled on each call (the objects go to localai_amd/_build/,
the library to localai_amd/liblocalai_hip.so). Packed-fp32 instruction
selection is disabled for all device code. Kernels whose global loads count
their own waits are checked in their generated assembly (isa_check.py); the
build fails if one touches a register whose load may still be in flight.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
BUILD = PKG / '_build'
LIB = PKG / 'liblocalai_hip.so'
ARCH = os.environ.get('LOCALAI_HIP_ARCH', 'gfx950')

HIPCC = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
COMMON = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}',
          '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
          '-Wno-unused-result', '-I', str(CSRC), '-I', str(PKG.parent / 'include')]


def sources():
    return sorted(list(CSRC.glob('*.hip')) + list(CSRC.glob('*.cpp')))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.name + '.o')
    cmd = [HIPCC, *COMMON, '-c', str(src), '-o', str(obj)]
    if src.suffix == '.cpp':
        cmd[1:1] = ['-x', 'hip']
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{r.stderr[-6000:]}')
    return obj


# kernels whose global loads are asm with hand-counted waits (isa_check.py):
# (source, kernel, None) for register loads, (source, kernel, n) for a ring of
# LDS stages filled by global_load_lds, n copies per stage and wave (n = 0: a
# double buffer, whose every copy from before the last barrier has landed by
# the LDS reads after it)
COUNTED_LOADS = [('gemm.hip', 'gemm_cu_q80_kernel', None), ('moe.hip', 'moe_route_logits_kernel', 4),
                 ('gemm.hip', 'gemm_tile_kernel', 0)]


def _check(item) -> None:
    from .isa_check import check_lds_ring, check_source
    src, kernel, per_stage = item
    out = BUILD / (src + '.' + kernel + '.s')
    if per_stage is None:
        check_source(HIPCC, COMMON, CSRC / src, kernel, out)
    else:
        check_lds_ring(HIPCC, COMMON, CSRC / src, kernel, per_stage, out)


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs) + len(COUNTED_LOADS))) as ex:
        checks = [ex.submit(_check, item) for item in COUNTED_LOADS]
        objs = list(ex.map(_compile, srcs))
        for c in checks:
            c.result()
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [HIPCC, '-shared', f'--offload-arch={ARCH}', '-o', str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'link failed:\n{r.stderr[-6000:]}')
    os.replace(tmp, LIB)
    if verbose:
        print(f'built {LIB}')
    return LIB


if __name__ == '__main__':
    build(verbose=True)
    sys.exit(0)
