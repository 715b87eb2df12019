"""Build-time check of kernels that count their own global loads.

Some kernels issue global loads as inline asm and wait for them with
hand-counted ``s_waitcnt vmcnt(N)`` (the compiler's own count was too
cautious to keep the prefetch in flight). The compiler sees such a load's
register as ready at once, so nothing but the kernel's own waits keeps it from
touching the register (a copy, a spill, a reuse as a temporary) while the load
is still in flight. This module reads the kernel's generated gfx9 assembly and
proves that no instruction does.

It is a dataflow analysis over the kernel's control-flow graph. The state at
each instruction is the list of loads that may be in flight (oldest first),
each with the VGPRs it writes; a load appends an entry, ``s_waitcnt vmcnt(N)``
drops all but the newest N (loads complete in order), and where paths join the
lists are aligned on their newest entries and merged register-wise (the more
pessimistic state). Any VALU, LDS or memory instruction that names a register
of an in-flight load is reported, as is a load whose address register is one.
LDS DMA (``global_load_lds``) counts in vmcnt but writes no register.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

_MAXQ = 64
_VRANGE = re.compile(r'v\[(\d+):(\d+)\]')
_VONE = re.compile(r'v(\d+)$')
_LABEL = re.compile(r'^(\.LBB\d+_\d+):')


def _regs(tok: str) -> frozenset:
    tok = tok.strip().split()[0] if tok.strip() else ''
    m = _VRANGE.match(tok)
    if m:
        return frozenset(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _VONE.match(tok)
    return frozenset({int(m.group(1))}) if m else frozenset()


def kernel_lines(asm: str, name: str) -> list[str]:
    """The instruction lines of the first kernel whose symbol contains name
    (or whose symbol is name, for a full mangled name)."""
    lines = asm.split('\n')
    pat = re.escape(name) + ':' if name.startswith('_Z') else r'_Z\S*' + re.escape(name) + r'\S*:'
    start = next(i for i, l in enumerate(lines) if re.match('^' + pat, l))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith('.Lfunc_end'))
    return [l.split(';')[0].strip() for l in lines[start + 1:end]]


def _merge(a: tuple, b: tuple) -> tuple:
    n = max(len(a), len(b))
    a = (frozenset(),) * (n - len(a)) + a
    b = (frozenset(),) * (n - len(b)) + b
    return tuple(x | y for x, y in zip(a, b))


def pending_violations(code: list[str]) -> list[tuple[int, str, str]]:
    """(index, reason, instruction) for every instruction that touches a
    register whose global load may still be in flight."""
    labels = {}
    for i, l in enumerate(code):
        m = _LABEL.match(l)
        if m:
            labels[m.group(1)] = i
    bad: dict[int, tuple[str, str]] = {}

    def run(i: int, q: tuple):
        q = list(q)
        l = code[i]
        if not l or l.startswith('.') or l.startswith('s_nop'):
            return [(i + 1, q)]
        op = l.split()[0]
        if op == 's_waitcnt':
            m = re.search(r'vmcnt\((\d+)\)', l)
            if m:
                del q[:max(0, len(q) - int(m.group(1)))]
            return [(i + 1, q)]
        if op == 's_endpgm':
            return []
        if op == 's_branch':
            return [(labels[l.split()[1]], q)]
        if op.startswith('s_cbranch'):
            return [(i + 1, q), (labels[l.split()[1]], q)]
        if op.startswith(('global_load_lds', 'buffer_load_lds')):
            return [(i + 1, (q + [frozenset()])[-_MAXQ:])]
        if op.startswith(('global_load', 'buffer_load', 'scratch_load', 'flat_load')):
            ops = l.split(None, 1)[1].split(',')
            for t in ops[1:]:
                if any(_regs(t) & r for r in q):
                    bad[i] = ('address register in flight', l)
            return [(i + 1, (q + [_regs(ops[0])])[-_MAXQ:])]
        if op.startswith(('v_', 'ds_', 'global_store', 'buffer_store', 'scratch_store', 'flat_store',
                          'global_atomic')):
            used = set()
            if ' ' in l:
                for t in l.split(None, 1)[1].split(','):
                    used |= _regs(t)
            if any(used & r for r in q):
                bad[i] = ('register in flight', l)
        return [(i + 1, q)]

    state = {0: ()}
    work = [0]
    while work:
        i = work.pop()
        if i >= len(code):
            continue
        for j, q in run(i, state[i]):
            q = tuple(q)
            old = state.get(j)
            new = q if old is None else _merge(old, q)
            if new != old:
                state[j] = new
                work.append(j)
    return [(i, *bad[i]) for i in sorted(bad)]


def lds_ring_violations(code: list[str], per_stage: int) -> list[tuple[int, str, str]]:
    """(index, reason, instruction) for every LDS read that may run while a
    global-to-LDS copy it could depend on is still in flight.

    The kernels this serves fill a ring of LDS stages with ``global_load_lds``
    two chunks ahead (moe_route_logits_kernel): chunk j + 2 is requested after
    the barrier at which chunk j is read, so at that read the copies of chunk
    j + 1 (one stage's worth, issued before this barrier and after the one
    before) may still be in flight, and nothing older. Each copy carries its
    age, the number of ``s_barrier`` instructions passed since it was issued.
    At every LDS read at most ``per_stage`` copies of age >= 1 and none of
    age >= 2 may be in flight: a wait count that is too large, a copy that
    the compiler moved, or a missing wait before the last chunk (whose copies
    are two barriers old by then) all break it. The queue state is the same
    in-order vmcnt model as pending_violations; where paths join, the queues
    are aligned on their newest entries and the older age kept. The check is
    path-insensitive, so it holds only for code whose waits are unconditional
    (the kernel peels its last two chunks for this)."""
    labels = {}
    for i, l in enumerate(code):
        m = _LABEL.match(l)
        if m:
            labels[m.group(1)] = i
    bad: dict[int, tuple[str, str]] = {}

    # an entry: 0 = a load or store, 1 + age = a copy (age capped at 2)
    def run(i: int, q: tuple):
        q = list(q)
        l = code[i]
        if not l or l.startswith('.') or l.startswith('s_nop'):
            return [(i + 1, q)]
        op = l.split()[0]
        if op == 's_waitcnt':
            m = re.search(r'vmcnt\((\d+)\)', l)
            if m:
                del q[:max(0, len(q) - int(m.group(1)))]
            return [(i + 1, q)]
        if op == 's_barrier':
            return [(i + 1, [min(e + 1, 3) if e else 0 for e in q])]
        if op == 's_endpgm':
            return []
        if op == 's_branch':
            return [(labels[l.split()[1]], q)]
        if op.startswith('s_cbranch'):
            return [(i + 1, q), (labels[l.split()[1]], q)]
        if op.startswith(('global_load_lds', 'buffer_load_lds')):
            return [(i + 1, (q + [1])[-_MAXQ:])]
        if op.startswith(('global_load', 'buffer_load', 'scratch_load', 'flat_load', 'global_store',
                          'buffer_store', 'scratch_store', 'flat_store', 'global_atomic')):
            return [(i + 1, (q + [0])[-_MAXQ:])]
        if op.startswith('ds_read'):
            aged = sum(1 for e in q if e >= 2)
            stale = sum(1 for e in q if e >= 3)
            if stale:
                bad[i] = (f'{stale} copies two or more barriers old in flight', l)
            elif aged > per_stage:
                bad[i] = (f'{aged} copies from before the barrier in flight (at most {per_stage})', l)
        return [(i + 1, q)]

    def merge(a: tuple, b: tuple) -> tuple:
        n = max(len(a), len(b))
        a = (0,) * (n - len(a)) + a
        b = (0,) * (n - len(b)) + b
        return tuple(max(x, y) for x, y in zip(a, b))

    state = {0: ()}
    work = [0]
    while work:
        i = work.pop()
        if i >= len(code):
            continue
        for j, q in run(i, state[i]):
            q = tuple(q)
            old = state.get(j)
            new = q if old is None else merge(old, q)
            if new != old:
                state[j] = new
                work.append(j)
    return [(i, *bad[i]) for i in sorted(bad)]


def check_lds_ring(hipcc: str, flags: list[str], src: Path, kernel: str, per_stage: int, out: Path) -> None:
    """Compile src to gfx9 assembly and raise if kernel reads LDS while more
    than per_stage of its pre-barrier global-to-LDS copies may be in flight."""
    cmd = [hipcc, *flags, '--cuda-device-only', '-S', str(src), '-o', str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc -S failed for {src.name}:\n{r.stderr[-4000:]}')
    asm = out.read_text()
    found = 0
    for name in sorted(set(re.findall(r'^(_Z\S*' + re.escape(kernel) + r'\S*):', asm, re.M))):
        found += 1
        bad = lds_ring_violations(kernel_lines(asm, name), per_stage)
        if bad:
            shown = '\n'.join(f'  {i}: {why}: {ins}' for i, why, ins in bad[:10])
            raise RuntimeError(f'{name} ({src.name}) reads LDS whose copies may still be in flight:\n{shown}')
    if not found:
        raise RuntimeError(f'{kernel} not found in {src.name}')


def check_source(hipcc: str, flags: list[str], src: Path, kernel: str, out: Path) -> None:
    """Compile src to gfx9 assembly and raise if kernel touches a register
    whose load may still be in flight."""
    cmd = [hipcc, *flags, '--cuda-device-only', '-S', str(src), '-o', str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f'hipcc -S failed for {src.name}:\n{r.stderr[-4000:]}')
    bad = pending_violations(kernel_lines(out.read_text(), kernel))
    if bad:
        shown = '\n'.join(f'  {i}: {why}: {ins}' for i, why, ins in bad[:10])
        raise RuntimeError(f'{kernel} ({src.name}) touches registers whose loads may still be in flight:\n{shown}')
