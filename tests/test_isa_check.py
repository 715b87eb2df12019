"""The build-time check for kernels that count their own global loads
(localai_amd/isa_check.py): planted hazards in small assembly listings must be
found, correct waits must pass, and the GEMM kernel that relies on it must be
clean in a fresh compile."""
import shutil

import pytest

from localai_amd import isa_check


def listing(body):
    return '\n'.join(['_Z6kernelv:', *body.strip().split('\n'), '.Lfunc_end0:'])


def violations(body):
    return isa_check.pending_violations(isa_check.kernel_lines(listing(body), 'kernel'))


def test_use_before_wait_is_found():
    bad = violations('''
        global_load_dwordx4 v[0:3], v10, s[0:1]
        v_add_f32 v4, v0, v5
        s_endpgm''')
    assert [b[0] for b in bad] == [1]


def test_wait_for_zero_clears():
    assert violations('''
        global_load_dwordx4 v[0:3], v10, s[0:1]
        s_waitcnt vmcnt(0)
        v_add_f32 v4, v0, v5
        s_endpgm''') == []


def test_loads_complete_in_order():
    # vmcnt(1): the older load is done, the newer one may not be
    body = '''
        global_load_dwordx4 v[0:3], v10, s[0:1]
        global_load_dword v8, v11, s[0:1]
        s_waitcnt vmcnt(1)
        v_add_f32 v4, v0, v5
        {}
        s_endpgm'''
    assert violations(body.format('')) == []
    assert len(violations(body.format('v_mov_b32 v20, v8'))) == 1


def test_overwrite_and_address_reuse_are_found():
    bad = violations('''
        global_load_dword v8, v11, s[0:1]
        v_mov_b32 v8, 0
        global_load_dword v9, v8, s[0:1]
        s_endpgm''')
    assert [b[0] for b in bad] == [1, 2]


def test_join_keeps_the_pessimistic_state():
    bad = violations('''
        global_load_dword v8, v11, s[0:1]
        s_cbranch_scc0 .LBB0_2
        s_waitcnt vmcnt(0)
.LBB0_2:
        v_mov_b32 v20, v8
        s_endpgm''')
    assert len(bad) == 1 and 'v_mov_b32' in bad[0][2]


def test_loop_carried_load_with_too_lax_wait():
    # the load at the end of the body is used at the top of the next pass:
    # vmcnt(1) leaves it in flight because the second load is newer
    body = '''
.LBB0_1:
        s_waitcnt vmcnt({})
        v_add_f32 v4, v0, v5
        global_load_dword v0, v10, s[0:1]
        global_load_dword v1, v11, s[0:1]
        s_cbranch_scc1 .LBB0_1
        s_endpgm'''
    assert violations(body.format(2)) != []
    assert violations(body.format(1)) == []


def test_lds_dma_writes_no_register():
    assert violations('''
        global_load_lds_dwordx4 v[2:3], off
        v_mov_b32 v2, 0
        s_endpgm''') == []


@pytest.mark.skipif(shutil.which('hipcc') is None and not __import__('os').path.exists('/opt/rocm/bin/hipcc'),
                    reason='hipcc not installed')
def test_counted_load_kernels_are_clean(tmp_path):
    from localai_amd import build
    for src, kernel in build.COUNTED_LOADS:
        isa_check.check_source(build.HIPCC, build.COMMON, build.CSRC / src, kernel, tmp_path / 'k.s')
