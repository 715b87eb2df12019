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


def ring(body, per_stage=2):
    return isa_check.lds_ring_violations(isa_check.kernel_lines(listing(body), 'kernel'), per_stage)


# a two-ahead ring of LDS stages with two copies per stage, shaped like
# moe_route_logits_kernel: chunks 0 and 1 requested up front; per pass of the
# loop: wait, barrier, request chunk j + 2, read chunk j; then chunk n - 2
# (nothing more to request) and the last chunk after a wait for every copy
RING = '''
        global_load_lds_dwordx4 v[2:3], off
        global_load_lds_dwordx4 v[4:5], off
        global_load_lds_dwordx4 v[2:3], off
        global_load_lds_dwordx4 v[4:5], off
.LBB0_1:
        s_waitcnt vmcnt({loop})
        s_barrier
        global_load_lds_dwordx4 v[2:3], off
        global_load_lds_dwordx4 v[4:5], off
        ds_read_b128 v[8:11], v1
        s_cbranch_scc1 .LBB0_1
        s_waitcnt vmcnt({peel})
        s_barrier
        ds_read_b128 v[8:11], v1
        s_waitcnt vmcnt({last})
        s_barrier
        ds_read_b128 v[8:11], v1
        s_endpgm'''


def test_lds_ring_correct_waits_pass():
    assert ring(RING.format(loop=2, peel=2, last=0)) == []


def test_lds_ring_wait_too_lax_is_found():
    bad = ring(RING.format(loop=3, peel=2, last=0))
    assert [b[0] for b in bad] == [9]      # a copy of chunk j may not have landed


def test_lds_ring_missing_last_wait_is_found():
    # without the final vmcnt(0) the last chunk's copies (two barriers old
    # by its read) may still be in flight
    bad = ring(RING.format(loop=2, peel=2, last=2))
    assert [b[0] for b in bad] == [16]
    assert 'two or more barriers old' in bad[0][1]


def test_lds_ring_plain_load_in_the_queue():
    # a plain load issued after the prologue's copies is one more entry the
    # loop's first wait must let go of: vmcnt(2) still leaves only chunk 1
    # in flight, vmcnt(3) would leave a copy of chunk 0
    body = RING.replace('        global_load_lds_dwordx4 v[4:5], off\n.LBB0_1:',
                        '        global_load_lds_dwordx4 v[4:5], off\n        global_load_dword v20, v11, s[0:1]\n.LBB0_1:')
    assert ring(body.format(loop=2, peel=2, last=0)) == []
    assert ring(body.format(loop=3, peel=2, last=0)) != []


@pytest.mark.skipif(shutil.which('hipcc') is None and not __import__('os').path.exists('/opt/rocm/bin/hipcc'),
                    reason='hipcc not installed')
def test_counted_load_kernels_are_clean(tmp_path):
    from localai_amd import build
    for src, kernel, per_stage in build.COUNTED_LOADS:
        if per_stage is None:
            isa_check.check_source(build.HIPCC, build.COMMON, build.CSRC / src, kernel, tmp_path / 'k.s')
        else:
            isa_check.check_lds_ring(build.HIPCC, build.COMMON, build.CSRC / src, kernel, per_stage, tmp_path / 'k.s')
