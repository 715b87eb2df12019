"""localai_hip_moe_forward_static -- the MoE layer with the library's static
device workspace (allocates nothing) -- against localai_hip_moe_forward with
a caller workspace, through the C ABI: the same kernels on the same inputs,
so routing, gates and outputs must be identical bit for bit, on two calls in
a row of which the second has fewer tokens (the static array keeps the first
call's contents). Sizes whose workspace exceeds the static one are EARG."""
import ctypes

import numpy as np
import pytest

from oracle import moe as omoe
from tests.conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _layer(seed, E, H, I, k, t):
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(seed)
    rw = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    gu = synth.quant_tensor(rng, t, 2 * I, H, batch=E)
    dn = synth.quant_tensor(rng, t, H, I, batch=E)
    return MoELayer(rw, gu, dn, t, E, H, I, k), (rw, gu, dn), rng


def _outputs(layer, T, dev):
    from localai_amd import device
    tt = device.torch()
    return (tt.empty((T, layer.H), dtype=tt.float32, device=dev), tt.empty((T, layer.k), dtype=tt.int32, device=dev),
            tt.empty((T, layer.k), dtype=tt.float32, device=dev))


def _static_status(layer, hd, outs, stream_ptr=None):
    from localai_amd import _lib, device
    p = device.ptr
    out, idx, gates = outs
    return _lib.load().localai_hip_moe_forward_static(
        p(hd), hd.shape[0], layer.H, p(layer.router_w), None, layer.E, layer.k, layer.gate_up.handle,
        layer.down.handle, p(out), p(idx), p(gates),
        ctypes.c_void_p(device.stream_ptr() if stream_ptr is None else stream_ptr))


def _static(layer, hd):
    from localai_amd import _lib
    outs = _outputs(layer, hd.shape[0], hd.device)
    _lib.check(_static_status(layer, hd, outs))
    return outs


@pytest.mark.parametrize('case', ['zaya_decode', 'q8_0_decode', 'qwen3_prefill'])
def test_static_workspace_matches_caller_workspace(case):
    from localai_amd import device, synth
    if case == 'zaya_decode':   # hidden 2048, 16 Q6_K experts, top-2, intermediate 4096: 8 tokens, then 1
        layer, (rw, gu, dn), rng = _layer(71, 16, 2048, 4096, 2, 14)
        sizes = (8, 1)
    elif case == 'q8_0_decode':   # 8 Q8_0 experts on the tile form (no row planes): 4 tokens, then 1
        layer, (rw, gu, dn), rng = _layer(73, 8, 1024, 512, 2, 8)
        sizes = (4, 1)
    else:                       # 64 Q4_K experts, top-8, intermediate 768: 96 tokens (GEMM path), then 8
        layer, (rw, gu, dn), rng = _layer(72, 64, 2048, 768, 8, 12)
        sizes = (96, 8)
    for T in sizes:
        h = synth.activations(rng, T, layer.H)
        hd = device.to_device_f32(h)
        so, si, sg = (a.cpu().numpy() for a in _static(layer, hd))
        wo, wi, wg = (a.cpu().numpy() for a in layer.forward_device(hd))
        np.testing.assert_array_equal(si, wi)
        np.testing.assert_array_equal(sg.view(np.uint32), wg.view(np.uint32))
        np.testing.assert_array_equal(so.view(np.uint32), wo.view(np.uint32))
        if T <= 8:
            t = {'zaya_decode': 14, 'q8_0_decode': 8}.get(case, 12)
            ref, ridx, _, _ = omoe.moe_forward(h, rw, gu, dn, t, layer.E, layer.k, layer.I)
            np.testing.assert_array_equal(si, ridx)
            assert normwise_rel(so, ref) < 1e-5


def test_static_refuses_paths_that_would_build_row_planes():
    """Q8_0 experts whose rows are not whole 256-value blocks (inter 320)
    below 32 tokens run the grouped kernels over the row planes, which a
    Q8_0 handle builds on first use (an allocation): the static entry
    refuses with LOCALAI_ETYPE before any launch, and the free device memory
    does not move. Once the ordinary entry has built the planes, the static
    entry takes that path, allocates nothing and matches it bit for bit (two
    calls, the second smaller)."""
    from localai_amd import _lib, device, synth
    lib = _lib.load()
    tt = device.torch()
    layer, (rw, gu, dn), rng = _layer(74, 8, 1024, 320, 2, 8)
    hd = device.to_device_f32(synth.activations(rng, 4, layer.H))
    outs = _outputs(layer, 4, hd.device)
    tt.cuda.synchronize()
    free0 = tt.cuda.mem_get_info()[0]
    st = _static_status(layer, hd, outs)
    tt.cuda.synchronize()
    assert st == 2, lib.localai_hip_last_error()
    assert b'allocates nothing' in lib.localai_hip_last_error()
    assert tt.cuda.mem_get_info()[0] == free0
    layer.forward_device(hd)           # the ordinary entry builds the planes
    for T in (4, 2):
        hT = synth.activations(rng, T, layer.H)
        hdT = device.to_device_f32(hT)
        wo, wi, wg = (a.cpu().numpy() for a in layer.forward_device(hdT))
        outs = _outputs(layer, T, hdT.device)
        tt.cuda.synchronize()
        free1 = tt.cuda.mem_get_info()[0]
        _lib.check(_static_status(layer, hdT, outs))
        tt.cuda.synchronize()
        assert tt.cuda.mem_get_info()[0] == free1
        so, si, sg = (a.cpu().numpy() for a in outs)
        np.testing.assert_array_equal(si, wi)
        np.testing.assert_array_equal(sg.view(np.uint32), wg.view(np.uint32))
        np.testing.assert_array_equal(so.view(np.uint32), wo.view(np.uint32))
        ref, ridx, _, _ = omoe.moe_forward(hT, rw, gu, dn, 8, layer.E, layer.k, layer.I)
        np.testing.assert_array_equal(si, ridx)
        assert normwise_rel(so, ref) < 1e-5


def test_static_under_graph_capture():
    """The static entry captured in a HIP graph (Q6_K experts, one token and
    eight tokens): every replay, with other static calls and synchronisation
    between the replays, equals the eager call."""
    from localai_amd import _lib, device, synth
    tt = device.torch()
    layer, _, rng = _layer(75, 16, 2048, 4096, 2, 14)
    for T in (1, 8):
        hd = device.to_device_f32(synth.activations(rng, T, layer.H))
        eo, ei, eg = (a.cpu().numpy() for a in _static(layer, hd))
        outs = _outputs(layer, T, hd.device)
        s = tt.cuda.Stream()
        g = tt.cuda.CUDAGraph()
        tt.cuda.synchronize()
        with tt.cuda.graph(g, stream=s):
            st = _static_status(layer, hd, outs, int(s.cuda_stream))
        _lib.check(st)
        out, idx, gates = outs
        for _ in range(3):
            out.fill_(float('nan'))
            idx.fill_(-1)
            tt.cuda.synchronize()
            g.replay()
            tt.cuda.synchronize()
            np.testing.assert_array_equal(idx.cpu().numpy(), ei)
            np.testing.assert_array_equal(gates.cpu().numpy().view(np.uint32), eg.view(np.uint32))
            np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), eo.view(np.uint32))
            _static(layer, device.to_device_f32(synth.activations(rng, 3, layer.H)))   # other work on the array
            tt.cuda.synchronize()


def test_static_workspace_size_limit():
    from localai_amd import _lib, device
    lib = _lib.load()
    cap = int(lib.localai_hip_static_workspace_bytes())
    assert cap == 64 << 20
    layer, _, _ = _layer(73, 128, 2048, 768, 8, 12)
    T = 4096
    assert int(lib.localai_hip_moe_workspace_size(T, 128, 8, 2048, 768)) > cap
    tt = device.torch()
    hd = tt.zeros((T, 2048), dtype=tt.float32, device=device.device())
    out = tt.empty((T, 2048), dtype=tt.float32, device=hd.device)
    idx = tt.empty((T, 8), dtype=tt.int32, device=hd.device)
    gates = tt.empty((T, 8), dtype=tt.float32, device=hd.device)
    p = device.ptr
    st = lib.localai_hip_moe_forward_static(p(hd), T, 2048, p(layer.router_w), None, 128, 8, layer.gate_up.handle,
                                            layer.down.handle, p(out), p(idx), p(gates), None)
    assert st == 1
    assert b'static' in lib.localai_hip_last_error()
