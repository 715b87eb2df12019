"""ZAYA MoE block on the GPU (localai_amd.zaya.ZayaMoEMixin) against the CPU
restatement of engine/zaya.py:274-307 (oracle/zaya_moe.py) on a synthetic
GGUF layer: router MLP (Q8_0 first projection with a bias, F16 / F32 small
matrices, EDA), Q6_K experts, the skip route and forced experts, through our
GGUFFile and through a plain reader with only `.tensors` and `._map`.

Q6_K experts run as the one-launch expert kernel (device-side index and skip
route, localai_hip_moe_experts1); Q8_0 experts take the matvec path with the
index read on the host; both are checked.

Tolerances: router state normwise <= 5e-6 (its Q8_0 first projection runs on
i8 MFMA with x in three int8 pieces, about 1e-6; the rest are fp32 sums);
probabilities within 2e-6 absolute; the expert index equal wherever the
oracle's best two routes are more than 1e-4 apart (np.exp's own rounding is
not restated); block output normwise <= 1e-5 (i8 MFMA expert matvecs).
"""
import numpy as np
import pytest

from oracle import quant
from oracle import zaya_moe as zm
from tests.conftest import normwise_rel
from tests.gguf_writer import build
from tests.gpu_util import random_ggml

pytestmark = pytest.mark.gpu

E, H, I, R = 16, 1024, 512, 256
EPS = 1e-5


def layer_tensors(rng, route_bias, xt=14):
    f32 = lambda a: np.asarray(a, np.float32)   # noqa: E731
    raw = {
        'ffn_gate_inp.weight': ((R, H), 8, random_ggml(rng, 8, R * H, 2e-4, 6e-4)),
        'ffn_gate_inp.bias': ((R,), 0, f32(rng.standard_normal(R) * 0.1).tobytes()),
        'zaya_router_eda.weight': ((R,), 0, f32(rng.uniform(-0.5, 0.5, R)).tobytes()),
        'ffn_norm.weight': ((R,), 0, f32(rng.uniform(0.5, 1.5, R)).tobytes()),
        'ffn_gate.weight': ((R, R), 1, (rng.standard_normal((R, R)) / 16).astype(np.float16).tobytes()),
        'ffn_gate.bias': ((R,), 0, f32(rng.standard_normal(R) * 0.1).tobytes()),
        'zaya_router_mlp2.weight': ((R, R), 0, f32(rng.standard_normal((R, R)) / 16).tobytes()),
        'zaya_router_mlp4.weight': ((E + 1, R), 0, f32(rng.standard_normal((E + 1, R)) / 4).tobytes()),
        'zaya_router_biases.weight': ((E + 1,), 0, f32(route_bias).tobytes()),
        'ffn_gate_up_exps.weight': ((E, 2 * I, H), xt, random_ggml(rng, xt, E * 2 * I * H, 1e-4, 2e-3)),
        'ffn_down_exps.weight': ((E, H, I), xt, random_ggml(rng, xt, E * H * I, 1e-4, 2e-3)),
    }
    return raw


def write_layer(path, raw):
    tensors = [(f'blk.1.{n}', shape, t, b) for n, (shape, t, b) in raw.items()]
    path.write_bytes(build(tensors, metadata=[('general.architecture', 8, 'zaya')], alignment=32))


def oracle_tensors(raw):
    d = {n: quant.dequantize(b, t, shape) for n, (shape, t, b) in raw.items()}
    return {'inp': d['ffn_gate_inp.weight'], 'inp_b': d['ffn_gate_inp.bias'], 'eda': d['zaya_router_eda.weight'],
            'norm': d['ffn_norm.weight'], 'gate': d['ffn_gate.weight'], 'gate_b': d['ffn_gate.bias'],
            'mlp2': d['zaya_router_mlp2.weight'], 'mlp2_b': None, 'mlp4': d['zaya_router_mlp4.weight'],
            'mlp4_b': None, 'route_bias': d['zaya_router_biases.weight'], 'gate_up': d['ffn_gate_up_exps.weight'],
            'down': d['ffn_down_exps.weight']}


class Model:
    n_experts = E
    eps = EPS

    def __init__(self, gguf):
        self.gguf = gguf


def model_class():
    from localai_amd.zaya import ZayaMoEMixin
    return type('ZayaGPU', (ZayaMoEMixin, Model), {})


class PlainReader:
    """Only what the reference's GGUFFile offers the model: tensors and _map."""

    def __init__(self, g):
        self.tensors, self._map = g.tensors, g._map


@pytest.fixture(scope='module')
def base(tmp_path_factory):
    rng = np.random.default_rng(21)
    raw = layer_tensors(rng, rng.uniform(0.0, 0.05, E + 1) * np.r_[np.ones(E), 0.0])
    path = tmp_path_factory.mktemp('zaya') / 'layer.gguf'
    write_layer(path, raw)
    return path, oracle_tensors(raw)


@pytest.mark.parametrize('reader', ['gguf', 'plain'])
def test_block_matches_oracle(base, reader):
    from localai_amd.gguf import GGUFFile
    path, t = base
    rng = np.random.default_rng(5)
    matched = 0
    with GGUFFile(path) as g:
        m = model_class()(g if reader == 'gguf' else PlainReader(g))
        prev = None
        for step in range(6):
            h = rng.standard_normal(H).astype(np.float32)
            moe, state = m._moe(1, h, prev)
            w_moe, w_state, w_probs, w_e, margin = zm.moe_block(t, E, EPS, h, prev)
            assert normwise_rel(state, w_state) < 5e-6
            if margin > 1e-4:
                assert normwise_rel(moe, w_moe) < 1e-5, step
                matched += 1
            prev = state
    assert matched >= 3


def test_router_probabilities_and_expert(base):
    """Read the router's outputs directly (probs and the index) through the C ABI."""
    import ctypes
    from localai_amd import _lib, device
    from localai_amd.gguf import GGUFFile
    path, t = base
    rng = np.random.default_rng(8)
    tt = device.torch()
    with GGUFFile(path) as g:
        m = model_class()(g)
        L = m._zaya_layer(1)
        for _ in range(4):
            h = rng.standard_normal(H).astype(np.float32)
            prev = rng.standard_normal(R).astype(np.float32)
            _, w_state, w_probs, w_e, margin = zm.moe_block(t, E, EPS, h, prev)
            r0 = m._zaya_matrix(L.inp).matvec(device.to_device_f32(h)).reshape(-1)
            pd = device.to_device_f32(prev)
            state = tt.empty(R, dtype=tt.float32, device=r0.device)
            probs = tt.empty(E + 1, dtype=tt.float32, device=r0.device)
            ex = tt.empty(1, dtype=tt.int32, device=r0.device)
            ew = tt.empty(1, dtype=tt.float32, device=r0.device)
            p = device.ptr
            _lib.check(_lib.load().localai_hip_zaya_router(
                p(r0), p(L.b_inp), p(pd), p(L.eda), p(L.norm), ctypes.c_float(EPS), R, p(L.w1), p(L.b1), R,
                p(L.w2), None, R, p(L.w3), None, E + 1, p(L.route_bias), p(state), p(probs), p(ex), p(ew), None))
            np.testing.assert_allclose(probs.cpu().numpy(), w_probs, rtol=0, atol=2e-6)
            # the chosen route's weight: bit for bit probs[expert]
            assert ew.cpu().numpy().view(np.uint32)[0] == probs.cpu().numpy().view(np.uint32)[int(ex.cpu().item())]
            assert normwise_rel(state.cpu().numpy(), w_state) < 5e-6
            if margin > 1e-4:
                assert int(ex.cpu().item()) == w_e


@pytest.mark.parametrize('xt', [14, 12])
@pytest.mark.parametrize('forced', [E, 5])
def test_skip_route_and_forced_expert(tmp_path, forced, xt):
    """Q6_K and Q4_K experts: the block must take the one-launch expert kernel
    (the skip route instantiation included) and match the oracle."""
    from localai_amd.gguf import GGUFFile
    rng = np.random.default_rng(30 + forced + xt)
    bias = np.zeros(E + 1)
    bias[forced] = 10.0
    raw = layer_tensors(rng, bias, xt=xt)
    path = tmp_path / 'forced.gguf'
    write_layer(path, raw)
    t = oracle_tensors(raw)
    h = rng.standard_normal(H).astype(np.float32)
    with GGUFFile(path) as g:
        m = model_class()(g)
        moe, state = m._moe(1, h, None)
        assert m._zaya_cache().get(('experts1', 'blk.1.')) is not False
    w_moe, w_state, w_probs, w_e, _ = zm.moe_block(t, E, EPS, h, None)
    assert w_e == forced
    assert normwise_rel(state, w_state) < 5e-6
    assert normwise_rel(moe, w_moe) < (5e-6 if forced == E else 1e-5)


@pytest.mark.parametrize('xt', [8, 13])
@pytest.mark.parametrize('forced', [E, 3])
def test_q8_0_and_matvec_path_experts(tmp_path, forced, xt):
    """Q8_0 experts (tile form) take the one-launch kernel like Q4_K / Q6_K;
    Q5_K experts have none: the block reads the index on the host and runs
    the matvecs. The skip route and an expert both checked."""
    from localai_amd.gguf import GGUFFile
    rng = np.random.default_rng(40 + forced + xt)
    bias = np.zeros(E + 1)
    bias[forced] = 10.0
    raw = layer_tensors(rng, bias, xt=xt)
    path = tmp_path / f'x{xt}.gguf'
    write_layer(path, raw)
    t = oracle_tensors(raw)
    h = rng.standard_normal(H).astype(np.float32)
    with GGUFFile(path) as g:
        m = model_class()(g)
        moe, state = m._moe(1, h, None)
        assert (m._zaya_cache().get(('experts1', 'blk.1.')) is False) == (xt == 13)
    w_moe, w_state, _, w_e, _ = zm.moe_block(t, E, EPS, h, None)
    assert w_e == forced
    assert normwise_rel(state, w_state) < 5e-6
    assert normwise_rel(moe, w_moe) < (5e-6 if forced == E else 1e-5)


@pytest.fixture(scope='module')
def base_q4k(tmp_path_factory):
    rng = np.random.default_rng(22)
    raw = layer_tensors(rng, rng.uniform(0.0, 0.05, E + 1) * np.r_[np.ones(E), 0.0], xt=12)
    path = tmp_path_factory.mktemp('zaya_q4k') / 'layer.gguf'
    write_layer(path, raw)
    return path, oracle_tensors(raw)


@pytest.mark.parametrize('which', ['q6k', 'q4k'])
def test_experts1_two_slots_with_skip(base, base_q4k, which):
    """localai_hip_moe_experts1 with top_k 2, one slot an expert and one the
    skip route: out = w0 * expert(h) + w1 * h, against the oracle's products;
    Q6_K and Q4_K experts."""
    from localai_amd import _lib, device
    from localai_amd.gguf import GGUFFile
    path, t = base if which == 'q6k' else base_q4k
    rng = np.random.default_rng(9)
    tt = device.torch()
    lib = _lib.load()
    with GGUFFile(path) as g:
        gu = g.device_matrix('blk.1.ffn_gate_up_exps.weight')
        dn = g.device_matrix('blk.1.ffn_down_exps.weight')
        for e0, w in ((7, (0.625, 0.375)), (0, (0.9, 0.1))):
            h = rng.standard_normal(H).astype(np.float32)
            hd = device.to_device_f32(h)
            idx = tt.tensor([e0, E], dtype=tt.int32, device=hd.device)
            wt = tt.tensor(w, dtype=tt.float32, device=hd.device)
            out = tt.empty(H, dtype=tt.float32, device=hd.device)
            n = int(lib.localai_hip_moe_workspace_size(1, E, 2, H, I))
            ws = tt.empty(n, dtype=tt.uint8, device=hd.device)
            p = device.ptr
            _lib.check(lib.localai_hip_moe_experts1(p(hd), H, gu.handle, dn.handle, 2, p(idx), p(wt), E, p(out),
                                                    p(ws), n, None))
            gate, up = np.split(zm.mat(t['gate_up'][e0], h), 2)
            y = zm.mat(t['down'][e0], gate / (1.0 + np.exp(-np.clip(gate, -80, 80))) * up)
            want = np.float32(w[0]) * y + np.float32(w[1]) * h
            assert normwise_rel(out.cpu().numpy(), want) < 1e-5
            _lib.check(lib.localai_hip_moe_error(p(ws), 1, E, None))


def test_experts1_checks_indices_and_skip(base):
    """A skip value inside [0, E) is an argument error at the call; an expert
    index outside [0, E) that is not the skip route makes its rows NaN and is
    reported by localai_hip_moe_error (EARG), while a valid call after it on
    the same workspace reports nothing."""
    from localai_amd import _lib, device
    from localai_amd.gguf import GGUFFile
    path, t = base
    tt = device.torch()
    lib = _lib.load()
    p = device.ptr
    with GGUFFile(path) as g:
        gu = g.device_matrix('blk.1.ffn_gate_up_exps.weight')
        dn = g.device_matrix('blk.1.ffn_down_exps.weight')
        hd = device.to_device_f32(np.random.default_rng(3).standard_normal(H).astype(np.float32))
        out = tt.empty(H, dtype=tt.float32, device=hd.device)
        n = int(lib.localai_hip_moe_workspace_size(1, E, 2, H, I))
        ws = tt.empty(n, dtype=tt.uint8, device=hd.device)
        wt = tt.tensor([0.5, 0.5], dtype=tt.float32, device=hd.device)
        idx = tt.tensor([2, E], dtype=tt.int32, device=hd.device)
        assert lib.localai_hip_moe_experts1(p(hd), H, gu.handle, dn.handle, 2, p(idx), p(wt), 3, p(out),
                                            p(ws), n, None) == 1
        bad = tt.tensor([2, E + 3], dtype=tt.int32, device=hd.device)
        _lib.check(lib.localai_hip_moe_experts1(p(hd), H, gu.handle, dn.handle, 2, p(bad), p(wt), -1, p(out),
                                                p(ws), n, None))
        assert lib.localai_hip_moe_error(p(ws), 1, E, None) == 1
        assert tt.isnan(out).all()
        _lib.check(lib.localai_hip_moe_experts1(p(hd), H, gu.handle, dn.handle, 2, p(idx), p(wt), E, p(out),
                                                p(ws), n, None))
        _lib.check(lib.localai_hip_moe_error(p(ws), 1, E, None))
        assert tt.isfinite(out).all()
