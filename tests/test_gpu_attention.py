"""GPU decode attention (localai_hip_attention_decode) and delta-net step
(localai_hip_delta_net_step) against oracle/attention.py.

Attention: fp32 on the GPU against the fp64 oracle, normwise <= 2e-5 (the
scores carry a few fp32 roundings of a 64..256-term dot product, the softmax
and the weighted sum a few more; about 1e-6 typical). The cache row of the
token must hold k_new / v_new bit for bit and every other row must be
untouched. Delta net: the GPU runs the reference loop's float32 operations in
its order, so state and core must equal the float32 oracle bit for bit."""
import numpy as np
import pytest

from oracle import attention as oatt
from tests.conftest import normwise_rel

pytestmark = pytest.mark.gpu


def _run_attention(nh, nkv, hd, pos, max_seq, window=0, gate=False, new_row=True, seed=0):
    import torch
    from localai_amd import attention, device
    rng = np.random.default_rng(seed)
    kc = rng.standard_normal((max_seq, nkv, hd)).astype(np.float32)
    vc = rng.standard_normal((max_seq, nkv, hd)).astype(np.float32)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kn = rng.standard_normal(nkv * hd).astype(np.float32) if new_row else None
    vn = rng.standard_normal(nkv * hd).astype(np.float32) if new_row else None
    g = (rng.standard_normal(nh * hd) * 2).astype(np.float32) if gate else None
    cache = attention.KVCache(1, nkv, hd, max_seq, n_heads=nh)
    cache.k[0].copy_(torch.from_numpy(kc))
    cache.v[0].copy_(torch.from_numpy(vc))
    dev = lambda a: device.to_device_f32(a) if a is not None else None
    out = attention.attention_decode(dev(q), dev(kn), dev(vn), cache, 0, pos, nh, window=window, gate=dev(g))
    torch.cuda.synchronize()
    want, kc2, vc2 = oatt.gqa_decode(q, kc, vc, pos, nh, nkv, hd, window=window, gate=g, k_new=kn, v_new=vn)
    got = out.cpu().numpy()
    err = normwise_rel(got, want)
    print(f'attention nh={nh} nkv={nkv} hd={hd} pos={pos} window={window} gate={gate}: normwise {err:.2e}')
    assert err <= 2e-5, err
    np.testing.assert_array_equal(cache.k[0].cpu().numpy(), kc2)
    np.testing.assert_array_equal(cache.v[0].cpu().numpy(), vc2)


@pytest.mark.parametrize('pos', [0, 1, 63, 64, 255, 256, 1000, 4095])
def test_llama3_8b_heads(pos):
    _run_attention(32, 8, 128, pos, 4096, seed=pos)


@pytest.mark.parametrize('nh,nkv,hd,pos', [
    (8, 8, 64, 100),        # multi-head (one query head per kv head)
    (64, 8, 128, 777),      # 8 query heads per kv head
    (28, 4, 128, 500),      # 7 per kv head (kernel sized for 8)
    (16, 4, 256, 300),      # head_dim 256
    (6, 2, 64, 129),        # 3 per kv head
    (4, 4, 256, 2047),      # head_dim 256, one per kv head
])
def test_head_shapes(nh, nkv, hd, pos):
    _run_attention(nh, nkv, hd, pos, 2048, seed=nh + pos)


@pytest.mark.parametrize('window,pos', [(128, 1000), (1, 700), (64, 63), (5000, 1000)])
def test_sliding_window(window, pos):
    _run_attention(32, 8, 128, pos, 2048, window=window, seed=window)


def test_output_gate_and_row_already_in_cache():
    _run_attention(16, 4, 256, 400, 1024, gate=True, seed=3)
    _run_attention(32, 8, 128, 900, 1024, new_row=False, seed=4)


def test_unsupported_head_dim_is_refused():
    import torch
    from localai_amd import _lib, attention, device
    cache = attention.KVCache(1, 2, 96, 16, n_heads=4)
    q = torch.zeros(4 * 96, dtype=torch.float32, device=device.device())
    with pytest.raises(_lib.HipError) as e:
        attention.attention_decode(q, None, None, cache, 0, 3, 4)
    assert 'head_dim' in str(e.value)


def _delta_inputs(rng, heads, kd, vd):
    state = rng.standard_normal((heads, kd, vd)).astype(np.float32)
    q = rng.standard_normal((heads, kd)).astype(np.float32)
    k = rng.standard_normal((heads, kd)).astype(np.float32)
    q /= np.maximum(np.linalg.norm(q, axis=1, keepdims=True), 1e-6) * np.sqrt(kd)
    k /= np.maximum(np.linalg.norm(k, axis=1, keepdims=True), 1e-6)
    v = rng.standard_normal((heads, vd)).astype(np.float32)
    decay = -rng.uniform(0.001, 3.0, heads).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, heads).astype(np.float32)
    return state, q, k, v, decay, beta


@pytest.mark.parametrize('heads,kd,vd', [(32, 128, 128), (3, 64, 96), (2, 200, 70), (5, 1, 1), (1, 128, 65)])
def test_delta_net_bit_exact(heads, kd, vd):
    import torch
    from localai_amd import attention, device
    rng = np.random.default_rng(heads * 1000 + kd + vd)
    state, *rest = _delta_inputs(rng, heads, kd, vd)
    st = device.to_device_f32(state)
    S = state
    for step in range(3):       # the state carries from step to step
        q, k, v, decay, beta = rest if step == 0 else _delta_inputs(rng, heads, kd, vd)[1:]
        core = attention.delta_net_step(st, *(device.to_device_f32(a) for a in (q, k, v, decay, beta)))
        torch.cuda.synchronize()
        S, want = oatt.delta_net_step(S, q, k, v, decay, beta)
        print(f'delta net {heads}x{kd}x{vd} step {step}')
        np.testing.assert_array_equal(core.cpu().numpy(), want)
        np.testing.assert_array_equal(st.cpu().numpy(), S)


def test_delta_net_against_numpy_float32_exponential():
    """The reference evaluates np.exp on float32 decay (engine/numba_kernels.py:25,
    engine/qwen35.py:242), which need not be correctly rounded; the kernel
    takes the correctly rounded exponential. Against the oracle with NumPy's
    float32 factor the kernel holds state and core within an ulp-level
    normwise bound. NumPy's float32 exponential differs from the correctly
    rounded one in the last bit or two for a good part of its inputs (about
    40 % of U(-3, 0) on an AVX-512 host), so only the state's recurrence, not
    the factor, can be bit-exact with the reference."""
    import torch
    from localai_amd import attention, device
    rng = np.random.default_rng(77)
    heads, kd, vd = 32, 128, 128
    state, q, k, v, decay, beta = _delta_inputs(rng, heads, kd, vd)
    f_np = np.exp(decay.astype(np.float32))
    f_rn = np.exp(decay.astype(np.float64)).astype(np.float32)
    assert np.max(np.abs(f_np.view(np.int32).astype(np.int64) - f_rn.view(np.int32))) <= 4
    st = device.to_device_f32(state)
    core = attention.delta_net_step(st, *(device.to_device_f32(a) for a in (q, k, v, decay, beta)))
    torch.cuda.synchronize()
    S, want = oatt.delta_net_step(state, q, k, v, decay, beta, factor_exp='numpy_f32')
    assert normwise_rel(core.cpu().numpy(), want) < 1e-6
    assert normwise_rel(st.cpu().numpy(), S) < 1e-6
