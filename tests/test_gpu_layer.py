"""GPU decode-layer matvec chain (localai_hip_layer_chain) against the oracle
of engine/model.py:229-233 + :181-210 (oracle/layer.py).

Tolerance: every matvec is the i8-MFMA decode matvec (about 1e-6 normwise of
its output). The chain multiplies two of them (silu(gate) * up), and a
product's normwise error grows by max|g| max|u| / max|g u| over its factors'
(about 2e-5 on these random weights), which the down matvec and the norms
carry on. Each output is held to normwise 1e-4 against the fp64 oracle,
inside the path's 1e-3 target; a chain that dropped or misplaced a term
would be off by order one."""
import numpy as np
import pytest

from oracle import layer as olayer
from tests.conftest import normwise_rel

pytestmark = pytest.mark.gpu

LLAMA3_8B = {'attn_output': (12, 4096, 4096), 'ffn_gate': (12, 14336, 4096), 'ffn_up': (12, 14336, 4096),
             'ffn_down': (14, 4096, 14336), 'attn_q': (12, 4096, 4096), 'attn_k': (12, 1024, 4096),
             'attn_v': (14, 1024, 4096)}


def build(shapes, seed):
    from localai_amd import device, synth
    from localai_amd.layer import DecodeLayerChain
    rng = np.random.default_rng(seed)
    dim = shapes['attn_output'][1]
    raws = {n: (synth.quant_tensor(rng, t, r, c), t, r, c) for n, (t, r, c) in shapes.items()}
    w_ffn = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    w_attn = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    mats = {n: device.QMat.from_ggml(raw, t, r, c) for n, (raw, t, r, c) in raws.items()}
    chain = DecodeLayerChain(mats, w_ffn, w_attn, 1e-5, head_dim=128)
    return chain, raws, w_ffn, w_attn, rng


@pytest.fixture(params=[False, True], ids=['four_launches', 'one_launch'])
def mode(request):
    """Runs a test with the chain as four glued launches and as one launch."""
    from localai_amd import layer
    layer.set_mode(request.param)
    yield request.param
    layer.set_mode(False)


def check_outputs(got, want, tol=1e-4):
    names = ('x_out', 'q', 'k', 'v')
    for n, g, w in zip(names, got, want):
        err = normwise_rel(g.cpu().numpy(), w)
        assert err < tol, f'{n}: {err}'


@pytest.mark.parametrize('rope', [False, True])
def test_llama3_8b_chain_matches_oracle(rope, mode):
    from localai_amd import device, synth
    chain, raws, w_ffn, w_attn, rng = build(LLAMA3_8B, 5 + rope)
    pre, att = synth.activations(rng, 4096), synth.activations(rng, 4096)
    rp = None
    cos = sin = None
    if rope:
        inv = 1.0 / (500000.0 ** (np.arange(64, dtype=np.float32) / 64))
        ang = np.float32(37) * inv
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
        rp = (device.to_device_f32(cos), device.to_device_f32(sin))
    got = chain.forward_device(device.to_device_f32(pre), device.to_device_f32(att), rope=rp)
    chain.check()
    want, _ = olayer.chain(raws, pre, att, w_ffn, w_attn, 1e-5, rope=(cos, sin) if rope else None, head_dim=128)
    check_outputs(got, want)


@pytest.mark.parametrize('shapes', [
    # 2048 / 5632 (one super-block per wave, down halves of 11)
    {'attn_output': (14, 2048, 2048), 'ffn_gate': (14, 5632, 2048), 'ffn_up': (14, 5632, 2048),
     'ffn_down': (12, 2048, 5632), 'attn_q': (12, 2048, 2048), 'attn_k': (14, 256, 2048), 'attn_v': (12, 256, 2048)},
    # 4096 / 11008 (three super-blocks per wave in down, an odd count of ffn super-blocks)
    {'attn_output': (12, 4096, 4096), 'ffn_gate': (12, 11008, 4096), 'ffn_up': (12, 11008, 4096),
     'ffn_down': (14, 4096, 11008), 'attn_q': (12, 4096, 4096), 'attn_k': (12, 1024, 4096),
     'attn_v': (14, 1024, 4096)},
])
def test_other_shapes_and_types(shapes, mode):
    from localai_amd import device, synth
    chain, raws, w_ffn, w_attn, rng = build(shapes, 9)
    dim = shapes['attn_output'][1]
    pre, att = synth.activations(rng, dim), synth.activations(rng, dim)
    got = chain.forward_device(device.to_device_f32(pre), device.to_device_f32(att))
    chain.check()
    want, _ = olayer.chain(raws, pre, att, w_ffn, w_attn, 1e-5)
    check_outputs(got, want)


def test_repeated_launches_and_graph_replays_are_identical(mode):
    """The counters return to zero after each launch: 20 launches in a row and
    replays of a captured graph (with eager launches between them) give the
    same bits as the first launch."""
    import torch
    from localai_amd import device, synth
    chain, raws, w_ffn, w_attn, rng = build(LLAMA3_8B, 13)
    pre = device.to_device_f32(synth.activations(rng, 4096))
    att = device.to_device_f32(synth.activations(rng, 4096))
    first = [o.clone() for o in chain.forward_device(pre, att)]
    torch.cuda.synchronize()
    for _ in range(20):
        outs = chain.forward_device(pre, att)
    torch.cuda.synchronize()
    for a, b in zip(first, outs):
        assert torch.equal(a, b)
    s = torch.cuda.Stream()
    outs = tuple(torch.empty_like(o) for o in first)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        chain.forward_device(pre, att, out=outs, stream=s)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            chain.forward_device(pre, att, out=outs, stream=s)
    torch.cuda.synchronize()
    for _ in range(5):
        for o in outs:
            o.fill_(0.0)
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(first, outs):
            assert torch.equal(a, b)
        chain.forward_device(pre, att)      # an eager launch between replays
        torch.cuda.synchronize()
    chain.check()


def test_wait_that_runs_out_is_reported_and_recovers():
    """Producers kept from counting and a bound of four polls: every wait runs
    out, every workgroup exits and the outputs are NaN. The next launch with
    the defaults matches the oracle whether or not check() ran in between
    (each launch starts from cleared counter blocks), and check() raises for
    the failed launch when it is the last one."""
    from localai_amd import _lib, device, layer, synth
    shapes = {'attn_output': (12, 1024, 1024), 'ffn_gate': (12, 2816, 1024), 'ffn_up': (12, 2816, 1024),
              'ffn_down': (14, 1024, 2816), 'attn_q': (12, 1024, 1024), 'attn_k': (12, 256, 1024),
              'attn_v': (14, 256, 1024)}
    chain, raws, w_ffn, w_attn, rng = build(shapes, 17)
    pre, att = synth.activations(rng, 1024), synth.activations(rng, 1024)
    pd, ad = device.to_device_f32(pre), device.to_device_f32(att)
    want, _ = olayer.chain(raws, pre, att, w_ffn, w_attn, 1e-5)
    lib = _lib.load()
    layer.set_mode(True)       # the waits are those of the one-launch chain
    try:
        for checked in (False, True):
            try:
                assert lib.localai_hip_debug_fused_wait(4, 0) == 0
                got = chain.forward_device(pd, ad)
                if checked:
                    with pytest.raises(_lib.HipError) as err:
                        chain.check()
                    assert err.value.status == 3
                else:
                    device.torch().cuda.synchronize()
                assert all(o.isnan().all() for o in got[1:])
            finally:
                lib.localai_hip_debug_fused_wait(0, 1)
            print(f'layer chain: default launch after a failed one (check() between: {checked})', flush=True)
            got = chain.forward_device(pd, ad)
            chain.check()
            check_outputs(got, want)
    finally:
        layer.set_mode(False)
