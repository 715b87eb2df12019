"""GPU MoE layer parity against the composition oracle (oracle/moe.py).

Routing indices must be identical (ties to the lower expert index); gates and
outputs within max-rel 1e-3 (normwise). Below 32 tokens the layer runs the
grouped matvec path (i8 MFMA on three-piece x for Q4_K / Q6_K experts, fp32
VALU otherwise), which lands near 1e-6; from 32 tokens on it runs the expert
GEMM path (f16 MFMA operands, fp32 accumulation), near 2e-4."""
import numpy as np
import pytest

from oracle import moe as omoe
from tests.conftest import normwise_rel

pytestmark = pytest.mark.gpu


def make_layer(rng, E, H, I, t, scale=0.02, bias=None):
    from localai_amd import synth
    rw = (rng.standard_normal((E, H)) * scale).astype(np.float32)
    gu = synth.quant_tensor(rng, t, 2 * I, H, batch=E)
    dn = synth.quant_tensor(rng, t, H, I, batch=E)
    return rw, gu, dn


def run_both(rw, gu, dn, t, E, H, I, k, h, bias=None):
    from localai_amd.moe import MoELayer
    layer = MoELayer(rw, gu, dn, t, E, H, I, k, router_b=bias)
    out, idx, g = layer.forward(h)
    ref_out, ref_idx, ref_g, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I, router_bias=bias)
    return (out, idx, g), (ref_out, ref_idx, ref_g)


@pytest.mark.parametrize('T', (1, 8))
def test_zaya_shaped_decode(T):
    """hidden 2048, 16 experts, top-2, SwiGLU intermediate 4096, Q6_K experts."""
    from localai_amd import synth
    rng = np.random.default_rng(40 + T)
    E, H, I, k = 16, 2048, 4096, 2
    rw, gu, dn = make_layer(rng, E, H, I, 14)
    h = synth.activations(rng, T, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, 14, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-3
    assert normwise_rel(out, rout) < 1e-5


def test_qwen3_moe_style_small_prefill():
    """128 experts, top-8, intermediate 768, Q4_K experts, Zipf-skewed router
    bias; 48 tokens take the expert GEMM path."""
    from localai_amd import synth
    rng = np.random.default_rng(7)
    E, H, I, k, T = 128, 2048, 768, 8, 48
    rw, gu, dn = make_layer(rng, E, H, I, 12)
    bias = synth.zipf_bias(E)
    h = synth.activations(rng, T, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, 12, E, H, I, k, h, bias=bias)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-3


@pytest.mark.parametrize('scale', (2.0 ** -30, 1.0, 2.0 ** 30))
@pytest.mark.parametrize('t,I', [(12, 256), (14, 256), (8, 256), (8, 320)])
def test_prefill_act_rows_at_extreme_scales(scale, t, I):
    """The gate_up GEMM scales its f16 SiLU*up rows by a power of two taken
    from a bound (expert row norms times |h|^2) when inter is a multiple of
    256; otherwise (Q8_0, I = 320) it writes fp32 rows that a conversion
    kernel scales by their maximum. Both keep the layer within 1e-3 of the
    oracle for activations 2^30 times smaller or larger than usual, and for a
    token whose row of h is all zero."""
    from localai_amd import synth
    rng = np.random.default_rng(int(np.log2(scale)) + 100 + I + t)
    E, H, k, T = 8, 512, 2, 40
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H) * np.float32(scale)
    h[5] = 0.0
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, t, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    assert np.isfinite(out).all()
    assert normwise_rel(out, rout) < 1e-3


@pytest.mark.parametrize('t', (12, 14, 8))
@pytest.mark.parametrize('T', (31, 32, 67, 200))
def test_gemm_path_threshold_and_ragged_tiles(t, T):
    """Both sides of the 32-token switch to the expert GEMM path, with expert
    token counts that are not multiples of the 64-token tile (67 and 200
    tokens: the eight-token router tiles end with a partial one)."""
    from localai_amd import synth
    rng = np.random.default_rng(T * 3 + t)
    E, H, I, k = 16, 512, 256, 4
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, t, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < (1e-5 if T < 32 else 1e-3)


def test_forced_router_ties_pick_lower_index():
    from localai_amd import synth
    rng = np.random.default_rng(8)
    E, H, I, k, T = 8, 256, 256, 3, 5
    rw, gu, dn = make_layer(rng, E, H, I, 14)
    rw[5] = rw[2]          # experts 2 and 5 always tie
    rw[6] = rw[2]          # and 6
    rw[2] *= 1.0
    h = synth.activations(rng, T, H)
    h[:, :] = np.abs(h) * np.sign(rw[2])[None, :]   # make expert 2's logit the largest
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, 14, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    assert np.all(idx[:, 0] == 2) and np.all(idx[:, 1] == 5) and np.all(idx[:, 2] == 6)
    np.testing.assert_allclose(g, 1.0 / 3, rtol=1e-6)
    assert normwise_rel(out, rout) < 1e-5


def test_routing_tables_and_gates_at_full_prefill_size():
    """512 tokens, 128 experts, top-8 (Qwen3-MoE-style shape): routing indices
    equal the oracle's, every token's gates sum to one, output finite."""
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(9)
    E, H, I, k, T = 128, 2048, 768, 8, 512
    rw, gu, dn = make_layer(rng, E, H, I, 12)
    bias = synth.zipf_bias(E)
    h = synth.activations(rng, T, H)
    layer = MoELayer(rw, gu, dn, 12, E, H, I, k, router_b=bias)
    out, idx, g = layer.forward(h)
    logits = omoe.router_logits(h, rw) + bias[None, :]
    ridx, _ = omoe.topk(logits.astype(np.float32), k)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g.sum(axis=1), 1.0, rtol=1e-5)
    assert np.isfinite(out).all()
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert counts.sum() == T * k and counts.max() > 4 * counts.mean()   # Zipf skew present
    # outputs of a sample of tokens against the oracle (a token's output depends on it alone)
    sample = np.arange(0, T, 37)
    rout, ridx2, _, _ = omoe.moe_forward(h[sample], rw, gu, dn, 12, E, k, I, router_bias=bias)
    np.testing.assert_array_equal(idx[sample], ridx2)
    assert normwise_rel(out[sample], rout) < 1e-3


def test_zaya_expert_matvec_mixin():
    from types import SimpleNamespace
    from localai_amd import synth
    from localai_amd.moe import ZayaExpertsMixin
    from oracle import quant
    rng = np.random.default_rng(10)
    E, rows, cols = 4, 128, 512
    raw = synth.quant_tensor(rng, 14, rows, cols, batch=E)
    blob = b'\x00' * 64 + raw
    gguf = SimpleNamespace(tensors={'blk.1.ffn_down_exps.weight': SimpleNamespace(
        shape=(E, rows, cols), ggml_type=14, offset=64)}, _map=blob)
    model = type('M', (ZayaExpertsMixin,), {})()
    model.gguf, model.n_experts = gguf, E
    x = rng.standard_normal(cols).astype(np.float32)
    per = len(raw) // E
    for e in range(E):
        got = model._expert_matvec('blk.1.ffn_down_exps.weight', e, x)
        want = quant.matvec_exact(raw[e * per:(e + 1) * per], 14, rows, cols, x)
        assert normwise_rel(got, want) < 1e-5


@pytest.mark.parametrize('t,k,H,I', [
    (12, 1, 1024, 512),     # top-1: down + combine fused for one token
    (12, 3, 1024, 512),     # top-3: grouped down, then the combine kernel
    (14, 2, 4608, 256),     # gate_up K = 18 super-blocks: four per wave
    (12, 2, 512, 4352),     # down K = 17 super-blocks: four per wave
])
@pytest.mark.parametrize('T', (1, 3))
def test_mfma_decode_path_shapes(t, k, H, I, T):
    """Decode (T < 32) with Q4_K / Q6_K experts runs the i8 MFMA expert
    kernels; every launch-shape branch against the oracle."""
    from localai_amd import synth
    rng = np.random.default_rng(T * 100 + k * 10 + t + H)
    E = 8
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, t, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-5


@pytest.mark.parametrize('T,E,H,k', [
    (1, 8, 288, 2),       # one token: the one-wave router, fused expert kernel; H ends in a partial chunk
    (1, 130, 256, 8),     # one token, 130 experts, top-8: one-wave router, selection in the permutation
    (5, 200, 288, 3),     # a few tokens, partial 256-chunk, more experts than a wave's lanes
    (15, 20, 256, 3),     # just below the tiled router
    (16, 20, 288, 3),     # tiled router, partial chunk, experts not a multiple of 16
    (37, 80, 320, 5),     # E > 64: DPP top-k; tokens not a multiple of 8
    (67, 130, 512, 8),    # three expert tiles, the last with 2 experts
    (40, 1, 256, 1),      # one expert: every assignment matches in the permutation
])
def test_router_logits_bit_exact(T, E, H, k):
    """Router logits (read back from the workspace) equal the canonical sum of
    oracle/moe.py bit for bit, with a bias, and the selection equals
    np.lexsort's, including ties planted between experts e and e + 64 (the same
    lane of the DPP reduction) and between neighbouring experts."""
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(T * 7 + E + H)
    I, t = 128, 8
    rw, gu, dn = make_layer(rng, E, H, I, t)
    if E > 2:
        rw[E - 1] = rw[1]            # tie between 1 and E - 1
    if E > 64:
        rw[66] = rw[2]               # tie between lanes' first and second experts
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32)
    if E > 2:
        bias[E - 1] = bias[1]
    if E > 64:
        bias[66] = bias[2]
    h = synth.activations(rng, T, H)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k, router_b=bias)
    out, idx, g = layer.forward(h)
    got = layer.last_router_logits(T).cpu().numpy()
    want = (omoe.router_logits(h, rw) + bias[None, :]).astype(np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    ridx, sel = omoe.topk(want, k)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, omoe.gates(sel), rtol=1e-5, atol=1e-6)
    assert np.isfinite(out).all()


@pytest.mark.parametrize('k', (2, 8))
def test_one_token_layer_repeated_and_graph_replayed(k):
    """The one-token layer runs as one launch whose workgroups hand work to
    each other through counters in the workspace; every call must leave them
    ready for the next: back-to-back calls with new tokens, a call of another
    size in between, and replays of a captured HIP graph (the token copied in
    between replays) all match the oracle. k = 8 takes the route, permute
    and grouped kernels, whose tables must be rebuilt every call."""
    import torch
    from localai_amd import synth, device
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(77 + k)
    E, H, I, t = 16, 1024, 512, 14
    rw, gu, dn = make_layer(rng, E, H, I, t)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)

    def check(h, out, idx, g):
        rout, ridx, rg, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
        assert normwise_rel(out, rout) < 1e-5

    for _ in range(3):
        h = synth.activations(rng, 1, H)
        check(h, *layer.forward(h))
    h3 = synth.activations(rng, 3, H)
    check(h3, *layer.forward(h3))
    h = synth.activations(rng, 1, H)
    check(h, *layer.forward(h))

    stream = torch.cuda.Stream()
    hd = device.to_device_f32(synth.activations(rng, 1, H))
    out = torch.empty((1, H), dtype=torch.float32, device=hd.device)
    idx = torch.empty((1, k), dtype=torch.int32, device=hd.device)
    gates = torch.empty((1, k), dtype=torch.float32, device=hd.device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
    torch.cuda.synchronize()
    for _ in range(3):
        h = synth.activations(rng, 1, H)
        hd.copy_(torch.from_numpy(h).to(hd.device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(h, out.cpu().numpy(), idx.cpu().numpy(), gates.cpu().numpy())


def test_prefill_repeated_and_graph_replayed():
    """The prefill path (routing kernels, f16 conversions, expert GEMMs,
    combine): eager calls with new tokens, and replays of a captured HIP graph
    (new tokens copied and an eager call of another size between replays),
    all match the oracle."""
    import torch
    from localai_amd import synth, device
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(91)
    E, H, I, k, t, T = 32, 1024, 256, 4, 12, 96
    rw, gu, dn = make_layer(rng, E, H, I, t)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)

    def check(h, out, idx, g):
        rout, ridx, rg, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
        assert normwise_rel(out, rout) < 1e-3

    for _ in range(2):
        h = synth.activations(rng, T, H)
        check(h, *layer.forward(h))
    stream = torch.cuda.Stream()
    hd = device.to_device_f32(synth.activations(rng, T, H))
    out = torch.empty((T, H), dtype=torch.float32, device=hd.device)
    idx = torch.empty((T, k), dtype=torch.int32, device=hd.device)
    gates = torch.empty((T, k), dtype=torch.float32, device=hd.device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
    torch.cuda.synchronize()
    for _ in range(3):
        h = synth.activations(rng, T, H)
        hd.copy_(torch.from_numpy(h).to(hd.device))
        out.fill_(0.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(h, out.cpu().numpy(), idx.cpu().numpy(), gates.cpu().numpy())
        h2 = synth.activations(rng, 40, H)
        check(h2, *layer.forward(h2))


def test_fused_wait_that_runs_out_is_reported():
    """The one-token fused expert kernel with its gate_up workgroups kept from
    counting themselves done and a bound of four polls: every wait runs out,
    every workgroup still exits, the output is NaN and the layer's check
    raises (EHIP). With the defaults restored the same layer matches the
    oracle again."""
    from localai_amd import _lib, synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(61)
    E, H, I, k = 8, 512, 256, 2
    rw, gu, dn = make_layer(rng, E, H, I, 14)
    h = synth.activations(rng, 1, H)
    layer = MoELayer(rw, gu, dn, 14, E, H, I, k)
    lib = _lib.load()
    try:
        assert lib.localai_hip_debug_fused_wait(4, 0) == 0
        out, _, _ = layer.forward_device(layer.router_w.new_tensor(h))
        with pytest.raises(_lib.HipError) as err:
            layer.check(1)
        assert err.value.status == 3
        assert out.isnan().all()
    finally:
        lib.localai_hip_debug_fused_wait(0, 1)
    (o, i, g), (ro, ri, rg) = run_both(rw, gu, dn, 14, E, H, I, k, h)
    np.testing.assert_array_equal(i, ri)
    assert normwise_rel(o, ro) < 1e-5


def expected_tables(idx, E, tile_w):
    """Stable counting sort of the flat assignments a = t * k + s by expert,
    its inverse, per-expert counts / offsets / active list and the expert GEMM
    tiles (runs of tile_w perm positions per expert: the full runs of every
    expert in expert order, then the partial last runs in expert order)."""
    flat = idx.reshape(-1).astype(np.int64)
    perm = np.argsort(flat, kind='stable').astype(np.int32)
    pos = np.empty_like(perm)
    pos[perm] = np.arange(perm.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=E).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    want = {'counts': counts, 'offsets': offsets, 'active': np.flatnonzero(counts).astype(np.int32),
            'perm': perm, 'pos': pos}
    if tile_w:
        te, tp, tn = [], [], []
        for e in np.flatnonzero(counts):
            for p in range(0, counts[e] - tile_w + 1, tile_w):
                te.append(e)
                tp.append(offsets[e] + p)
                tn.append(tile_w)
        for e in np.flatnonzero(counts % tile_w):
            te.append(e)
            tp.append(offsets[e] + counts[e] - counts[e] % tile_w)
            tn.append(counts[e] % tile_w)
        want.update(tile_e=np.array(te, np.int32), tile_p0=np.array(tp, np.int32), tile_n=np.array(tn, np.int32))
    return want


@pytest.mark.parametrize('E,T,k', [
    (16, 1, 2),        # one token (Q8_0 experts of inter 128: route, permute, grouped kernels)
    (16, 8, 2),        # few assignments over few experts (one wave's worth)
    (64, 16, 4),       # 64 assignments over 64 experts
    (2, 5, 1),         # two experts, one expert per token
    (1, 40, 1),        # one expert: every assignment matches
    (16, 31, 4),       # matvec path (no tiles), sixteen waves of eight assignments or fewer
    (128, 512, 8),     # lane masks in LDS, ranks in registers, perm staged in LDS
    (128, 1100, 8),    # wave ranges past 512 assignments: ranks kept in pos[] between steps
    (64, 2200, 8),     # perm too large to stage: scattered stores
    (512, 200, 8),     # too many experts for the LDS lane masks: ballots
    (1024, 40, 2),     # the largest expert count
    (1024, 3, 16),     # the largest expert count and top-k below the tiled router
    (130, 1, 8),       # one token over more than 64 experts: selected in the permutation
    (16, 15, 4),       # the most tokens of the one-wave router
])
def test_routing_tables_are_a_stable_sort(E, T, k):
    """perm lists the assignments in (expert, a) order, pos inverts it, and
    counts / offsets / active / tiles follow, for every variant of the
    permutation kernel. Random router weights with a Zipf bias make some
    experts crowded and others empty."""
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(E * 31 + T)
    H, I, t = 256, 128, 8
    rw, gu, dn = make_layer(rng, E, H, I, t, scale=0.05)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k, router_b=synth.zipf_bias(E) if E > 1 else None)
    h = synth.activations(rng, T, H)
    _, idx, _ = layer.forward(h)
    got = layer.last_tables(T)
    want = expected_tables(idx, E, got.get('tile_w', 0))
    assert ('tile_e' in got) == (T >= 32)
    for name, w in want.items():
        np.testing.assert_array_equal(got[name], w, err_msg=name)


@pytest.mark.parametrize('t,E,T,k,H,I', [
    (14, 16, 8, 2, 1024, 512),     # ZAYA-like, one workgroup tile of down rows per 16
    (12, 16, 2, 2, 512, 256),      # two tokens
    (12, 64, 31, 2, 512, 256),     # 62 assignments over 64 experts (one wave's worth)
    (14, 4, 31, 2, 256, 256),      # few experts, many assignments each
    (12, 8, 5, 1, 2048, 4096),     # top-1, K = 8 / 16 super-blocks (ZAYA's row widths)
    (14, 2, 3, 2, 256, 256),       # both experts for every token
])
def test_few_token_layer_and_tables(t, E, T, k, H, I):
    """2 .. 31 tokens on Q4_K / Q6_K experts (route and permute kernels, then
    the grouped i8 MFMA kernels): routing, gates and output against the
    oracle, and the routing tables against a stable sort."""
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(T * 13 + E + t)
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)
    out, idx, g = layer.forward(h)
    rout, ridx, rg, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-5
    got = layer.last_tables(T)
    for name, w in expected_tables(idx, E, 0).items():
        np.testing.assert_array_equal(got[name], w, err_msg=name)


@pytest.mark.parametrize('T', (1, 8))
def test_routing_tables_on_the_mfma_decode_path(T):
    """One token (the fused kernel's first workgroup writes the tables) and
    eight (route and permute kernels), Q6_K experts: the tables against a
    stable sort."""
    from localai_amd import synth
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(5 + T)
    E, H, I, k, t = 16, 512, 256, 2, 14
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)
    _, idx, _ = layer.forward(h)
    got = layer.last_tables(T)
    for name, w in expected_tables(idx, E, 0).items():
        np.testing.assert_array_equal(got[name], w, err_msg=name)


@pytest.mark.parametrize('T', (1, 8))
def test_output_in_place_of_h(T):
    """out given as h's own buffer: the fused kernels (which clear out while
    other workgroups still read h) are not taken; the separate kernels and
    the combine give the oracle's result."""
    import torch
    from localai_amd import synth, device
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(71 + T)
    E, H, I, k, t = 16, 512, 256, 2, 14
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, T, H)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)
    hd = device.to_device_f32(h)
    out, idx, g = layer.forward_device(hd, out=hd)
    torch.cuda.synchronize()
    assert out.data_ptr() == hd.data_ptr()
    rout, ridx, rg, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I)
    np.testing.assert_array_equal(idx.cpu().numpy(), ridx)
    assert normwise_rel(out.cpu().numpy(), rout) < 1e-5


def test_few_token_layer_repeated_and_graph_replayed():
    """The few-token path (route, permute, grouped gate_up and down):
    back-to-back calls of 8 tokens, a call of 3 and one of 1 in between, and
    replays of a captured graph all match the oracle."""
    import torch
    from localai_amd import synth, device
    from localai_amd.moe import MoELayer
    rng = np.random.default_rng(78)
    E, H, I, k, t, T = 16, 1024, 512, 2, 14, 8
    rw, gu, dn = make_layer(rng, E, H, I, t)
    layer = MoELayer(rw, gu, dn, t, E, H, I, k)

    def check(h, out, idx, g):
        rout, ridx, rg, _ = omoe.moe_forward(h, rw, gu, dn, t, E, k, I)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
        assert normwise_rel(out, rout) < 1e-5

    for n in (T, T, 3, 1, T):
        h = synth.activations(rng, n, H)
        check(h, *layer.forward(h))
    stream = torch.cuda.Stream()
    hd = device.to_device_f32(synth.activations(rng, T, H))
    out = torch.empty((T, H), dtype=torch.float32, device=hd.device)
    idx = torch.empty((T, k), dtype=torch.int32, device=hd.device)
    gates = torch.empty((T, k), dtype=torch.float32, device=hd.device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            layer.forward_device(hd, out=out, idx=idx, gates=gates, stream=stream)
    torch.cuda.synchronize()
    for _ in range(3):
        h = synth.activations(rng, T, H)
        hd.copy_(torch.from_numpy(h).to(hd.device))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        check(h, out.cpu().numpy(), idx.cpu().numpy(), gates.cpu().numpy())
        h3 = synth.activations(rng, 3, H)
        check(h3, *layer.forward(h3))



@pytest.mark.parametrize('t', (8, 12, 14))
@pytest.mark.parametrize('T,k', [(1, 2), (1, 3), (5, 2), (8, 1)])
def test_long_expert_rows_on_mfma(t, T, k):
    """Expert rows of 33-64 blocks of 256 (down K = 9216: 36 blocks; gate_up K
    = 9216 in the second layer) take the streamed i8 MFMA kernels (eight
    blocks per wave through two register sets), one token and several, for
    Q8_0, Q4_K and Q6_K: routing, gates and output against the oracle.
    Normwise 1e-4 (the specification's bar is 1e-3): a Q4_K row is
    d * sum(sc q x) - dmin * sum(mn x) with both sums far larger than the
    result (the quants are unsigned, the minima subtracted), and with these
    random weights the fp32 roundings of that difference over 36 blocks
    leave ~3e-5 of a one-token output (~5e-6 on the shorter rows of the
    other tests)."""
    from localai_amd import synth
    rng = np.random.default_rng(T * 10 + k + t)
    E = 4
    for H, I in ((512, 9216), (9216, 256)):
        rw, gu, dn = make_layer(rng, E, H, I, t)
        h = synth.activations(rng, T, H)
        (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, t, E, H, I, k, h)
        np.testing.assert_array_equal(idx, ridx)
        np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
        assert normwise_rel(out, rout) < 1e-4


@pytest.mark.parametrize('T,k,I', [(1, 2, 512), (1, 1, 256), (3, 2, 512), (8, 2, 256), (4, 3, 512), (6, 2, 320)])
def test_q8_0_experts_decode(T, k, I):
    """Q8_0 experts below 32 tokens: the fused one-token kernel and the
    grouped i8 MFMA kernels on the tile form (inter a multiple of 256), the
    row-plane kernels otherwise (inter 320), against the oracle."""
    from localai_amd import synth
    rng = np.random.default_rng(T * 31 + k + I)
    E, H = 8, 1024
    rw, gu, dn = make_layer(rng, E, H, I, 8)
    h = synth.activations(rng, T, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, 8, E, H, I, k, h)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-5


@pytest.mark.parametrize('t', (12, 14, 8))
@pytest.mark.parametrize('E,k', [(16, 3), (128, 8), (64, 4), (8, 8)])
def test_one_token_top_k(t, E, k):
    """One token with top-3 .. top-8 (Qwen3-MoE decode: 128 experts, top-8):
    the router over (expert, token) workgroups, the selection inside the
    permutation, the grouped kernels and the combine. Routing, gates and
    output against the oracle."""
    from localai_amd import synth
    rng = np.random.default_rng(E * 7 + k + t)
    H, I = 1024, 512
    rw, gu, dn = make_layer(rng, E, H, I, t)
    h = synth.activations(rng, 1, H)
    (out, idx, g), (rout, ridx, rg) = run_both(rw, gu, dn, t, E, H, I, k, h, bias=synth.zipf_bias(E))
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(g, rg, rtol=1e-5, atol=1e-6)
    assert normwise_rel(out, rout) < 1e-5
