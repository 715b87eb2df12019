"""Pins the decode-layer chain oracle (oracle/layer.py) with checks a plausible
mistake fails: the norm's unit RMS and scale invariance, RoPE as complex
multiplication, and the chain as a composition of separately pinned pieces."""
import numpy as np

from oracle import layer, quant


def test_norm_has_unit_rms_and_is_scale_invariant():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4096) * 3.0
    y = layer.norm(x, np.ones(4096), 0.0)
    assert abs(np.sqrt(np.mean(y * y)) - 1.0) < 1e-12
    np.testing.assert_allclose(layer.norm(7.5 * x, np.ones(4096), 0.0), y, rtol=1e-12)
    w = rng.uniform(0.5, 2.0, 4096)
    np.testing.assert_allclose(layer.norm(x, w, 0.0), y * w, rtol=1e-12)
    # eps acts inside the root: a zero vector stays zero, a tiny one is damped
    assert np.all(layer.norm(np.zeros(8), np.ones(8), 1e-5) == 0.0)
    small = np.full(8, 1e-4)
    np.testing.assert_allclose(layer.norm(small, np.ones(8), 1e-5), small / np.sqrt(1e-8 + 1e-5), rtol=1e-12)


def test_rope_is_complex_rotation():
    rng = np.random.default_rng(1)
    head_dim, heads, half = 128, 4, 60            # rotary prefix shorter than the head
    a = rng.standard_normal(heads * head_dim)
    ang = rng.uniform(-10, 10, half)
    got = layer.rope_pairs(a, np.cos(ang), np.sin(ang), head_dim).reshape(heads, head_dim)
    h = a.reshape(heads, head_dim)
    z = (h[:, 0:2 * half:2] + 1j * h[:, 1:2 * half:2]) * np.exp(1j * ang)[None, :]
    np.testing.assert_allclose(got[:, 0:2 * half:2], z.real, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got[:, 1:2 * half:2], z.imag, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(got[:, 2 * half:], h[:, 2 * half:])
    # rotation keeps each pair's norm
    np.testing.assert_allclose(np.abs(z), np.abs(h[:, 0:2 * half:2] + 1j * h[:, 1:2 * half:2]), rtol=1e-12)


def test_chain_is_the_composition_of_pinned_pieces():
    """Each stage recomputed from quant.matvec_exact and SciPy's expit."""
    from scipy.special import expit
    from localai_amd import synth
    rng = np.random.default_rng(2)
    dim, ffn = 256, 512
    shapes = {'attn_output': (12, dim, dim), 'ffn_gate': (12, ffn, dim), 'ffn_up': (12, ffn, dim),
              'ffn_down': (14, dim, ffn), 'attn_q': (12, dim, dim), 'attn_k': (12, 64, dim), 'attn_v': (14, 64, dim)}
    mats = {n: (synth.quant_tensor(rng, t, r, c), t, r, c) for n, (t, r, c) in shapes.items()}
    pre, att = rng.standard_normal(dim), rng.standard_normal(dim)
    w1, w2 = rng.uniform(0.5, 1.5, dim), rng.uniform(0.5, 1.5, dim)
    (x2, q, k, v), (o, act, d) = layer.chain(mats, pre, att, w1, w2, 1e-5)
    mv = lambda n, x: quant.matvec_exact(*mats[n][:1], *mats[n][1:], x)   # noqa: E731
    np.testing.assert_allclose(o, mv('attn_output', att), rtol=1e-15)
    x1 = pre + o
    u = x1 / np.sqrt(np.mean(x1 ** 2) + 1e-5) * w1
    g, up = mv('ffn_gate', u), mv('ffn_up', u)
    np.testing.assert_allclose(act, g * expit(g) * up, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(x2, x1 + mv('ffn_down', act), rtol=1e-12)
    vin = x2 / np.sqrt(np.mean(x2 ** 2) + 1e-5) * w2
    for got, n in ((q, 'attn_q'), (k, 'attn_k'), (v, 'attn_v')):
        np.testing.assert_allclose(got, mv(n, vin), rtol=1e-12, atol=1e-12)
