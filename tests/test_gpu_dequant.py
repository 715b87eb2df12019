"""GPU dequant parity: bit-exact against the oracle (and the reference golden
decodes) for every GGML type of engine/dequant.py; repack round trips."""
import numpy as np
import pytest

from oracle import quant
from tests.conftest import normwise_rel
from tests.gpu_util import bits, random_ggml

pytestmark = pytest.mark.gpu

ALL_TYPES = (0, 1, 2, 3, 6, 7, 8, 12, 13, 14)
REPACK_TYPES = (2, 8, 12, 13, 14)


@pytest.mark.parametrize('t', ALL_TYPES)
@pytest.mark.parametrize('nblocks', (1, 3, 37))
def test_dequant_bit_exact(t, nblocks):
    from localai_amd import dequant
    rng = np.random.default_rng(100 + t * 7 + nblocks)
    block, _ = quant.block_layout(t)
    n = block * nblocks * (64 if block == 1 else 1)
    raw = random_ggml(rng, t, n)
    got = dequant.dequantize(raw, t, (n,))
    ref = quant.dequantize(raw, t, (n,))
    np.testing.assert_array_equal(bits(got), bits(ref))


@pytest.mark.parametrize('t', (2, 3, 6, 7, 8, 12, 13, 14))
def test_dequant_subnormal_zero_and_extreme_scales(t):
    from localai_amd import dequant
    rng = np.random.default_rng(200 + t)
    block, _ = quant.block_layout(t)
    scales = [0.0, -0.0, 6e-8, 3e-6, -6.1e-5, 1.0, 65504.0, -2.0, 0.03125]
    raw = random_ggml(rng, t, block * 64, scales=scales)
    got = dequant.dequantize(raw, t, (64, block))
    ref = quant.dequantize(raw, t, (64, block))
    np.testing.assert_array_equal(bits(got), bits(ref))


@pytest.mark.parametrize('t', (8, 2, 13, 12, 14))
def test_dequant_matches_reference_golden_decode(golden, t):
    from localai_amd import dequant
    block, bpb = quant.block_layout(t)
    want = golden[f'decode_{t}']
    raw = golden[f'raw_{t}'].tobytes()[:want.shape[0] * (512 // block) * bpb]
    np.testing.assert_array_equal(dequant.dequantize(raw, t, want.shape), want)


def test_dequant_full_size_q4_k_ffn():
    """14336 x 4096 Q4_K (the Llama-3-8B ffn_gate shape), bit-exact."""
    from localai_amd import dequant, synth
    rng = np.random.default_rng(1)
    raw = synth.quant_tensor(rng, 12, 14336, 4096)
    got = dequant.dequantize(raw, 12, (14336, 4096))
    ref = quant.dequantize(raw, 12, (14336, 4096))
    np.testing.assert_array_equal(bits(got), bits(ref))


def test_dequant_empty_and_errors():
    from localai_amd import dequant
    assert dequant.dequantize(b'', 12, (0,)).shape == (0,)
    with pytest.raises(NotImplementedError):
        dequant.dequantize(b'\x00' * 32, 99, (16,))
    with pytest.raises(ValueError):
        dequant.dequantize(b'\x00' * 144, 12, (100,))


@pytest.mark.parametrize('t', REPACK_TYPES)
@pytest.mark.parametrize('rows,cols,batch', [(1, 256, 1), (100, 512, 3), (64, 2048, 2), (130, 768, 1)])
def test_repack_round_trip_and_expert_dequant(t, rows, cols, batch):
    from localai_amd import device
    rng = np.random.default_rng(300 + t + rows)
    raw = random_ggml(rng, t, batch * rows * cols)
    q = device.QMat.from_ggml(raw, t, rows, cols, batch)
    back = q.unpack().cpu().numpy().tobytes()
    assert back == raw
    per = len(raw) // batch
    for e in range(batch):
        got = q.dequant(e).cpu().numpy()
        want = quant.dequantize(raw[e * per:(e + 1) * per], t, (rows, cols))
        np.testing.assert_array_equal(bits(got), bits(want))
    q.close()


ALL_F16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _nan_aware_equal(got, ref):
    """Bit equality wherever the oracle value is not a NaN; NaN exactly where
    the oracle has one. NaN payloads that went through a product or a
    difference are not compared: x86 and gfx950 propagate NaN payloads and
    signs through arithmetic differently, and the reference's arithmetic on a
    NaN scale gives a NaN with no meaningful payload either way."""
    got, ref = np.asarray(got, np.float32), np.asarray(ref, np.float32)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(bits(got)[~nan], bits(ref)[~nan])


def test_dequant_f16_every_bit_pattern():
    """All 65536 fp16 patterns as the F16 type: bit for bit, NaN payloads and
    signalling NaNs included (engine/dequant.py:20-24; half_to_float,
    engine/native_quant.cpp:12-33)."""
    from localai_amd import dequant
    raw = ALL_F16.tobytes()
    got = dequant.dequantize(raw, 1, (65536,))
    ref = quant.dequantize(raw, 1, (65536,))
    np.testing.assert_array_equal(bits(got), bits(ref))


@pytest.mark.parametrize('t', (8, 2, 3, 6, 7, 12, 13, 14))
def test_dequant_every_fp16_scale_pattern(t):
    """Every fp16 pattern as the block scale d (and, with a different pattern
    per block, as the second fp16 field: dmin of Q4_K / Q5_K, m of Q4_1 /
    Q5_1), random quants: bit-exact for every non-NaN value, NaN where the
    oracle has NaN."""
    from localai_amd import dequant
    block, bpb = quant.block_layout(t)
    rng = np.random.default_rng(900 + t)
    nb = 65536
    buf = rng.integers(0, 256, size=(nb, bpb), dtype=np.uint8)
    off = 208 if t == 14 else 0
    buf[:, off:off + 2] = ALL_F16.view(np.uint8).reshape(nb, 2)
    if t in (3, 7, 12, 13):
        second = ALL_F16[(np.arange(nb) * 7919) % nb]
        buf[:, 2:4] = second.view(np.uint8).reshape(nb, 2)
    raw = buf.tobytes()
    got = dequant.dequantize(raw, t, (nb * block,))
    with np.errstate(invalid='ignore', over='ignore'):
        ref = quant.dequantize(raw, t, (nb * block,))
    _nan_aware_equal(got, ref)


@pytest.mark.parametrize('t', (12, 14, 8))
def test_tile_form_only_until_row_planes_are_needed(t):
    """Q4_K / Q6_K / Q8_0 handles hold the tile form only (as many bytes as
    GGML, up to the padding of the last 16-row tile); one-vector and
    several-vector matvecs both run on it and build no row planes. Results
    and the GGML bytes read back do not change."""
    from localai_amd import device
    rng = np.random.default_rng(500 + t)
    rows, cols, batch = 100, 1024, 2
    raw = random_ggml(rng, t, batch * rows * cols)
    q = device.QMat.from_ggml(raw, t, rows, cols, batch)
    try:
        before = q.device_bytes
        tiles = batch * ((rows + 15) // 16) * 16 * (cols // 256) * {12: 144, 14: 210, 8: 272}[t]
        assert tiles <= before <= tiles + 256 * batch
        x = rng.standard_normal((3, cols)).astype(np.float32)
        xd = device.to_device_f32(x)
        one = q.matvec(xd[0], expert=1).cpu().numpy()
        assert q.device_bytes == before
        per = len(raw) // batch
        want = np.stack([quant.matvec_exact(raw[per:], t, rows, cols, x[i]) for i in range(3)])
        got = q.matvec(xd, expert=1).cpu().numpy()
        assert q.device_bytes == before
        for i in range(3):
            assert normwise_rel(got[i], want[i]) < 1e-5
        assert q.unpack().cpu().numpy().tobytes() == raw
        np.testing.assert_array_equal(bits(q.matvec(xd[0], expert=1).cpu().numpy()), bits(one))
    finally:
        q.close()
