"""GPU prefill matmul (MFMA, f16 operands, fp32 accumulation) against the fp64
oracle X @ dequant(W)^T and the reference's own batched-matmul outputs.

Tolerance: weights are decoded exactly and rounded once to f16, x rows are
scaled by a power of two and rounded to f16, so each product carries at most
2^-11 relative error and each output at most about 2^-11 * sum|w*x| (fp32
accumulation adds K * 2^-24 of the same sum). Gates: every output within
1e-3 * sum_k |w_k x_k| (the dot-product error bound, which holds however much
the sum cancels), and the path's max-rel 1e-3 target (normwise:
max|y - y_ref| / max|y_ref|) for tiles of at least 64 outputs, where the
typical figure is near 2e-4."""
import numpy as np
import pytest

from oracle import quant
from tests.conftest import normwise_rel
from tests.gpu_util import random_ggml

pytestmark = pytest.mark.gpu

TYPES = (2, 8, 12, 13, 14)
MAX_REL = 1e-3


def check(got, raw, t, rows, cols, xs):
    ref = quant.matmul_exact(raw, t, rows, cols, xs)
    w = quant.dequantize(raw, t, (rows, cols)).astype(np.float64)
    absdot = np.abs(np.asarray(xs, dtype=np.float64)) @ np.abs(w).T
    assert np.all(np.abs(got - ref) <= MAX_REL * absdot + 1e-30)
    if ref.size >= 64:
        assert normwise_rel(got, ref) < MAX_REL
    return ref


def gpu_matmul(raw, t, rows, cols, xs, rows_major=False):
    from localai_amd import device
    q = device.QMat.from_ggml(raw, t, rows, cols)
    y = q.matmul(device.to_device_f32(xs), rows_major=rows_major).cpu().numpy()
    q.close()
    return y


@pytest.mark.parametrize('t', TYPES)
def test_golden_matmul(golden, t):
    """The reference test-suite matmul case (64 x 512, 5 tokens, tests/test_dequant.py:160-177)."""
    raw, xs = golden[f'raw_mm_{t}'].tobytes(), golden['vectors']
    got = gpu_matmul(raw, t, 64, 512, xs)
    assert got.shape == (5, 64)
    check(got, raw, t, 64, 512, xs)
    assert normwise_rel(got, golden[f'matmul_{t}']) < MAX_REL


@pytest.mark.parametrize('t', TYPES)
@pytest.mark.parametrize('rows,tokens', [(1, 1), (200, 37), (128, 128), (300, 130), (129, 257)])
def test_ragged_tiles(t, rows, tokens):
    rng = np.random.default_rng(rows * 7 + tokens + t)
    block, _ = quant.block_layout(t)
    cols = 512 if block == 256 else 160      # Q8_0/Q4_0: 5 blocks, an odd number of 64-value units
    raw = random_ggml(rng, t, rows * cols)
    xs = rng.standard_normal((tokens, cols)).astype(np.float32)
    got = gpu_matmul(raw, t, rows, cols, xs)
    assert got.shape == (tokens, rows)
    check(got, raw, t, rows, cols, xs)


@pytest.mark.parametrize('t', (8, 12, 14))
@pytest.mark.parametrize('nblocks', (1, 3, 8, 17))
def test_k_lengths(t, nblocks):
    rng = np.random.default_rng(nblocks * 5 + t)
    block, _ = quant.block_layout(t)
    rows, cols, tokens = 96, block * nblocks, 40
    raw = random_ggml(rng, t, rows * cols)
    xs = rng.standard_normal((tokens, cols)).astype(np.float32)
    got = gpu_matmul(raw, t, rows, cols, xs)
    check(got, raw, t, rows, cols, xs)


@pytest.mark.parametrize('rows,cols,tokens', [(112, 256, 256), (113, 512, 257), (300, 160, 300), (16, 768, 600),
                                            (1000, 1024, 512), (1800, 256, 256)])
def test_q8_0_workgroup_tiles(rows, cols, tokens):
    """Q8_0 with 256 tokens or more runs on 112-row x 256-token workgroup
    tiles: ragged row and token edges, K padded up to whole 256-value blocks
    (cols 160), one and several tiles each way, and both output layouts."""
    rng = np.random.default_rng(rows + cols + tokens)
    raw = random_ggml(rng, 8, rows * cols)
    xs = rng.standard_normal((tokens, cols)).astype(np.float32)
    got = gpu_matmul(raw, 8, rows, cols, xs)
    assert got.shape == (tokens, rows)
    check(got, raw, 8, rows, cols, xs)
    if rows * tokens <= 300 * 300:
        np.testing.assert_array_equal(gpu_matmul(raw, 8, rows, cols, xs, rows_major=True), got.T)


def test_rows_major_layout_matches_reference_convention():
    """y_layout 1 is the [rows, tokens] buffer of localai_*_matmul (engine/native_quant.cpp:492)."""
    rng = np.random.default_rng(11)
    raw = random_ggml(rng, 8, 70 * 256)
    xs = rng.standard_normal((9, 256)).astype(np.float32)
    a = gpu_matmul(raw, 8, 70, 256, xs)
    b = gpu_matmul(raw, 8, 70, 256, xs, rows_major=True)
    assert b.shape == (70, 9)
    np.testing.assert_array_equal(a, b.T)


def test_token_rows_of_very_different_magnitude():
    """Each token row gets its own power-of-two scale into f16 range, so rows
    far outside f16's range (1e6, 1e-7) keep full relative accuracy."""
    rng = np.random.default_rng(5)
    rows, cols = 64, 512
    raw = random_ggml(rng, 12, rows * cols)
    xs = rng.standard_normal((4, cols)).astype(np.float32)
    xs[1] *= 1e6
    xs[2] *= 1e-7
    xs[3, :] = 0.0
    got = gpu_matmul(raw, 12, rows, cols, xs)
    ref = quant.matmul_exact(raw, 12, rows, cols, xs)
    w = quant.dequantize(raw, 12, (rows, cols)).astype(np.float64)
    absdot = np.abs(xs.astype(np.float64)) @ np.abs(w).T
    for r in range(3):
        assert normwise_rel(got[r], ref[r]) < MAX_REL
        assert np.all(np.abs(got[r] - ref[r]) <= MAX_REL * absdot[r])
    assert np.all(got[3] == 0.0)


def test_q8_0_prefill_shape_sampled_rows():
    """The Q8_0 prefill workload at full size (512 tokens x 4096 -> 14336 rows):
    every output is computed on the GPU; rows sampled every 97 are checked
    against the fp64 oracle, and all outputs must be finite."""
    from localai_amd import device
    from localai_amd import synth
    rows, cols, tokens = 14336, 4096, 512
    raw = synth.quant_tensor(np.random.default_rng(3), 8, rows, cols)
    xs = np.random.default_rng(4).standard_normal((tokens, cols)).astype(np.float32)
    q = device.QMat.from_ggml(raw, 8, rows, cols)
    got = q.matmul(device.to_device_f32(xs)).cpu().numpy()
    q.close()
    assert np.all(np.isfinite(got))
    sample = np.arange(0, rows, 97)
    _, bpb = quant.block_layout(8)
    row_bytes = cols // 32 * bpb
    buf = np.frombuffer(raw, dtype=np.uint8).reshape(rows, row_bytes)[sample]
    check(got[:, sample], buf.tobytes(), 8, len(sample), cols, xs)
