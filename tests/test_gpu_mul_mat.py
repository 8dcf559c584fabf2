"""Q8_0 decode mat-vec (levo_hip_quantize_chunk of the activations, then
levo_hip_mul_mat_q8_0) against the oracle's restatement of ggml's CPU
mul_mat for a Q8_0 weight (activation quantized with the reference
quantizer, ggml_vec_dot_q8_0_q8_0 per row).

Bars: F32 max|a - b| / max(|b|, 1) <= 1e-5 (the kernel sums the same block
terms in another order); bit-exact where every term and partial sum is an
exact integer (d = 1 blocks). Shapes: LeLM medium's decode matrices
(1536 / 8960 / 16385 rows, K 1536 and 8960), the Flow's padded K = 2208,
ragged row counts, one block per row, up to 8 activation columns, a y
pitch, and matrices whose byte size is not a multiple of 16 (the
half-word tail path).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _run(hip, dev, wb, x, rows, k, *, y_pitch=None):
    import torch
    n_vec = x.shape[0]
    yp = y_pitch or rows
    xd = to_dev(np.ascontiguousarray(x, np.float32), dev)
    xb = torch.empty(n_vec * (k // 32) * 34, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(8, xd, xb, 0, n_vec, k)
    y = torch.full((n_vec * yp,), float("nan"), dtype=torch.float32, device=dev)
    w = to_dev(wb, dev)
    hip.mul_mat_q8_0(w, xb, y, yp, rows, k, n_vec)
    return from_dev(y).reshape(n_vec, yp)[:, :rows]


def _case(oracle, rows, k, n_vec, seed):
    w = (oracle.gaussian(rows * k, seed) * np.float32(0.02)).reshape(rows, k)
    x = oracle.gaussian(n_vec * k, seed + 1).reshape(n_vec, k)
    return oracle.quantize(8, w), x


@pytest.mark.parametrize("rows,k,n_vec", [
    (1536, 1536, 2),    # attention projections, CFG pair
    (8960, 1536, 2),    # ffn gate / up
    (1536, 8960, 2),    # ffn down: rows streamed in 256-block pieces
    (16385, 1536, 1),   # one codebook head
    (2200, 2208, 2),    # Flow's padded hidden (K = 2208: 69 blocks)
    (4400, 4416, 1),    # Flow's padded intermediate
    (4096, 1536, 8),
])
def test_matches_oracle(hip, dev, oracle, rows, k, n_vec):
    wb, x = _case(oracle, rows, k, n_vec, rows + k)
    got = _run(hip, dev, wb, x, rows, k)
    want = oracle.mul_mat_q8_0(wb, x, rows, k)
    assert f32_err(got, want) <= 1e-5


@pytest.mark.parametrize("rows,k,n_vec", [(1, 32, 2), (3, 32, 2), (5, 64, 2), (17, 1536, 2), (63, 2048, 2),
                                          (66, 4096, 2), (2, 8960, 2), (7, 11008, 2), (33, 8960, 3), (9, 8224, 1),
                                          (5, 16416, 1), (8, 32, 8)])
def test_ragged_shapes(hip, dev, oracle, rows, k, n_vec):
    """Row counts that leave workgroups part-filled, rows split over 2 waves
    (K 8224 ... 16384) and 4 waves (K > 16384)."""
    wb, x = _case(oracle, rows, k, n_vec, 7 * rows + k)
    got = _run(hip, dev, wb, x, rows, k)
    want = oracle.mul_mat_q8_0(wb, x, rows, k)
    assert f32_err(got, want) <= 1e-5


def test_y_pitch(hip, dev, oracle):
    rows, k = 300, 1536
    wb, x = _case(oracle, rows, k, 3, 99)
    want = oracle.mul_mat_q8_0(wb, x, rows, k)
    got = _run(hip, dev, wb, x, rows, k, y_pitch=rows + 5)
    assert f32_err(got, want) <= 1e-5


def test_integer_blocks_bit_exact(hip, dev, oracle):
    """d = 1 blocks (largest |value| 127): every term and sum is an exact
    integer, so any summation order gives the exact product."""
    rng = np.random.default_rng(11)
    rows, k, n_vec = 777, 2048, 2
    w = rng.integers(-127, 128, (rows, k)).astype(np.float32)
    x = rng.integers(-127, 128, (n_vec, k)).astype(np.float32)
    w[:, ::32] = 127.0
    x[:, 3::32] = -127.0
    wb = oracle.quantize(8, w)
    got = _run(hip, dev, wb, x, rows, k)
    want = (w.astype(np.int64) @ x.astype(np.int64).T).T.astype(np.float32)
    assert np.array_equal(got, want)
    assert np.array_equal(oracle.mul_mat_q8_0(wb, x, rows, k), want)


def test_activation_special_values(hip, dev, oracle):
    """Zero blocks (d = 0), tiny blocks (1/d overflows) and ties of x * id at
    k + 0.5 quantize as the reference quantizer does."""
    rows, k = 64, 256
    wb, x = _case(oracle, rows, k, 2, 5)
    x[0, :32] = 0.0
    x[0, 32:64] = 1e-41
    x[1, 64:96] = np.arange(32, dtype=np.float32) - 15.5   # amax 16.5 -> id = 127/16.5
    x[1, 96:128] = np.float32(127.0) * (np.arange(32) % 3 - 1) + np.float32(0.5) * (np.arange(32) % 2)
    got = _run(hip, dev, wb, x, rows, k)
    want = oracle.mul_mat_q8_0(wb, x, rows, k)
    assert f32_err(got, want) <= 1e-5


def test_rejects_bad_arguments(hip, dev, binding):
    import torch
    w = torch.zeros(34 * 4, dtype=torch.uint8, device=dev)
    xb = torch.zeros(34 * 2, dtype=torch.uint8, device=dev)
    y = torch.zeros(8, dtype=torch.float32, device=dev)
    with pytest.raises(binding.LevoHipError, match="multiple of 32"):
        hip.mul_mat_q8_0(w, xb, y, 8, 2, 48, 1)
    with pytest.raises(binding.LevoHipError, match="at most 8"):
        hip.mul_mat_q8_0(w, xb, y, 8, 2, 64, 9)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.mul_mat_q8_0(w.data_ptr() + 2, xb, y, 8, 2, 64, 1)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.mul_mat_q8_0(w, xb.data_ptr() + 2, y, 8, 2, 64, 1)
    with pytest.raises(binding.LevoHipError, match="too large"):
        hip.mul_mat_q8_0(w, xb, y, 8, 2, 32768, 2)


# ---- levo_hip_mul_mat_q8_0_multi: several matrices sharing the activations ------------

def _two_step(hip, dev, mats, x, k):
    """quantize_chunk + one mul_mat_q8_0 per matrix (the reference path of the
    multi call): y per matrix."""
    import torch
    n_vec = x.shape[0]
    xd = to_dev(np.ascontiguousarray(x[:, :k], np.float32), dev)
    xb = torch.empty(n_vec * (k // 32) * 34 + 16, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(8, xd, xb, 0, n_vec, k)
    out = []
    for wd, rows in mats:
        y = torch.full((n_vec * rows,), float("nan"), dtype=torch.float32, device=dev)
        hip.mul_mat_q8_0(wd, xb, y, rows, rows, k, n_vec)
        out.append(from_dev(y).reshape(n_vec, rows))
    return out, xb


def _multi(hip, dev, mats, k, n_vec, *, xb=None, x=None, pitch_pad=0):
    import torch
    ys, spec = [], []
    for wd, rows in mats:
        yp = rows + pitch_pad
        y = torch.full((n_vec * yp,), float("nan"), dtype=torch.float32, device=dev)
        ys.append((y, yp, rows))
        spec.append((wd, y, yp, rows))
    if x is not None:
        xp = x.shape[1]
        xd = to_dev(np.ascontiguousarray(x, np.float32), dev)
        hip.mul_mat_q8_0_multi(spec, k, n_vec, x=xd, x_pitch=xp)
    else:
        hip.mul_mat_q8_0_multi(spec, k, n_vec, x_blocks=xb)
    return [from_dev(y).reshape(n_vec, yp)[:, :rows] for y, yp, rows in ys]


def _bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


@pytest.mark.parametrize("k,n_vec,rows", [
    (1536, 2, (1536, 1536, 1536)),   # a decode layer's q / k / v
    (1536, 2, (8960, 8960)),         # gate / up
    (1536, 2, (1536, 17, 5, 300)),   # ragged matrices, four at once
    (4096, 2, (66, 129)),            # 256 activation blocks: the largest fused quantization
    (2208, 1, (2200, 33)),           # the Flow's padded K
    (64, 8, (3, 9)),
])
def test_multi_equals_separate_calls(hip, dev, oracle, k, n_vec, rows):
    """Each matrix's y equals quantize_chunk + mul_mat_q8_0 bit for bit, with
    the activations passed quantized or in F32 (quantized in the launch)."""
    x = oracle.gaussian(n_vec * k, 3 * k + n_vec).reshape(n_vec, k)
    mats = []
    for i, r in enumerate(rows):
        wb = oracle.quantize(8, (oracle.gaussian(r * k, 11 * r + i) * np.float32(0.02)).reshape(r, k))
        mats.append((to_dev(wb, dev), r))
    want, xb = _two_step(hip, dev, mats, x, k)
    for got in (_multi(hip, dev, mats, k, n_vec, xb=xb), _multi(hip, dev, mats, k, n_vec, x=x)):
        for g, w in zip(got, want):
            assert _bits_equal(g, w)


def test_multi_wide_k_from_blocks(hip, dev, oracle):
    """K = 8960 (rows split over 4 waves) with quantized activations."""
    k, n_vec = 8960, 2
    x = oracle.gaussian(n_vec * k, 77).reshape(n_vec, k)
    mats = []
    for i, r in enumerate((1536, 7)):
        wb = oracle.quantize(8, (oracle.gaussian(r * k, 90 + i) * np.float32(0.02)).reshape(r, k))
        mats.append((to_dev(wb, dev), r))
    want, xb = _two_step(hip, dev, mats, x, k)
    for g, w in zip(_multi(hip, dev, mats, k, n_vec, xb=xb), want):
        assert _bits_equal(g, w)


@pytest.mark.parametrize("k,n_vec", [(256, 2), (4096, 2)])
def test_multi_fused_quantization_special_values_and_pitch(hip, dev, oracle, k, n_vec):
    """Zero blocks, tiny blocks (1/d overflows), ties at k + 0.5, NaN and inf
    quantize in the launch as levo_hip_quantize_chunk does, with two lanes
    per block (16 blocks) and one lane per block (256 blocks); rows of x and
    y with a pitch; a matrix of zero rows is skipped."""
    import torch
    x = oracle.gaussian(n_vec * k, 5).reshape(n_vec, k)
    x[0, :32] = 0.0
    x[0, 32:64] = 1e-41
    x[1, 64:96] = np.arange(32, dtype=np.float32) - 15.5
    x[1, 96:128] = np.float32(127.0) * (np.arange(32) % 3 - 1) + np.float32(0.5) * (np.arange(32) % 2)
    x[0, 130] = np.nan
    x[1, 200] = np.inf
    x[1, 160] = np.nan   # a block's first value: the index-order MAX restarts after it
    x[0, 180] = np.nan   # in the second half of a block (the other lane of a pair)
    x[1, 250] = np.nan
    xp = np.zeros((n_vec, k + 12), np.float32)
    xp[:, :k] = x
    mats = [(to_dev(oracle.quantize(8, (oracle.gaussian(r * k, r) * np.float32(0.02)).reshape(r, k)), dev), r)
            for r in (64, 13)]
    want, _ = _two_step(hip, dev, mats, xp, k)
    got = _multi(hip, dev, mats, k, n_vec, x=xp, pitch_pad=3)
    for g, w in zip(got, want):
        assert _bits_equal(g, w)
    empty = torch.zeros(16, dtype=torch.uint8, device=dev)
    y = torch.zeros(4, dtype=torch.float32, device=dev)
    hip.mul_mat_q8_0_multi([(empty, y, 1, 0)], k, n_vec, x=to_dev(xp, dev), x_pitch=k + 12)


def test_multi_rejects_bad_arguments(hip, dev, binding):
    import torch
    w = torch.zeros(34 * 8 * 4, dtype=torch.uint8, device=dev)
    xb = torch.zeros(34 * 16, dtype=torch.uint8, device=dev)
    x = torch.zeros((2, 8960), dtype=torch.float32, device=dev)
    y = torch.zeros(64, dtype=torch.float32, device=dev)
    m = [(w, y, 4, 4)]
    with pytest.raises(binding.LevoHipError, match="1 to 4 matrices"):
        hip.mul_mat_q8_0_multi([], 256, 2, x_blocks=xb)
    with pytest.raises(binding.LevoHipError, match="1 to 4 matrices"):
        hip.mul_mat_q8_0_multi(m * 5, 256, 2, x_blocks=xb)
    with pytest.raises(binding.LevoHipError, match="exactly one"):
        hip.mul_mat_q8_0_multi(m, 256, 2)
    with pytest.raises(binding.LevoHipError, match="exactly one"):
        hip.mul_mat_q8_0_multi(m, 256, 2, x_blocks=xb, x=x, x_pitch=8960)
    with pytest.raises(binding.LevoHipError, match="<= 256 blocks"):
        hip.mul_mat_q8_0_multi(m, 8960, 2, x=x, x_pitch=8960)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned rows"):
        hip.mul_mat_q8_0_multi(m, 256, 2, x=x.data_ptr() + 4, x_pitch=8960)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned rows"):
        hip.mul_mat_q8_0_multi(m, 256, 2, x=x, x_pitch=258)
    with pytest.raises(binding.LevoHipError, match="y pitch"):
        hip.mul_mat_q8_0_multi([(w, y, 3, 4)], 256, 2, x=x, x_pitch=8960)
    with pytest.raises(binding.LevoHipError, match="multiple of 32"):
        hip.mul_mat_q8_0_multi(m, 48, 2, x_blocks=xb)
