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
