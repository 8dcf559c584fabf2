"""Packed Q8_0 decode mat-vec: levo_hip_repack_q8_0 (the weights rearranged
once at load), levo_hip_quantize_q8_0_columns (the activations quantized to
the form the mat-vec keeps in LDS) and levo_hip_mul_mat_q8_0_packed /
_packed_multi.

Bars: the repacked bytes and the columns equal the layouts' definitions
applied to the oracle's Q8_0 blocks byte for byte; y equals the block-layout
entry points' y on the original blocks bit for bit (the same terms summed in
the same order), and is within 1e-5 of the oracle's restatement of ggml's
CPU mul_mat (the block-layout tests' bar). Shapes cover every geometry and
blocks-per-lane instance: 16 lanes per row with 1-4 blocks per lane (K 32 ..
2048), 32 lanes (K 2080 .. 4096), 64 lanes (K 4128 .. 8192), rows over two
waves (K 8224 .. 16384) and four (K 16416 and up), with ragged row counts.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _packed_layout(blocks: np.ndarray, rows: int, k: int) -> np.ndarray:
    """The packed matrix from its definition: per row the first 16 quants of
    every block, then the last 16; the F16 scales of all rows after them."""
    nb = k // 32
    b = blocks.reshape(rows, nb, 34)
    q = b[:, :, 2:]
    quants = np.concatenate([q[:, :, :16].reshape(rows, -1), q[:, :, 16:].reshape(rows, -1)], axis=1)
    return np.concatenate([quants.reshape(-1), b[:, :, :2].reshape(-1)])


def _columns_layout(blocks: np.ndarray, n_vec: int, k: int) -> np.ndarray:
    """Columns from their definition: the quants in value order, then the
    scales widened to F32."""
    b = blocks[:n_vec * (k // 32) * 34].reshape(-1, 34)
    scales = b[:, :2].copy().view(np.float16).reshape(-1).astype(np.float32)
    return np.concatenate([b[:, 2:].reshape(-1), scales.view(np.uint8)])


def _bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


def _case(oracle, rows, k, n_vec, seed):
    w = (oracle.gaussian(rows * k, seed) * np.float32(0.02)).reshape(rows, k)
    x = oracle.gaussian(n_vec * k, seed + 1).reshape(n_vec, k)
    return oracle.quantize(8, w), x


def _both(hip, dev, wb, x, rows, k, y_pitch=None):
    """(block-layout y, packed y, packed matrix, columns) on the same inputs."""
    import torch
    n_vec = x.shape[0]
    yp = y_pitch or rows
    xd = to_dev(np.ascontiguousarray(x, np.float32), dev)
    xb = torch.empty(n_vec * (k // 32) * 34 + 16, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(8, xd, xb, 0, n_vec, k)
    xc = torch.empty(n_vec * (k // 32) * 36, dtype=torch.uint8, device=dev)
    hip.quantize_q8_0_columns(xd, k, xc, n_vec, k)
    w = to_dev(wb, dev)
    pk = torch.empty_like(w)
    hip.repack_q8_0(w, pk, rows, k)
    y0 = torch.full((n_vec * yp,), float("nan"), dtype=torch.float32, device=dev)
    y1 = torch.full((n_vec * yp,), float("nan"), dtype=torch.float32, device=dev)
    hip.mul_mat_q8_0(w, xb, y0, yp, rows, k, n_vec)
    hip.mul_mat_q8_0_packed(pk, xc, y1, yp, rows, k, n_vec)
    y0 = from_dev(y0).reshape(n_vec, yp)
    y1 = from_dev(y1).reshape(n_vec, yp)
    return y0, y1, from_dev(pk), from_dev(xc), from_dev(xb)


@pytest.mark.parametrize("rows,k,n_vec", [
    (1536, 1536, 2),    # attention projections, CFG pair (16 lanes, 3 blocks each)
    (8960, 1536, 2),    # ffn gate / up
    (1536, 8960, 2),    # ffn down (two waves per row, 3 blocks per lane)
    (16385, 1536, 1),   # one codebook head
    (2200, 2208, 2),    # Flow's padded hidden (69 blocks: 32 lanes, 3 blocks)
])
def test_lelm_shapes_match_blocks_and_oracle(hip, dev, oracle, rows, k, n_vec):
    wb, x = _case(oracle, rows, k, n_vec, rows + 3 * k)
    y0, y1, pk, xc, xb = _both(hip, dev, wb, x, rows, k)
    assert np.array_equal(pk, _packed_layout(wb, rows, k))
    assert np.array_equal(xc, _columns_layout(xb, n_vec, k))
    assert _bits_equal(y1, y0)
    assert f32_err(y1, oracle.mul_mat_q8_0(wb, x, rows, k)) <= 1e-5


@pytest.mark.parametrize("rows,k,n_vec", [
    (1, 32, 2), (3, 512, 2), (17, 1024, 3), (5, 2048, 8),              # 16 lanes, 1 / 2 / 3 / 4 blocks
    (33, 2080, 2), (66, 4096, 2),                                      # 32 lanes, 3 / 4
    (9, 4128, 1), (70, 8192, 2),                                       # 64 lanes, 3 / 4
    (2, 8224, 2), (7, 8960, 3), (3, 16384, 1),                         # two waves per row
    (5, 16416, 1), (2, 26624, 1), (7, 11008, 2),                       # four waves per row
])
def test_every_geometry_equals_blocks(hip, dev, oracle, rows, k, n_vec):
    wb, x = _case(oracle, rows, k, n_vec, 7 * rows + k)
    y0, y1, pk, _, _ = _both(hip, dev, wb, x, rows, k, y_pitch=rows + 3)
    assert np.array_equal(pk, _packed_layout(wb, rows, k))
    assert _bits_equal(y1[:, :rows], y0[:, :rows])
    assert np.all(np.isnan(y1[:, rows:]))  # nothing written past the rows
    assert f32_err(y1[:, :rows], oracle.mul_mat_q8_0(wb, x, rows, k)) <= 1e-5


def test_integer_blocks_bit_exact(hip, dev, oracle):
    """d = 1 blocks: every term and partial sum is an exact integer."""
    rng = np.random.default_rng(12)
    rows, k, n_vec = 301, 8960, 2
    w = rng.integers(-127, 128, (rows, k)).astype(np.float32)
    x = rng.integers(-127, 128, (n_vec, k)).astype(np.float32)
    w[:, ::32] = 127.0
    x[:, 5::32] = -127.0
    wb = oracle.quantize(8, w)
    _, y1, _, _, _ = _both(hip, dev, wb, x, rows, k)
    want = (w.astype(np.int64) @ x.astype(np.int64).T).T.astype(np.float32)
    assert np.array_equal(y1, want)


def test_columns_special_values(hip, dev, oracle):
    """Zero blocks, tiny blocks (1/d overflows), ties at k + 0.5, NaN and inf
    give the columns of levo_hip_quantize_chunk's blocks; rows of x with a
    pitch."""
    import torch
    k, n_vec = 256, 3
    x = oracle.gaussian(n_vec * k, 8).reshape(n_vec, k)
    x[0, :32] = 0.0
    x[0, 32:64] = 1e-41
    x[1, 64:96] = np.arange(32, dtype=np.float32) - 15.5
    x[1, 96:128] = np.float32(127.0) * (np.arange(32) % 3 - 1) + np.float32(0.5) * (np.arange(32) % 2)
    x[2, 130] = np.nan
    x[2, 200] = np.inf
    xp = np.zeros((n_vec, k + 20), np.float32)
    xp[:, :k] = x
    xd = to_dev(xp, dev)
    xc = torch.empty(n_vec * (k // 32) * 36, dtype=torch.uint8, device=dev)
    hip.quantize_q8_0_columns(xd, k + 20, xc, n_vec, k)
    blocks = oracle.quantize(8, x)
    assert np.array_equal(from_dev(xc), _columns_layout(blocks, n_vec, k))


@pytest.mark.parametrize("k,n_vec,rows", [
    (1536, 2, (1536, 1536, 1536)),   # a decode layer's q / k / v
    (1536, 2, (8960, 8960)),         # gate / up
    (1536, 2, (1536, 17, 5, 300)),   # ragged matrices, four at once
    (4096, 2, (66, 129)),            # 256 activation blocks: the largest fused quantization
    (8960, 2, (1536, 7)),            # columns only (560 blocks)
    (64, 8, (3, 9)),
])
def test_multi_equals_block_multi(hip, dev, oracle, k, n_vec, rows):
    """Each matrix's y from one packed multi launch equals the block-layout
    multi launch's, with the activations as columns or in F32."""
    import torch
    x = oracle.gaussian(n_vec * k, 5 * k + n_vec).reshape(n_vec, k)
    xd = to_dev(x, dev)
    xb = torch.empty(n_vec * (k // 32) * 34 + 16, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(8, xd, xb, 0, n_vec, k)
    xc = torch.empty(n_vec * (k // 32) * 36, dtype=torch.uint8, device=dev)
    hip.quantize_q8_0_columns(xd, k, xc, n_vec, k)
    blocks, packed, want = [], [], []
    for i, r in enumerate(rows):
        wb = oracle.quantize(8, (oracle.gaussian(r * k, 13 * r + i) * np.float32(0.02)).reshape(r, k))
        w = to_dev(wb, dev)
        pk = torch.empty_like(w)
        hip.repack_q8_0(w, pk, r, k)
        blocks.append(w)
        packed.append(pk)
    ys0 = [torch.full((n_vec * r,), float("nan"), device=dev) for r in rows]
    hip.mul_mat_q8_0_multi([(w, y, r, r) for w, y, r in zip(blocks, ys0, rows)], k, n_vec, x_blocks=xb)
    want = [from_dev(y) for y in ys0]
    forms = [dict(x_blocks=xc)]
    if n_vec * (k // 32) <= 256:
        forms.append(dict(x=xd, x_pitch=k))
    for form in forms:
        ys = [torch.full((n_vec * r,), float("nan"), device=dev) for r in rows]
        hip.mul_mat_q8_0_multi([(p, y, r, r) for p, y, r in zip(packed, ys, rows)], k, n_vec, packed=True, **form)
        for y, w in zip(ys, want):
            assert _bits_equal(from_dev(y), w)


def test_rejects_bad_arguments(hip, dev, binding):
    import torch
    w = torch.zeros(34 * 8, dtype=torch.uint8, device=dev)
    pk = torch.zeros(34 * 8, dtype=torch.uint8, device=dev)
    x = torch.zeros((2, 256), dtype=torch.float32, device=dev)
    xc = torch.zeros(36 * 16, dtype=torch.uint8, device=dev)
    y = torch.zeros(8, dtype=torch.float32, device=dev)
    with pytest.raises(binding.LevoHipError, match="multiple of 32"):
        hip.repack_q8_0(w, pk, 2, 48)
    with pytest.raises(binding.LevoHipError, match="must not overlap"):
        hip.repack_q8_0(w, w.data_ptr() + 16, 2, 64)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.repack_q8_0(w, pk.data_ptr() + 2, 2, 64)
    with pytest.raises(binding.LevoHipError, match="at most 8"):
        hip.quantize_q8_0_columns(x, 256, xc, 9, 256)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned rows"):
        hip.quantize_q8_0_columns(x, 258, xc, 2, 256)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.quantize_q8_0_columns(x, 256, xc.data_ptr() + 4, 2, 256)
    with pytest.raises(binding.LevoHipError, match="multiple of 32"):
        hip.mul_mat_q8_0_packed(pk, xc, y, 8, 2, 48, 1)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.mul_mat_q8_0_packed(pk.data_ptr() + 2, xc, y, 8, 2, 64, 1)
    with pytest.raises(binding.LevoHipError, match="too large"):
        hip.mul_mat_q8_0_packed(pk, xc, y, 8, 2, 32768, 2)
    with pytest.raises(binding.LevoHipError, match="exactly one"):
        hip.mul_mat_q8_0_multi([(pk, y, 4, 4)], 256, 2, packed=True)
    # zero rows / zero columns: nothing to do
    hip.repack_q8_0(w, pk, 0, 64)
    hip.quantize_q8_0_columns(x, 256, xc, 0, 256)
    hip.mul_mat_q8_0_packed(pk, xc, y, 8, 0, 64, 1)
