"""The K-quant block quantizers on the GPU (levo_hip_quantize_chunk and
levo_hip_quantize_rows for Q4_K / Q5_K / Q6_K) against the oracle's
restatement of ggml's quantize_row_q{4,5,6}_K_ref, the path of
ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, NULL) in the
conversion tool (tools/levo-quantize.cpp:355-388) for the Q4_K_M / Q5_K_M /
Q6_K profiles (src/levo-quantization.h:47-55, 96-130).

Bar: every byte equal. Shapes: LeLM medium's matrices (1536 and 8960
columns), the Flow's widths padded to 256-value blocks from F16 rows
(2200 -> 2304, 4400 -> 4608), one super-block, ragged super-block counts
per wave; blocks of zeros, constants, integer grids, outliers, sub-blocks
whose quantized scale rounds to 0 (they keep their search codes), and
sub-blocks whose values are all equal.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

Q4_K, Q5_K, Q6_K = 12, 13, 14
BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}
KQ = [Q4_K, Q5_K, Q6_K]
IDS = ["q4_K", "q5_K", "q6_K"]


def _gpu_quantize(hip, dev, qtype, x):
    import torch
    rows, cols = x.shape
    n = rows * (cols // 256) * BYTES[qtype]
    out = torch.full((n + 64,), 0xAB, dtype=torch.uint8, device=dev)
    assert hip.quantize_chunk(qtype, to_dev(x, dev), out, 0, rows, cols) == n
    got = from_dev(out)
    assert np.all(got[n:] == 0xAB)  # nothing past the last block
    return got[:n]


def _check(qtype, got, want):
    bad = np.nonzero((got != want).reshape(-1, BYTES[qtype]).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} of {want.size // BYTES[qtype]} super-blocks differ, first {bad[:8]}"


def special_rows(cols=1024):
    rng = np.random.default_rng(77)
    x = (rng.standard_normal((12, cols)) * 0.02).astype(np.float32)
    x[0] = 0.0
    x[1] = 0.25                                                     # constant: max == min in every sub-block
    x[2] = np.tile(np.arange(32, dtype=np.float32) % 16, cols // 32)  # integer grid 0..15
    x[3] = np.tile(np.arange(32, dtype=np.float32) - 16, cols // 32)  # integer grid -16..15
    x[4, ::61] = 3.0                                                # outliers
    x[5] += 0.1                                                     # all-positive sub-blocks
    x[6] -= 0.1                                                     # all-negative
    x[7, :256] *= np.repeat(np.geomspace(1e-5, 1.0, 16), 16).astype(np.float32)  # quantized scales 0
    x[8, :256] *= np.repeat(np.geomspace(1e-5, 1.0, 8), 32).astype(np.float32)
    x[9, 32:64] = 0.0                                               # one empty sub-block
    x[10] = np.float32(1e-20) * rng.standard_normal(cols).astype(np.float32)  # tiny values
    x[11, 5] = -1e4                                                 # a large negative extreme
    return x


@pytest.mark.parametrize("qtype", KQ, ids=IDS)
@pytest.mark.parametrize("rows,cols", [(1, 256), (3, 512), (9, 1536), (33, 1536), (4, 8960), (65, 256)])
def test_gaussian_rows_bit_exact(hip, dev, oracle, qtype, rows, cols):
    x = (oracle.gaussian(rows * cols, 300 + rows + cols) * 0.02).reshape(rows, cols)
    _check(qtype, _gpu_quantize(hip, dev, qtype, x), oracle.quantize(qtype, x))


@pytest.mark.parametrize("qtype", KQ, ids=IDS)
def test_special_blocks_bit_exact(hip, dev, oracle, qtype):
    x = special_rows()
    _check(qtype, _gpu_quantize(hip, dev, qtype, x), oracle.quantize(qtype, x))


@pytest.mark.parametrize("qtype,src_cols,dst_cols", [(Q4_K, 2200, 2304), (Q5_K, 2200, 2304), (Q6_K, 4400, 4608),
                                                     (Q4_K, 1536, 1536)])
def test_padded_f16_rows(hip, dev, oracle, qtype, src_cols, dst_cols):
    """write_tensor's chunk path: F16 rows widened exactly and zero-padded to
    the storage width (src/levo-quantization.h:127-130)."""
    import torch
    rows = 17
    xh = oracle.f32_to_f16((oracle.gaussian(rows * src_cols, 900 + src_cols) * 0.02).reshape(rows, src_cols))
    n = rows * (dst_cols // 256) * BYTES[qtype]
    out = torch.empty(n, dtype=torch.uint8, device=dev)
    assert hip.quantize_rows(qtype, to_dev(xh.view(np.int16), dev), 1, src_cols, src_cols, out, rows, dst_cols) == n
    _check(qtype, from_dev(out), oracle.quantize_f16_padded(qtype, xh, dst_cols))


def test_chunk_start_offsets_rows(hip, dev, oracle):
    """start is a row boundary: the chunk lands at start / n_per_row rows in."""
    import torch
    cols = 512
    x = (oracle.gaussian(6 * cols, 41) * 0.02).reshape(6, cols)
    want = oracle.quantize(Q4_K, x)
    out = torch.zeros(want.size, dtype=torch.uint8, device=dev)
    xd = to_dev(x, dev)
    row = 2 * BYTES[Q4_K]
    assert hip.quantize_chunk(Q4_K, xd, out, 2 * cols, 3, cols) == 3 * row
    got = from_dev(out)
    assert np.array_equal(got[2 * row:5 * row], want[2 * row:5 * row])
    assert not got[:2 * row].any() and not got[5 * row:].any()


def test_rejects_bad_arguments(hip, dev, binding):
    import torch
    x = torch.zeros(512, device=dev)
    out = torch.empty(4096, dtype=torch.uint8, device=dev)
    with pytest.raises(binding.LevoHipError, match="multiple of 256"):
        hip.quantize_chunk(Q4_K, x, out, 0, 1, 384)
    with pytest.raises(binding.LevoHipError, match="importance matrix"):
        hip.quantize_chunk(Q6_K, x, out, 0, 1, 256, imatrix=x)
    with pytest.raises(binding.LevoHipError, match="multiple of 256"):
        hip.quantize_rows(Q5_K, x, 0, 200, 200, out, 1, 224)


def test_non_finite_and_extreme_blocks_bit_exact(hip, dev, oracle):
    """Sub-blocks holding NaN, +-inf or values at the F16 range's ends: the
    search's codes come from ggml's integer rounding (nearest_int's 1.5 * 2^23
    addition) on every input, including where that is not a rounding of its
    argument; the kernels' float code form must not be taken there."""
    rng = np.random.default_rng(91)
    cols = 1024
    x = (rng.standard_normal((10, cols)) * 0.02).astype(np.float32)
    x[0, 3] = np.nan
    x[1, 40] = np.inf
    x[2, 7] = -np.inf
    x[3, :32] = 60000.0
    x[3, 5] = -60000.0
    x[4, 100] = 65504.0
    x[5, ::37] = np.nan
    x[6, 256:512] = np.inf
    x[7, 300] = 3e38          # finite, with squares that overflow
    x[8, :16] = -65504.0
    x[9, 17] = 1e-30
    for qtype in KQ:
        _check(qtype, _gpu_quantize(hip, dev, qtype, x), oracle.quantize(qtype, x))
