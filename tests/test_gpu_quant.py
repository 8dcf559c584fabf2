"""Q8_0 / Q4_0 quantize and dequantize on the GPU vs the oracle's restatement
of ggml's reference quantizers (ggml_quantize_chunk, tools/levo-quantize.cpp:386-388).

Bar: quantized blocks bit-exact (memcmp); dequantized values bit-exact (the
products are exact in F32); F16 dequantization is the RNE rounding of them.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

Q8, Q4 = 8, 2
BB = {Q8: 34, Q4: 18}


def _quant_f16(hip, dev, qt, xh, dst_cols=None):
    import torch
    rows, cols = xh.shape
    dst_cols = dst_cols or cols
    out = torch.empty(rows * (dst_cols // 32) * BB[qt], dtype=torch.uint8, device=dev)
    n = hip.quantize_rows(qt, to_dev(xh.view(np.int16), dev), 1, cols, cols, out, rows, dst_cols)
    assert n == out.numel()
    return from_dev(out)


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
def test_config_weights_bit_exact(hip, dev, oracle, qt):
    """F16 weights [4096, 1536] ~N(0, 0.02), 196,608 blocks."""
    xh = oracle.f32_to_f16((oracle.gaussian(4096 * 1536, 1500) * 0.02).reshape(4096, 1536))
    got = _quant_f16(hip, dev, qt, xh)
    want = oracle.quantize_f16_padded(qt, xh, 1536)
    assert np.array_equal(got, want), np.count_nonzero(got != want)


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
def test_quantize_chunk_f32_with_start(hip, dev, oracle, qt):
    import torch
    rows, cols = 40, 2208
    x = (oracle.gaussian(rows * cols, 1600) * 0.5).reshape(rows, cols)
    out = torch.zeros(rows * (cols // 32) * BB[qt], dtype=torch.uint8, device=dev)
    xd = to_dev(x, dev)
    n1 = hip.quantize_chunk(qt, xd, out, 0, 17, cols)
    n2 = hip.quantize_chunk(qt, xd, out, 17 * cols, rows - 17, cols)
    row_size = hip.row_size(qt, cols)
    assert n1 == 17 * row_size and n2 == (rows - 17) * row_size
    assert np.array_equal(from_dev(out), oracle.quantize(qt, x))


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
def test_padded_rows_flow_hidden(hip, dev, oracle, qt):
    """write_tensor zero-pads 2200 -> 2208 columns (src/levo-quantization.h:120-130)."""
    xh = oracle.f32_to_f16((oracle.gaussian(33 * 2200, 1700) * 0.02).reshape(33, 2200))
    assert np.array_equal(_quant_f16(hip, dev, qt, xh, 2208), oracle.quantize_f16_padded(qt, xh, 2208))


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
def test_special_blocks(hip, dev, oracle, qt):
    import torch
    x = (oracle.gaussian(64 * 32, 1800) * 0.02).reshape(64, 32)
    x[0] = 0.0
    x[1] = -0.0
    x[2] = 0.0
    x[2, 0], x[2, 1], x[2, 2], x[2, 3] = 127.0, 2.5, -2.5, 0.5     # Q8_0 ties round away from zero
    x[3] = 1e-6 * np.arange(32)                                       # F16-subnormal scale
    x[4] = 0.0
    x[4, 1], x[4, 3] = -0.5, 0.5                                      # Q4_0: first of equal |x| wins
    x[5] = 3e-39 * np.arange(1, 33)                                   # F32 subnormals: 1/d overflows
    x[6] = 1e-38
    x[7, :] = np.float32(-8.0) * np.arange(32) / 31                   # exact -8 multiples
    x[8, :] = 65504.0
    x[9, 5] = 1e30                                                    # huge outlier, F16 d overflows to inf
    x[10, 5], x[10, 20] = -0.7, 0.7                                   # Q4_0: equal |x| in different 8-value quarters
    x[11, 30], x[11, 9] = -0.7, 0.7                                   # ... first one positive, later one negative
    x[12, 7], x[12, 8] = 0.7, -0.7                                    # ... at a quarter boundary
    x[13, 24], x[13, 31] = -0.7, 0.7                                  # ... both in the last quarter
    x[14, 0] = np.nan                                                 # NaN leading, tie later across quarters
    x[14, 3], x[14, 27] = -0.7, 0.7
    x[15, 6], x[15, 14], x[15, 22], x[15, 30] = 0.5, -0.6, 0.6, -0.6  # larger |x| in quarters 1, 2, 3
    out = torch.empty(64 * BB[qt], dtype=torch.uint8, device=dev)
    hip.quantize_chunk(qt, to_dev(x, dev), out, 0, 64, 32)
    got, want = from_dev(out), oracle.quantize(qt, x)
    bad = np.nonzero((got != want).reshape(64, BB[qt]).any(axis=1))[0]
    assert bad.size == 0, bad


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
@pytest.mark.parametrize("nblocks", [1, 7, 8, 9, 15, 16, 17, 100, 4099])
def test_tail_groups(hip, dev, oracle, qt, nblocks):
    import torch
    x = oracle.gaussian(nblocks * 32, 1900 + nblocks).reshape(nblocks, 32)
    xh = oracle.f32_to_f16(x)
    assert np.array_equal(_quant_f16(hip, dev, qt, xh), oracle.quantize_f16_padded(qt, xh, 32))
    out = torch.full((nblocks * BB[qt] + 64,), 0xAB, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(qt, to_dev(x, dev), out, 0, nblocks, 32)
    got = from_dev(out)
    assert np.array_equal(got[: nblocks * BB[qt]], oracle.quantize(qt, x))
    assert np.all(got[nblocks * BB[qt]:] == 0xAB)  # nothing written past the last block


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
@pytest.mark.parametrize("nblocks", [1, 9, 16, 17, 196608])
def test_dequantize_bit_exact(hip, dev, oracle, qt, nblocks):
    import torch
    x = (oracle.gaussian(nblocks * 32, 2000 + nblocks) * 0.02).astype(np.float32)
    q = oracle.quantize(qt, x.reshape(nblocks, 32))
    want = oracle.dequantize(qt, q, x.size)
    qd = to_dev(q, dev)
    y = torch.full((x.size + 8,), 3.0, dtype=torch.float32, device=dev)
    hip.dequantize(qt, qd, y, 0, x.size)
    got = from_dev(y)
    assert np.array_equal(got[: x.size].view(np.uint32), want.view(np.uint32))
    assert np.all(got[x.size:] == 3.0)
    h = torch.empty(x.size, dtype=torch.int16, device=dev)
    hip.dequantize(qt, qd, h, 1, x.size)
    assert np.array_equal(from_dev(h).view(np.uint16), want.astype(np.float16).view(np.uint16))


def test_reference_padded_q8_product(hip, dev):
    """tests/test-quantization.cpp:46-75 through the GPU quantizer and dequantizer."""
    import torch
    m = np.zeros((4, 32), np.float32)
    for r in range(4):
        for c in range(6):
            m[r, c] = 0.03125 * (r + 1) * (c + 1)
    q = torch.empty(4 * 34, dtype=torch.uint8, device=dev)
    assert hip.quantize_chunk(Q8, to_dev(m, dev), q, 0, 4, 32) == 4 * 34
    y = torch.empty(128, dtype=torch.float32, device=dev)
    hip.dequantize(Q8, q, y, 0, 128)
    deq = from_dev(y).reshape(4, 32)
    inp = np.zeros(32, np.float32)
    inp[:6] = [0.25, -0.5, 0.75, -1.0, 1.25, -1.5]
    assert np.all(np.abs(deq @ inp - m @ inp) < 0.015)


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
def test_unaligned_buffers(hip, dev, oracle, qt):
    """ggml_quantize_chunk with start > 0 writes at start_row * row_size: 2-byte aligned only."""
    import torch
    nblocks = 1000
    x = (oracle.gaussian(nblocks * 32, 2100) * 0.1).reshape(nblocks, 32)
    want = oracle.quantize(qt, x)
    buf = torch.zeros(nblocks * BB[qt] + 16, dtype=torch.uint8, device=dev)
    hip.quantize_chunk(qt, to_dev(x, dev), buf[2:], 0, nblocks, 32)
    got = from_dev(buf)
    assert np.array_equal(got[2: 2 + nblocks * BB[qt]], want)
    assert np.all(got[:2] == 0) and np.all(got[2 + nblocks * BB[qt]:] == 0)
    src = torch.zeros(want.size + 16, dtype=torch.uint8, device=dev)
    src[6: 6 + want.size] = to_dev(want, dev)
    y = torch.full((nblocks * 32 + 8,), 5.0, dtype=torch.float32, device=dev)
    hip.dequantize(qt, src[6:], y[1:], 0, nblocks * 32)
    yd = from_dev(y)
    assert np.array_equal(yd[1: 1 + nblocks * 32], oracle.dequantize(qt, want, nblocks * 32))
    assert yd[0] == 5.0 and np.all(yd[1 + nblocks * 32:] == 5.0)


@pytest.mark.parametrize("qt", [Q8, Q4], ids=["q8_0", "q4_0"])
@pytest.mark.parametrize("dense", [True, False], ids=["packed", "padded"])
def test_non_finite_blocks_follow_the_reference_scan(hip, dev, oracle, qt, dense):
    """NaN and +-inf inside blocks. ggml's Q8_0 max is MAX(amax, fabsf(v))
    applied in index order, so a NaN forgets every earlier value and a NaN in
    the last slot makes d NaN; Q4_0's `amax < fabsf(v)` never picks a NaN.
    The oracle restates that order; both the packed-row kernel and the padded
    (strided) kernel must reproduce it byte for byte."""
    import torch
    nb = 40
    x = (oracle.gaussian(nb * 32, 2100) * 0.5).reshape(nb, 32)
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    x[0, 0] = nan                       # NaN first
    x[1, 17] = nan                      # NaN in the middle: earlier maxima forgotten
    x[2, 31] = nan                      # NaN last: d = NaN
    x[3, :] = nan                       # all NaN
    x[4, 9] = inf                       # +inf: d = inf, id = 0
    x[5, 3] = -inf
    x[6, 4], x[6, 20] = nan, inf
    x[7, 12], x[7, 30] = inf, nan
    x[8, :16] = nan                     # NaN run then finite values
    x[9, 5], x[9, 6] = -inf, inf
    want = oracle.quantize(qt, x)
    if dense:
        out = torch.empty(nb * BB[qt], dtype=torch.uint8, device=dev)
        hip.quantize_chunk(qt, to_dev(x, dev), out, 0, nb, 32)
        got = from_dev(out)
    else:
        # the same blocks as rows of 32 values stored 40 floats apart
        src = np.zeros((nb, 40), np.float32)
        src[:, :32] = x
        out = torch.empty(nb * BB[qt], dtype=torch.uint8, device=dev)
        n = hip.quantize_rows(qt, to_dev(src, dev), 0, 32, 40, out, nb, 32)
        assert n == out.numel()
        got = from_dev(out)
    bad = np.nonzero((got != want).reshape(nb, BB[qt]).any(axis=1))[0]
    assert bad.size == 0, bad
