"""K-quants on the decode path (levo_hip_quantize_q8_K, levo_hip_dequantize
for Q4_K / Q5_K / Q6_K, levo_hip_mul_mat_kquant) against the oracle's
restatement of ggml's quantize_row_q8_K_ref, dequantize_row_q{4,5,6}_K and
ggml_vec_dot_q{4,5,6}_K_q8_K: the matrices of the Q6_K / Q5_K_M / Q4_K_M
profiles (src/levo-quantization.h:47-55, 96-118).

Bars: Q8_K blocks and dequantized values bit-exact (F32 and F16 outputs);
the mat-vec F32 max|a - b| / max(|b|, 1) <= 1e-5 (the kernel sums the same
block terms in another order), bit-exact where every term is an exact
integer. Shapes: LeLM medium's decode matrices (1536 / 8960 / 16385 rows,
K 1536 and 8960), the Flow's hidden and intermediate padded for 256-value
blocks (2200 -> 2304, 4400 -> 4608, src/levo-quantization.h:127-130), one
block per row, ragged rows, up to 8 activation columns, a y pitch, Q6_K rows
whose blocks start 2 bytes past a dword.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu

Q4_K, Q5_K, Q6_K = 12, 13, 14
BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210}


def random_blocks(qtype, n, rng, lo=1e-4, hi=5e-4):
    """n random blocks: random quants and scales, finite F16 d (and dmin) in [lo, hi]."""
    b = rng.integers(0, 256, (n, BYTES[qtype]), dtype=np.uint8)
    d = rng.uniform(lo, hi, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    if qtype == Q6_K:
        b[:, 208:210] = d
    else:
        b[:, 0:2] = d
        b[:, 2:4] = rng.uniform(lo, hi, n).astype(np.float16).view(np.uint8).reshape(n, 2)
    return b.ravel()


def pack_scales_k4(sc, mn):
    """[n, 8] 6-bit scales and mins -> [n, 12] packed bytes (ggml's K-quant layout)."""
    b = np.zeros((sc.shape[0], 12), np.uint8)
    for j in range(4):
        b[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        b[:, j + 4] = (mn[:, j] & 63) | ((mn[:, j + 4] >> 4) << 6)
        b[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    return b


def realistic_blocks(qtype, w):
    """Blocks of the K-quant structure for weights w [n, 256] (~N(0, 0.02)):
    per-sub-block scale (and min), 6-bit (Q6_K: int8) scales under a
    super-block d, codes rounded into range. A plain quantizer, not ggml's
    search: only the mat-vec's arithmetic is under test."""
    w = w.astype(np.float64)
    n = w.shape[0]
    if qtype == Q6_K:
        sub = w.reshape(n, 16, 16)
        scale = np.abs(sub).max(2) / 31.5 + 1e-12
        d = (scale.max(1) / 127.0).astype(np.float16)
        sc = np.clip(np.rint(scale / d.astype(np.float64)[:, None]), 1, 127).astype(np.int64)
        step = d.astype(np.float64)[:, None, None] * sc[:, :, None]
        c = (np.clip(np.rint(sub / step), -32, 31) + 32).astype(np.uint8).reshape(n, 256)
        ql = np.zeros((n, 128), np.uint8)
        qh = np.zeros((n, 64), np.uint8)
        for h in range(2):
            b = c[:, 128 * h:128 * h + 128]
            ql[:, 64 * h:64 * h + 32] = (b[:, 0:32] & 15) | ((b[:, 64:96] & 15) << 4)
            ql[:, 64 * h + 32:64 * h + 64] = (b[:, 32:64] & 15) | ((b[:, 96:128] & 15) << 4)
            qh[:, 32 * h:32 * h + 32] = ((b[:, 0:32] >> 4) | ((b[:, 32:64] >> 4) << 2) |
                                         ((b[:, 64:96] >> 4) << 4) | ((b[:, 96:128] >> 4) << 6))
        return np.concatenate([ql, qh, sc.astype(np.int8).view(np.uint8), d.view(np.uint8).reshape(n, 2)], 1).ravel()
    top = 15 if qtype == Q4_K else 31
    sub = w.reshape(n, 8, 32)
    lo = np.minimum(sub.min(2), 0.0)
    scale = (sub.max(2) - lo) / top + 1e-12
    d = (scale.max(1) / 63.0).astype(np.float16)
    dmin = (np.maximum((-lo).max(1), 1e-12) / 63.0).astype(np.float16)
    sc = np.clip(np.rint(scale / d.astype(np.float64)[:, None]), 1, 63).astype(np.int64)
    mn = np.clip(np.rint(-lo / dmin.astype(np.float64)[:, None]), 0, 63).astype(np.int64)
    step = d.astype(np.float64)[:, None, None] * sc[:, :, None]
    off = dmin.astype(np.float64)[:, None, None] * mn[:, :, None]
    c = np.clip(np.rint((sub + off) / step), 0, top).astype(np.uint8).reshape(n, 256)
    qs = np.zeros((n, 128), np.uint8)
    qh = np.zeros((n, 32), np.uint8)
    for g in range(4):
        lo4, hi4 = c[:, 64 * g:64 * g + 32], c[:, 64 * g + 32:64 * g + 64]
        qs[:, 32 * g:32 * g + 32] = (lo4 & 15) | ((hi4 & 15) << 4)
        qh |= ((lo4 >> 4) << (2 * g)).astype(np.uint8) | ((hi4 >> 4) << (2 * g + 1)).astype(np.uint8)
    head = np.concatenate([d.view(np.uint8).reshape(n, 2), dmin.view(np.uint8).reshape(n, 2),
                           pack_scales_k4(sc, mn)], 1)
    parts = [head, qs] if qtype == Q4_K else [head, qh, qs]
    return np.concatenate(parts, 1).ravel()


def q8_K_dev(hip, dev, x):
    import torch
    x = np.ascontiguousarray(x, np.float32)
    xb = torch.empty(x.size // 256 * 292, dtype=torch.uint8, device=dev)
    hip.quantize_q8_K(to_dev(x.ravel(), dev), xb, x.size)
    return xb


def test_q8_K_bit_exact(hip, dev, oracle):
    rng = np.random.default_rng(1)
    rows = [rng.standard_normal(256) * s for s in (1.0, 1e-3, 300.0, 1e-30)]
    rows.append(np.zeros(256))
    tie = rng.standard_normal(256)
    tie[[9, 77, 200]] = [-4.0, 4.0, -4.0]  # equal magnitudes: the first one is the max
    rows.append(tie)
    halves = np.arange(256) % 9 - 4.0 + 0.5  # max -127 below makes iscale 1: x.5 ties round to even
    halves[3] = -127.0
    rows.append(halves)
    big = rng.standard_normal(256)
    big[100] = 5.0e37
    rows.append(big)
    x = np.concatenate(rows).astype(np.float32)
    got = from_dev(q8_K_dev(hip, dev, x))
    want = oracle.quantize_q8_K(x)
    assert np.array_equal(got, want)
    # a long run of rows in one launch
    x = (rng.standard_normal(256 * 301) * 0.7).astype(np.float32)
    assert np.array_equal(from_dev(q8_K_dev(hip, dev, x)), oracle.quantize_q8_K(x))


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_dequantize_bit_exact(hip, dev, oracle, qtype):
    import torch
    rng = np.random.default_rng(qtype)
    nb = 37  # odd: Q6_K blocks alternate between dword-aligned and 2 bytes past
    blocks = random_blocks(qtype, nb, rng, 1e-3, 3.0)
    want = oracle.dequantize_kquant(qtype, blocks, 256 * nb)
    src = to_dev(blocks, dev)
    out = torch.full((256 * nb,), float("nan"), dtype=torch.float32, device=dev)
    hip.dequantize(qtype, src, out, 0, 256 * nb)
    assert np.array_equal(from_dev(out).view(np.uint32), want.view(np.uint32))
    out16 = torch.zeros(256 * nb, dtype=torch.float16, device=dev)
    hip.dequantize(qtype, src, out16, 1, 256 * nb)
    assert np.array_equal(from_dev(out16).view(np.uint16), want.astype(np.float16).view(np.uint16))


def _run(hip, dev, qtype, wb, x, rows, k, y_pitch=None):
    import torch
    n_vec = x.shape[0]
    yp = y_pitch or rows
    xb = q8_K_dev(hip, dev, x)
    y = torch.full((n_vec * yp,), float("nan"), dtype=torch.float32, device=dev)
    hip.mul_mat_kquant(qtype, to_dev(wb, dev), xb, y, yp, rows, k, n_vec)
    return from_dev(y).reshape(n_vec, yp)[:, :rows]


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("rows,k,n_vec", [
    (1536, 1536, 2),    # attention projections, CFG pair
    (8960, 1536, 2),    # ffn gate / up
    (1536, 8960, 2),    # ffn down (35 blocks per row)
    (16385, 1536, 1),   # one codebook head
    (6600, 2304, 2),    # Flow qkv over the padded hidden
    (2200, 4608, 1),    # Flow ffn out over the padded intermediate
    (1024, 1536, 8),
])
def test_mul_mat_matches_oracle(hip, dev, oracle, qtype, rows, k, n_vec):
    w = oracle.gaussian(rows * k, rows + k + qtype) * np.float32(0.02)
    wb = realistic_blocks(qtype, w.reshape(-1, 256))
    x = oracle.gaussian(n_vec * k, rows + n_vec).reshape(n_vec, k)
    got = _run(hip, dev, qtype, wb, x, rows, k)
    want = oracle.mul_mat_kquant(qtype, wb, x, rows, k)
    assert f32_err(got, want) <= 1e-5


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("rows,k,n_vec", [(1, 256, 1), (3, 256, 2), (7, 2304, 3), (65, 512, 2), (5, 8960, 8),
                                          (2049, 768, 2), (4095, 256, 1),  # 32 lanes per row, last workgroup short
                                          (9, 9728, 2), (11, 9984, 3), (6, 16384, 4),  # half-row instances
                                          (4097, 1536, 2), (17, 2560, 2), (13, 5120, 2)])  # the tight instances' edges
def test_mul_mat_ragged(hip, dev, oracle, qtype, rows, k, n_vec):
    w = oracle.gaussian(rows * k, 7 * rows + k + qtype) * np.float32(0.02)
    wb = realistic_blocks(qtype, w.reshape(-1, 256))
    x = oracle.gaussian(n_vec * k, rows).reshape(n_vec, k)
    got = _run(hip, dev, qtype, wb, x, rows, k, y_pitch=rows + 3)
    assert f32_err(got, oracle.mul_mat_kquant(qtype, wb, x, rows, k)) <= 1e-5


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K, Q6_K])
def test_mul_mat_integer_blocks_exact(hip, dev, oracle, qtype):
    """d_w = 1 (dmin = 1) and integer activations whose Q8_K d is exactly 1
    (max |x| = 127): every term and sum is an exact integer."""
    rng = np.random.default_rng(90 + qtype)
    rows, k = 33, 1536
    wb = random_blocks(qtype, rows * k // 256, rng).reshape(-1, BYTES[qtype])
    one = np.array([1.0], np.float16).view(np.uint8)
    if qtype == Q6_K:
        wb[:, 208:210] = one
    else:
        wb[:, 0:2] = one
        wb[:, 2:4] = one
    wb = wb.ravel()
    x = rng.integers(-127, 128, (2, k)).astype(np.float32)
    x[:, ::256] = -127.0  # each block's first extreme is -127: d = 1, quants = x
    got = _run(hip, dev, qtype, wb, x, rows, k)
    want = oracle.mul_mat_kquant(qtype, wb, x, rows, k)
    assert np.array_equal(got, want)


def test_rejects_bad_arguments(hip, dev, binding):
    import torch
    w = torch.zeros(144 * 8, dtype=torch.uint8, device=dev)
    xb = torch.zeros(292 * 8, dtype=torch.uint8, device=dev)
    y = torch.zeros(64, device=dev)
    with pytest.raises(binding.LevoHipError, match="Q4_K, Q5_K or Q6_K"):
        hip.mul_mat_kquant(8, w, xb, y, 4, 4, 256, 1)
    with pytest.raises(binding.LevoHipError, match="multiple of 256"):
        hip.mul_mat_kquant(Q4_K, w, xb, y, 4, 4, 300, 1)
    with pytest.raises(binding.LevoHipError, match="n_vec"):
        hip.mul_mat_kquant(Q4_K, w, xb, y, 4, 4, 256, 9)
    with pytest.raises(binding.LevoHipError, match="at most 16384"):
        hip.mul_mat_kquant(Q4_K, w, xb, y, 4, 4, 256 * 80, 8)
    with pytest.raises(binding.LevoHipError, match="multiple of 256"):
        hip.quantize_q8_K(y, xb, 100)
    assert hip.row_size(Q4_K, 2304) == 9 * 144
    assert hip.row_size(Q6_K, 4608) == 18 * 210
    assert hip.row_size(15, 256) == 292


# ---- shared-input launches (levo_hip_mul_mat_kquant_multi) ---------------------------

def _weights(qtype, rows, k, seed, oracle):
    w = oracle.gaussian(rows * k, seed) * np.float32(0.02)
    return realistic_blocks(qtype, w.reshape(-1, 256))


def _single(hip, dev, qtype, wb, xb, rows, k, n_vec):
    import torch
    y = torch.full((n_vec * rows,), float("nan"), dtype=torch.float32, device=dev)
    hip.mul_mat_kquant(qtype, to_dev(wb, dev), xb, y, rows, rows, k, n_vec)
    return from_dev(y).reshape(n_vec, rows)


def _multi(hip, dev, specs, k, n_vec, x=None, xb=None, pitch=0):
    """specs: (qtype, blocks, rows); returns each matrix's y [n_vec][rows]."""
    import torch
    keep, mats, ys = [], [], []
    for qtype, wb, rows in specs:
        wd = to_dev(wb, dev)
        y = torch.full((n_vec * (rows + 5),), float("nan"), dtype=torch.float32, device=dev)
        keep += [wd, y]
        mats.append((qtype, wd, y, rows + 5, rows))
        ys.append((y, rows))
    xd = None
    if x is not None:
        xd = to_dev(np.ascontiguousarray(x, np.float32), dev)
    hip.mul_mat_kquant_multi(mats, k, n_vec, x_blocks=xb, x=xd, x_pitch=pitch)
    return [from_dev(y).reshape(n_vec, rows + 5)[:, :rows] for y, rows in ys]


@pytest.mark.parametrize("types", [(Q4_K, Q4_K, Q6_K), (Q5_K, Q5_K, Q6_K), (Q6_K, Q6_K, Q6_K)],
                         ids=["q4_k_m", "q5_k_m", "q6_k"])
def test_multi_attention_group_equals_separate_calls(hip, dev, oracle, types):
    """A decode layer's q / k / v under each profile (src/levo-quantization.h:
    75-95: attn_v is promoted to Q6_K in the K_M profiles), 1536 x 1536, the
    CFG pair of activation columns given as F32 and quantized in the launch:
    every y equals quantize_q8_K + mul_mat_kquant for that matrix, bit for bit,
    and the oracle within 1e-5."""
    rows, k, n_vec = 1536, 1536, 2
    x = oracle.gaussian(n_vec * k, 501).reshape(n_vec, k)
    specs = [(t, _weights(t, rows, k, 510 + i, oracle), rows) for i, t in enumerate(types)]
    got = _multi(hip, dev, specs, k, n_vec, x=x, pitch=k)
    xb = q8_K_dev(hip, dev, x)
    for (t, wb, _), g in zip(specs, got):
        assert np.array_equal(g.view(np.uint32), _single(hip, dev, t, wb, xb, rows, k, n_vec).view(np.uint32))
        assert f32_err(g, oracle.mul_mat_kquant(t, wb, x, rows, k)) <= 1e-5


@pytest.mark.parametrize("qtype", [Q4_K, Q5_K])
def test_multi_gate_up_from_blocks(hip, dev, oracle, qtype):
    """gate / up, 8960 x 1536, from Q8_K blocks: bit-identical to separate calls."""
    rows, k, n_vec = 8960, 1536, 2
    x = oracle.gaussian(n_vec * k, 520).reshape(n_vec, k)
    xb = q8_K_dev(hip, dev, x)
    specs = [(qtype, _weights(qtype, rows, k, 521 + i, oracle), rows) for i in range(2)]
    got = _multi(hip, dev, specs, k, n_vec, xb=xb)
    for (t, wb, _), g in zip(specs, got):
        assert np.array_equal(g.view(np.uint32), _single(hip, dev, t, wb, xb, rows, k, n_vec).view(np.uint32))


@pytest.mark.parametrize("k,n_vec,pitch", [(4096, 1, 4096), (2048, 2, 2052), (256, 8, 260), (2304, 1, 2304)])
def test_multi_uneven_rows_and_fused_limits(hip, dev, oracle, k, n_vec, pitch):
    """Matrices of different row counts and types (one empty, skipped), F32
    activations at the in-launch quantization's limit (n_vec * k <= 4096) and
    with a row pitch: each y within 1e-5 of the oracle."""
    rng = np.random.default_rng(k + n_vec)
    x = np.zeros((n_vec, pitch), np.float32)
    x[:, :k] = rng.standard_normal((n_vec, k)).astype(np.float32)
    x[0, :256] = 0.0  # an all-zero Q8_K block
    specs = [(Q6_K, _weights(Q6_K, 1000, k, 530, oracle), 1000), (Q4_K, _weights(Q4_K, 37, k, 531, oracle), 37),
             (Q5_K, np.zeros(0, np.uint8), 0), (Q4_K, _weights(Q4_K, 4100, k, 532, oracle), 4100)]
    got = _multi(hip, dev, specs, k, n_vec, x=x, pitch=pitch)
    for (t, wb, rows), g in zip(specs, got):
        if rows:
            assert f32_err(g, oracle.mul_mat_kquant(t, wb, x[:, :k], rows, k)) <= 1e-5


def test_multi_rejects_bad_arguments(hip, dev, binding):
    import torch
    w = torch.zeros(144 * 8, dtype=torch.uint8, device=dev)
    xb = torch.zeros(292 * 8, dtype=torch.uint8, device=dev)
    xf = torch.zeros(8192, device=dev)
    y = torch.zeros(64, device=dev)
    m = [(Q4_K, w, y, 4, 4)]
    with pytest.raises(binding.LevoHipError, match="exactly one"):
        hip.mul_mat_kquant_multi(m, 256, 1, x_blocks=xb, x=xf, x_pitch=256)
    with pytest.raises(binding.LevoHipError, match="exactly one"):
        hip.mul_mat_kquant_multi(m, 256, 1)
    with pytest.raises(binding.LevoHipError, match="1 to 4 matrices"):
        hip.mul_mat_kquant_multi(m * 5, 256, 1, x_blocks=xb)
    with pytest.raises(binding.LevoHipError, match="4096"):
        hip.mul_mat_kquant_multi(m, 4096, 2, x=xf, x_pitch=4096)
    with pytest.raises(binding.LevoHipError, match="x_pitch"):
        hip.mul_mat_kquant_multi(m, 256, 1, x=xf, x_pitch=250)
    with pytest.raises(binding.LevoHipError, match="Q4_K, Q5_K or Q6_K"):
        hip.mul_mat_kquant_multi([(8, w, y, 4, 4)], 256, 1, x_blocks=xb)
