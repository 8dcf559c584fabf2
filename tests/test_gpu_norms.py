"""Fused residual add + RMSNorm / LayerNorm on the GPU vs the oracle.

Bars: the residual output h is bit-exact (one F16 / F32 rounding of x + d);
F16 outputs within 1 F16 ulp, F32 outputs within max |a-b|/max(|b|,1) <= 1e-5.
(In practice both sides reduce in double and agree bit-for-bit; the tests
also report how many elements differ.)
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f16_ulp, f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _inputs(oracle, rows, D, seed, f16):
    x = oracle.gaussian(rows * D, seed).reshape(rows, D)
    d = oracle.gaussian(rows * D, seed + 1).reshape(rows, D)
    w = (oracle.gaussian(D, seed + 2) * 0.02 + 1).astype(np.float32)
    b = (oracle.gaussian(D, seed + 3) * 0.02).astype(np.float32)
    if f16:
        return tuple(oracle.f32_to_f16(t) for t in (x, d, w, b))
    return x, d, w, b


def _run(hip, dev, layer, x, d, w, b, eps, with_delta=True, with_h=True):
    import torch
    f16 = x.dtype == np.uint16
    act = 1 if f16 else 0
    view = (lambda a: a.view(np.int16)) if f16 else (lambda a: a)
    xd = to_dev(view(x), dev)
    dd = to_dev(view(d), dev) if with_delta else None
    wd, bd = to_dev(view(w), dev), to_dev(view(b), dev)
    hd = torch.empty_like(xd) if with_h else None
    yd = torch.empty_like(xd)
    rows, D = x.shape
    if layer:
        hip.layer_norm(act, xd, dd, wd, bd, act, hd, yd, rows, D, eps)
    else:
        hip.rms_norm(act, xd, dd, wd, act, hd, yd, rows, D, eps)
    back = (lambda a: a.view(np.uint16)) if f16 else (lambda a: a)
    return (back(from_dev(hd)) if with_h else None), back(from_dev(yd))


@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
@pytest.mark.parametrize("D", [1536, 2048])
@pytest.mark.parametrize("rows", [1, 2, 756])
def test_f16_config_shapes(hip, dev, oracle, layer, D, rows):
    x, d, w, b = _inputs(oracle, rows, D, 100 + rows + D, True)
    eps = 1e-6
    h, y = _run(hip, dev, layer, x, d, w, b, eps)
    if layer:
        hw, yw = oracle.layer_norm(x, d, w, b, eps, threads=8)
    else:
        hw, yw = oracle.rms_norm(x, d, w, eps, threads=8)
    assert np.array_equal(h, hw)
    ulp = f16_ulp(y, yw)
    print(f"differing elements: {np.count_nonzero(y != yw)} of {y.size}")
    assert ulp <= 1


@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
@pytest.mark.parametrize("D", [1536, 2200, 4400])
def test_f32_reference_chains(hip, dev, oracle, layer, D):
    rows = 37
    x, d, w, b = _inputs(oracle, rows, D, 7 * D, False)
    eps = 1e-5
    h, y = _run(hip, dev, layer, x, d, w, b, eps)
    if layer:
        hw, yw = oracle.layer_norm(x, d, w, b, eps, threads=8)
    else:
        hw, yw = oracle.rms_norm(x, d, w, eps, threads=8)
    assert np.array_equal(h.view(np.uint32), hw.view(np.uint32))
    assert f32_err(y, yw) <= 1e-5


def test_flow_estimator_layernorm_full_shape(hip, dev, oracle):
    """The Flow estimator's residual + LayerNorm at its real shape: F32
    activations [2 (CFG), 1000 frames, 2200] = 2000 rows of 2200 values, F32
    gamma / beta, eps 1e-5 (src/levo-flow-estimator.cpp:20, :106-109, :221-247):
    the residual bit-exact, y within 1e-5 of the oracle."""
    rows, D = 2000, 2200
    x, d, w, b = _inputs(oracle, rows, D, 2200, False)
    h, y = _run(hip, dev, True, x, d, w, b, 1e-5)
    hw, yw = oracle.layer_norm(x, d, w, b, 1e-5, threads=8)
    assert np.array_equal(h.view(np.uint32), hw.view(np.uint32))
    assert f32_err(y, yw) <= 1e-5


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
@pytest.mark.parametrize("rows,D", [(1025, 2056), (1500, 3072), (1111, 4096)])
def test_long_rows(hip, dev, oracle, f16, layer, rows, D):
    """1024 rows or more of 2049-4096 elements (two waves per row): three and
    four groups per lane, F32 groups as two 4-value pieces with the second
    piece of the last groups past the row, row counts that leave the last
    workgroup's second slot empty."""
    x, d, w, b = _inputs(oracle, rows, D, rows * 3 + D, f16)
    eps = 1e-5
    h, y = _run(hip, dev, layer, x, d, w, b, eps)
    if layer:
        hw, yw = oracle.layer_norm(x, d, w, b, eps, threads=8)
    else:
        hw, yw = oracle.rms_norm(x, d, w, eps, threads=8)
    assert np.array_equal(h, hw)
    if f16:
        assert f16_ulp(y, yw) <= 1
    else:
        assert f32_err(y, yw) <= 1e-5


@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
def test_long_rows_without_delta(hip, dev, oracle, layer):
    """Two waves per F32 row with no residual input and no residual output."""
    rows, D = 1200, 2200
    x, d, w, b = _inputs(oracle, rows, D, 99, False)
    zero = np.zeros_like(x)
    _, y = _run(hip, dev, layer, x, d, w, b, 1e-5, with_delta=False, with_h=False)
    if layer:
        _, yw = oracle.layer_norm(x, zero, w, b, 1e-5, threads=8)
    else:
        _, yw = oracle.rms_norm(x, zero, w, 1e-5, threads=8)
    assert f32_err(y, yw) <= 1e-5


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
@pytest.mark.parametrize("rows,D", [(514, 2048), (513, 2056), (600, 3072), (520, 4104), (515, 8192), (511, 1536),
                                    (7, 8192)])
def test_row_layouts(hip, dev, oracle, f16, layer, rows, D):
    """Every workgroup layout of the vector kernel: one wave per row (512 rows
    or more, rows up to 2048), two or four waves per long row, and four waves
    per row for fewer than 512 rows; row counts that leave the last
    workgroup's row slots partly empty."""
    x, d, w, b = _inputs(oracle, rows, D, rows + D, f16)
    eps = 1e-6
    h, y = _run(hip, dev, layer, x, d, w, b, eps)
    if layer:
        hw, yw = oracle.layer_norm(x, d, w, b, eps, threads=8)
    else:
        hw, yw = oracle.rms_norm(x, d, w, eps, threads=8)
    assert np.array_equal(h, hw)
    if f16:
        assert f16_ulp(y, yw) <= 1
    else:
        assert f32_err(y, yw) <= 1e-5


@pytest.mark.parametrize("f16", [True, False])
@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
def test_scalar_path_and_optional_buffers(hip, dev, oracle, f16, layer):
    rows, D = 5, 1003
    x, d, w, b = _inputs(oracle, rows, D, 55, f16)
    eps = 1e-6
    for with_delta, with_h in ((True, True), (False, False), (True, False)):
        h, y = _run(hip, dev, layer, x, d, w, b, eps, with_delta, with_h)
        dd = d if with_delta else None
        if layer:
            hw, yw = oracle.layer_norm(x, dd, w, b, eps)
        else:
            hw, yw = oracle.rms_norm(x, dd, w, eps)
        if with_h:
            assert np.array_equal(h, hw)
        if f16:
            assert f16_ulp(y, yw) <= 1
        else:
            assert f32_err(y, yw) <= 1e-5


def test_layer_norm_constant_rows_give_beta(hip, dev, oracle):
    D = 2048
    x = np.full((4, D), 0.3, np.float32)
    _, _, w, b = _inputs(oracle, 1, D, 3, False)
    _, y = _run(hip, dev, True, x, x, w, b, 1e-6, with_delta=False)
    assert np.array_equal(y, np.broadcast_to(b, y.shape))


def test_rms_f32_with_f16_weight(hip, dev, oracle):
    """src/levo-lm.cpp:131-137 casts an F16 GGUF weight to F32 (exact)."""
    import torch
    rows, D = 9, 1536
    x, d, w, _ = _inputs(oracle, rows, D, 17, False)
    w16 = oracle.f32_to_f16(w)
    xd, dd = to_dev(x, dev), to_dev(d, dev)
    yd = torch.empty_like(xd)
    hip.rms_norm(0, xd, dd, to_dev(w16.view(np.int16), dev), 1, None, yd, rows, D, 1e-5)
    _, yw = oracle.rms_norm(x, d, oracle.f16_to_f32(w16), 1e-5)
    assert f32_err(from_dev(yd), yw) <= 1e-5


@pytest.mark.parametrize("layer", [False, True], ids=["rms", "ln"])
def test_f16_subnormal_results_follow_the_f32_then_f16_chain(hip, dev, oracle, layer):
    """Rows whose normalised values land in the F16 subnormal range: h * scale
    is rounded to F32 and then to F16 (src/levo-kv.cpp:157-159), never fused."""
    rows, D = 64, 2048
    half = oracle.gaussian(rows * D // 2, 31).reshape(rows, D // 2)
    half[:, :512] = np.geomspace(6e-8, 6e-5, 512).astype(np.float32) * np.where(np.arange(512) % 2, 1, -1)
    half = oracle.f16_to_f32(oracle.f32_to_f16(half))
    # +v / -v pairs of F16 values: the row mean is exactly 0 in any summation
    # order, so LayerNorm also keeps the tiny values tiny
    x = np.concatenate([half, -half], axis=1)
    xh = oracle.f32_to_f16(x)
    dh = oracle.f32_to_f16(np.zeros_like(x))
    w = oracle.f32_to_f16(oracle.gaussian(D, 32) * 0.02 + 1)
    b = oracle.f32_to_f16(np.zeros(D, np.float32))
    h, y = _run(hip, dev, layer, xh, dh, w, b, 1e-6)
    if layer:
        hw, yw = oracle.layer_norm(xh, dh, w, b, 1e-6)
    else:
        hw, yw = oracle.rms_norm(xh, dh, w, 1e-6)
    assert np.array_equal(h, hw)
    sub = (yw & 0x7C00) == 0
    assert np.count_nonzero(sub) > 1000
    print(f"differing elements: {np.count_nonzero(y != yw)}")
    assert f16_ulp(y, yw) <= 1
