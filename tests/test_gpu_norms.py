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


# ---- gated residual + LayerNorm + AdaLN modulation (Flow estimator blocks) ----------

def _mod_vec(rng, batches, dim, stride, learned=True, scale=0.3):
    dyn = (rng.standard_normal((batches, stride)) * scale).astype(np.float32)
    lrn = (rng.standard_normal(dim) * scale).astype(np.float32) if learned else None
    return dyn, lrn


def _run_mod(hip, binding, dev, x, d, gate, gamma, beta, scale, shift, rpb, eps, f16_params=False,
             in_place=False, with_h=True):
    """levo_hip_residual_layer_norm_modulated on device copies; returns (h, y)."""
    import torch
    keep = []

    def put(a):
        t = to_dev(a, dev)
        keep.append(t)
        return t

    def vec(v):
        """v: None, (dynamic, learned) or (dynamic, learned, first column)."""
        bv = binding.BatchVector()
        if v is None:
            return bv
        dyn, lrn = v[0], v[1]
        col = v[2] if len(v) > 2 else 0
        bv.dynamic, bv.stride = put(dyn).data_ptr() + 4 * col, dyn.shape[1]
        bv.learned = put(lrn).data_ptr() if lrn is not None else None
        return bv

    rows, dim = x.shape
    xd = put(x)
    a = binding.ModulatedNormArgs()
    a.x = xd.data_ptr()
    a.delta = put(d).data_ptr() if d is not None else None
    a.gate, a.scale, a.shift = vec(gate), vec(scale), vec(shift)
    conv = (lambda t: oracle_f16(t)) if f16_params else (lambda t: t)
    a.gamma, a.beta = put(conv(gamma)).data_ptr(), put(conv(beta)).data_ptr()
    a.param_type = 1 if f16_params else 0
    hd = xd if in_place else (torch.empty_like(xd) if with_h else None)
    yd = torch.empty_like(xd)
    a.h_out = hd.data_ptr() if hd is not None else None
    a.y = yd.data_ptr()
    a.rows, a.rows_per_batch, a.dim, a.eps = rows, rpb, dim, eps
    hip.layer_norm_modulated(a)
    return (from_dev(hd) if hd is not None else None), from_dev(yd)


def oracle_f16(a):
    return a.astype(np.float16).view(np.int16)


def _mod_inputs(rows, dim, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float32)
    gamma = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    beta = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    return rng, x, d, gamma, beta


def test_modulated_flow_estimator_full_shape(hip, binding, dev, oracle):
    """The Flow estimator's block boundary at its real shape: batch 2 x 1000
    frames x 2200, gate / scale / shift = chunks 2 / 4 / 3 of a [batch][6 x
    2200] time modulation (read in place, 6 x 2200 floats apart) plus the
    block's learned table (modulation_chunk), eps 1e-5. h bit-exact; y within
    1e-5 of the oracle."""
    rows, dim, rpb = 2000, 2200, 1000
    rng, x, d, gamma, beta = _mod_inputs(rows, dim, 31)
    tm = (rng.standard_normal((2, 6 * dim)) * 0.3).astype(np.float32)
    table = (rng.standard_normal(6 * dim) * 0.3).astype(np.float32)
    chunk = lambda k: (tm, table[k * dim:(k + 1) * dim], k * dim)
    h, y = _run_mod(hip, binding, dev, x, d, chunk(2), gamma, beta, chunk(4), chunk(3), rpb, 1e-5)
    view = lambda k: (tm[:, k * dim:], table[k * dim:(k + 1) * dim])
    hw, yw = oracle.layer_norm_modulated(x, d, view(2), gamma, beta, view(4), view(3), rpb, 1e-5)
    assert np.array_equal(h.view(np.uint32), hw.view(np.uint32))
    assert f32_err(y, yw) <= 1e-5, f"{np.count_nonzero(y != yw)} values differ"


@pytest.mark.parametrize("delta,gate,mod", [(True, True, True), (True, True, False), (True, False, True),
                                            (True, False, False), (False, False, True), (False, False, False)])
@pytest.mark.parametrize("dim", [512, 1028, 2200, 2560, 2564, 4096])
def test_modulated_variants(hip, binding, dev, oracle, delta, gate, mod, dim):
    """Every combination of delta / gate / modulation at each row-length
    instance (up to 1024, 2560, 4096 values; lengths that leave a lane's last
    piece past the row), 3 batch entries of 7 rows (workgroups of 4 rows end
    inside an entry)."""
    rows, rpb = 21, 7
    rng, x, d, gamma, beta = _mod_inputs(rows, dim, dim + 8 * delta + 4 * gate + 2 * mod)
    g = _mod_vec(rng, 3, dim, dim + 12) if gate else None
    s = _mod_vec(rng, 3, dim, dim + 4) if mod else None
    sh = _mod_vec(rng, 3, dim, dim, learned=False) if mod else None
    h, y = _run_mod(hip, binding, dev, x, d if delta else None, g, gamma, beta, s, sh, rpb, 1e-5)
    hw, yw = oracle.layer_norm_modulated(x, d if delta else None, g, gamma, beta, s, sh, rpb, 1e-5)
    assert np.array_equal(h.view(np.uint32), hw.view(np.uint32))
    assert f32_err(y, yw) <= 1e-5


def test_modulated_f16_params_in_place(hip, binding, dev, oracle):
    """F16 gamma / beta (widened exactly) and the residual written over x."""
    rows, dim, rpb = 16, 2200, 8
    rng, x, d, gamma, beta = _mod_inputs(rows, dim, 41)
    gamma16 = gamma.astype(np.float16).astype(np.float32)
    beta16 = beta.astype(np.float16).astype(np.float32)
    g, s, sh = (_mod_vec(rng, 2, dim, 6 * dim) for _ in range(3))
    h, y = _run_mod(hip, binding, dev, x, d, g, gamma16, beta16, s, sh, rpb, 1e-5, f16_params=True, in_place=True)
    hw, yw = oracle.layer_norm_modulated(x, d, g, gamma16, beta16, s, sh, rpb, 1e-5)
    assert np.array_equal(h.view(np.uint32), hw.view(np.uint32))
    assert f32_err(y, yw) <= 1e-5
    _, y2 = _run_mod(hip, binding, dev, x, d, g, gamma16, beta16, s, sh, rpb, 1e-5, f16_params=True, with_h=False)
    assert np.array_equal(y2.view(np.uint32), y.view(np.uint32))


def test_modulated_rejects_bad_arguments(hip, binding, dev):
    import torch
    x = torch.zeros((8, 64), device=dev)
    p = torch.ones(64, device=dev)
    v = torch.zeros((2, 64), device=dev)

    def args(**kw):
        a = binding.ModulatedNormArgs()
        a.x, a.y, a.gamma, a.beta = x.data_ptr(), x.data_ptr(), p.data_ptr(), p.data_ptr()
        a.rows, a.rows_per_batch, a.dim, a.eps = 8, 4, 64, 1e-5
        for k, val in kw.items():
            setattr(a, k, val)
        return a

    bv = binding.BatchVector(v.data_ptr(), 64, None)
    for bad, msg in ((args(gate=bv), "gate needs delta"), (args(scale=bv), "scale and shift"),
                     (args(rows_per_batch=3), "whole number"), (args(dim=62), "multiple of 4"),
                     (args(dim=4100), "multiple of 4"), (args(x=x.data_ptr() + 4), "aligned"),
                     (args(scale=binding.BatchVector(v.data_ptr(), 60, None),
                           shift=binding.BatchVector(v.data_ptr(), 60, None)), "stride"),
                     (args(param_type=2), "F32 or F16")):
        with pytest.raises(binding.LevoHipError, match=msg):
            hip.layer_norm_modulated(bad)
    hip.layer_norm_modulated(args(rows=0))  # nothing to do
