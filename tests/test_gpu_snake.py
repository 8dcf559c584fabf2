"""SnakeBeta on the GPU vs the oracle's ggml-cpu chain (src/levo-audio-ops.cpp:146-151).

F32 bar: max |a-b| / max(|b|, 1) <= 1e-5 against the oracle; the reference's
own KAT tolerance (2e-5 on its GPU backend, tests/test-audio-ops.cpp:214-215)
against the closed form.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev
from test_oracle import SNAKE_A, SNAKE_B, SNAKE_X, snake_expected_kat

pytestmark = pytest.mark.gpu

TOL = 1e-5
LADDER = [(2048, 252), (1024, 504), (512, 2016), (256, 8064), (128, 48384), (128, 483840)]


def _params(C, seed):
    rng = np.random.default_rng(seed)
    return (rng.uniform(-0.5, 0.5, C).astype(np.float32), rng.uniform(-0.5, 0.5, C).astype(np.float32))


def _gpu(hip, dev, x, a, b, param_type=0):
    import torch
    xd = to_dev(x, dev)
    yd = torch.empty_like(xd)
    hip.snake_beta(xd, to_dev(a, dev), to_dev(b, dev), yd, param_type=param_type)
    return from_dev(yd)


def test_reference_kat(hip, dev, oracle):
    y = _gpu(hip, dev, SNAKE_X, SNAKE_A, SNAKE_B)
    assert np.max(np.abs(y - snake_expected_kat())) <= 2e-5
    assert f32_err(y, oracle.snake_beta(SNAKE_X, SNAKE_A, SNAKE_B)) <= TOL


def test_reference_kat_f16_params(hip, dev, oracle):
    a16, b16 = oracle.f32_to_f16(SNAKE_A), oracle.f32_to_f16(SNAKE_B)
    y = _gpu(hip, dev, SNAKE_X, a16, b16, param_type=1)
    assert np.max(np.abs(y - snake_expected_kat())) <= 2e-3
    want = oracle.snake_beta(SNAKE_X, oracle.f16_to_f32(a16), oracle.f16_to_f32(b16))
    assert f32_err(y, want) <= TOL


@pytest.mark.parametrize("shape", [(128, 48000)] + LADDER)
def test_config_shapes_vs_oracle(hip, dev, oracle, shape):
    C, T = shape
    x = oracle.gaussian(C * T, 1000 + C + T).reshape(C, T)
    a, b = _params(C, C * 7 + T)
    y = _gpu(hip, dev, x, a, b)
    err = f32_err(y, oracle.snake_beta(x, a, b, threads=16))
    assert err <= TOL, err


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (7, 1001), (2, 6), (1025, 3)])
def test_scalar_path_shapes(hip, dev, oracle, shape):
    C, T = shape
    x = oracle.gaussian(C * T, 77 + T).reshape(C, T) * 3
    a, b = _params(C, T)
    assert f32_err(_gpu(hip, dev, x, a, b), oracle.snake_beta(x, a, b)) <= TOL


def test_strided_and_in_place(hip, dev, oracle):
    import torch
    C, T = 33, 640
    x = oracle.gaussian(C * T, 5).reshape(C, T)
    a, b = _params(C, 9)
    want = oracle.snake_beta(x, a, b)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    for xpad, ypad in ((12, 4), (3, 1)):  # vector path, then scalar path
        xbuf = torch.zeros((C, T + xpad), dtype=torch.float32, device=dev)
        xbuf[:, :T] = to_dev(x, dev)
        ybuf = torch.full((C, T + ypad), 7.0, dtype=torch.float32, device=dev)
        hip.snake_beta(xbuf, ad, bd, ybuf, channels=C, time=T, x_stride=T + xpad, y_stride=T + ypad)
        yb = from_dev(ybuf)
        assert f32_err(yb[:, :T], want) <= TOL
        assert np.all(yb[:, T:] == 7.0)  # padding untouched
    xd = to_dev(x, dev)
    hip.snake_beta(xd, ad, bd, xd)
    assert f32_err(from_dev(xd), want) <= TOL


def test_zero_input_is_exact(hip, dev):
    x = np.zeros((16, 4096), np.float32)
    a, b = _params(16, 1)
    assert np.array_equal(_gpu(hip, dev, x, a, b), x)


def test_large_arguments_take_the_slow_sin_path(hip, dev, oracle):
    # |x * alpha| beyond the fast range reduction: still within the F32 bar
    x = (oracle.gaussian(4 * 1024, 3) * 3.0e5).reshape(4, 1024)
    a, b = _params(4, 2)
    assert f32_err(_gpu(hip, dev, x, a, b), oracle.snake_beta(x, a, b)) <= TOL


def test_closed_form_float64(hip, dev, oracle):
    C, T = 64, 8064
    x = oracle.gaussian(C * T, 21).reshape(C, T)
    a, b = _params(C, 4)
    want = x.astype(np.float64) + np.sin(x * np.exp(a.astype(np.float64))[:, None]) ** 2 / (
        np.exp(b.astype(np.float64)) + 1e-9)[:, None]
    assert f32_err(_gpu(hip, dev, x, a, b), want) <= TOL
    assert math.isfinite(float(want.sum()))


def test_batch_matches_single_launches(hip, dev, oracle):
    """levo_hip_snake_beta_batch over the ladder's six shapes plus an F16
    parameter job, an in-place job, a scalar-path job (T = 1001) and an empty
    one: every output bit-identical to its own levo_hip_snake_beta launch (the
    same arithmetic) and within the bar of the oracle."""
    import torch
    shapes = LADDER + [(96, 4000), (33, 1001), (64, 512), (0, 16)]
    jobs, singles, want = [], [], []
    for i, (C, T) in enumerate(shapes):
        x = oracle.gaussian(C * T, 500 + i).reshape(C, T) if C else np.zeros((0, T), np.float32)
        a, b = _params(max(C, 1), 900 + i)
        pt = 1 if i == 6 else 0
        if pt:
            a, b = oracle.f32_to_f16(a), oracle.f32_to_f16(b)
        xd, ad, bd = to_dev(x, dev), to_dev(a, dev), to_dev(b, dev)
        yd = xd if i == 8 else torch.full_like(xd, float("nan"))  # job 8 in place
        jobs.append((xd, ad, bd, yd, pt))
        if C:
            x2 = to_dev(x, dev)
            y2 = torch.empty_like(x2)
            hip.snake_beta(x2, ad, bd, y2, param_type=pt)
            singles.append(from_dev(y2))
            af, bf = (oracle.f16_to_f32(a), oracle.f16_to_f32(b)) if pt else (a, b)
            want.append(oracle.snake_beta(x, af[:C], bf[:C], threads=16))
    hip.snake_beta_batch(jobs)
    torch.cuda.synchronize()
    for (xd, ad, bd, yd, pt), single, w in zip([j for j in jobs if j[0].shape[0]], singles, want):
        got = from_dev(yd)
        assert np.array_equal(got.view(np.uint32), single.view(np.uint32))
        assert f32_err(got, w) <= TOL


def test_batch_rejects_bad_arguments(hip, dev, binding):
    import torch
    x = torch.zeros((4, 8), device=dev)
    a = torch.zeros(4, device=dev)
    with pytest.raises(binding.LevoHipError, match="0 to 16 jobs"):
        hip.snake_beta_batch([(x, a, a, x)] * 17)
    with pytest.raises(binding.LevoHipError, match="F32 or F16"):
        hip.snake_beta_batch([(x, a, a, x, 8)])


def test_batch_rejected_call_writes_nothing(hip, dev, binding):
    """A batch whose last job is invalid fails before any job runs: the
    earlier jobs' outputs (a scalar-path job, T = 1001, and a vector-path job)
    keep their contents."""
    import torch
    xs = torch.ones((4, 1001), device=dev)
    xv = torch.ones((4, 64), device=dev)
    a = torch.zeros(4, device=dev)
    ys = torch.full_like(xs, float("nan"))
    yv = torch.full_like(xv, float("nan"))
    with pytest.raises(binding.LevoHipError, match="F32 or F16"):
        hip.snake_beta_batch([(xs, a, a, ys), (xv, a, a, yv), (xv, a, a, yv, 8)])
    torch.cuda.synchronize()
    assert torch.isnan(ys).all() and torch.isnan(yv).all()
