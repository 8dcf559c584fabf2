"""Split-K SnakeBeta + Conv1d (levo_hip_snake_conv1d_split): the input
channels of each 128 x 128 output tile split over up to four workgroups,
their partial sums combined in split order by a second launch, then the
bias and the residual (the epilogue of conv_1d_f32 and run_residual,
src/levo-audio-ops.cpp:56-87, src/levo-vae.cpp:91-100).

Bars (F32 max|a - b| / max(|b|, 1)): <= 1e-5 against the same convolution
(of the oracle's F32 SnakeBeta output) in float64, and <= 2e-5 against the
oracle's chain (lo_snake_beta_f32, lo_conv1d_f32, the residual add). At
the decoder's stage 1 (K = 1024 x 7 = 7168 terms per output) the oracle's
sequential F32 sum is itself 9.4e-6 from the float64 value, the unsplit
matrix-core sum (one accumulator chain per output, as sequential as the
oracle's) 1.1e-5 and the three split partial sums 6.6e-6, so the split
result differs from the oracle by up to the sum of two F32 errors while
lying closer to the exact convolution than either; two calls bit-identical
(the combine adds in a fixed order);
without a workspace, with a grid that fills the GPU or with fewer K chunks
than splits need, bit-identical to levo_hip_snake_conv1d. Shapes: the
decoder's stage 1 at a 10.08 s window (1024 channels x 2520 samples, k = 7
at dilation 9 and k = 1 with the residual: 160 tiles), the input conv
(64 -> 2048 channels, 2 K chunks per split), a partial last chunk, ragged
lengths, F16 SnakeBeta parameters, y written over the residual, a workspace
for two splits only.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu


def _params(oracle, c, seed):
    a = (oracle.gaussian(c, seed) * np.float32(0.5)).astype(np.float32)
    b = (oracle.gaussian(c, seed + 1) * np.float32(0.5)).astype(np.float32)
    return a, b


def _want(oracle, x, w, b, pad, dil, a=None, bl=None, residual=None):
    xs = oracle.snake_beta(x, a, bl, threads=8) if a is not None else x
    y = oracle.conv1d(xs, w, b, pad, dil, threads=8)
    if residual is not None:
        y = (residual + y).astype(np.float32)
    return y


def _run(hip, dev, x, w, b, pad, dil, a=None, bl=None, residual=None, param_type=0, ws_floats=-1,
         in_place=False):
    """ws_floats: -1 for the full workspace, None for levo_hip_snake_conv1d."""
    import torch
    c_in, t_in = x.shape
    c_out, _, kw = w.shape
    t_out = t_in + 2 * pad - dil * (kw - 1)
    keep = [to_dev(x, dev), to_dev(w, dev)]
    bd = to_dev(b, dev) if b is not None else None
    ad = to_dev(a, dev) if a is not None else None
    bld = to_dev(bl, dev) if bl is not None else None
    rd = to_dev(residual, dev) if residual is not None else None
    y = rd if in_place else torch.full((c_out, t_out), float("nan"), dtype=torch.float32, device=dev)
    kwargs = dict(alpha_log=ad, beta_log=bld, param_type=param_type, bias=bd, padding=pad, dilation=dil,
                  residual=rd, y=y)
    if ws_floats is None:
        hip.snake_conv1d(keep[0], c_in, t_in, keep[1], c_out, kw, **kwargs)
    else:
        n = hip.snake_conv1d_split_workspace_floats(c_out, t_out) if ws_floats < 0 else ws_floats
        ws = torch.full((n,), float("nan"), dtype=torch.float32, device=dev) if n > 0 else None
        hip.snake_conv1d_split(keep[0], c_in, t_in, keep[1], c_out, kw, workspace=ws, workspace_floats=n, **kwargs)
    torch.cuda.synchronize()
    return from_dev(y)


def _f64_rows(oracle, x, w, b, pad, dil, a, bl, residual, rows):
    """The convolution of the oracle's F32 SnakeBeta output in float64, for
    output channels `rows`."""
    xs = (oracle.snake_beta(x, a, bl, threads=8) if a is not None else x).astype(np.float64)
    c_in, t_in = x.shape
    kw = w.shape[2]
    t_out = t_in + 2 * pad - dil * (kw - 1)
    xp = np.zeros((c_in, t_in + 2 * pad))
    xp[:, pad:pad + t_in] = xs
    y = np.zeros((len(rows), t_out))
    for k in range(kw):
        y += w[rows, :, k].astype(np.float64) @ xp[:, k * dil:k * dil + t_out]
    if b is not None:
        y += b[rows, None]
    if residual is not None:
        y += residual[rows]
    return y


def _check(got, oracle, x, w, b, pad, dil, a=None, bl=None, residual=None, every=16):
    """<= 1e-5 against float64 (every `every`-th output channel), <= 2e-5
    against the oracle's F32 chain."""
    rows = np.arange(0, w.shape[0], every)
    assert f32_err(got[rows], _f64_rows(oracle, x, w, b, pad, dil, a, bl, residual, rows)) <= 1e-5
    assert f32_err(got, _want(oracle, x, w, b, pad, dil, a, bl, residual)) <= 2e-5


def _case(oracle, c_in, c_out, t, kw, seed, residual=False):
    x = oracle.gaussian(c_in * t, seed).reshape(c_in, t)
    w = (oracle.gaussian(c_out * c_in * kw, seed + 1) * np.float32(1.0 / np.sqrt(c_in * kw))).reshape(c_out, c_in, kw)
    b = (oracle.gaussian(c_out, seed + 2) * np.float32(0.1)).astype(np.float32)
    a, bl = _params(oracle, c_in, seed + 3)
    r = oracle.gaussian(c_out * t, seed + 5).reshape(c_out, t) if residual else None
    return x, w, b, a, bl, r


@pytest.mark.parametrize("kw,dil", [(7, 9), (7, 1), (1, 1)])
def test_stage1_shapes(hip, dev, oracle, kw, dil):
    """1024 x 2520 (stage 1 of a 10.08 s window): 160 tiles, three splits;
    k = 1 adds the residual in the combine."""
    c, t = 1024, 2520
    pad = 3 * dil if kw == 7 else 0
    x, w, b, a, bl, r = _case(oracle, c, c, t, kw, 20 + kw + dil, residual=kw == 1)
    got = _run(hip, dev, x, w, b, pad, dil, a, bl, r)
    _check(got, oracle, x, w, b, pad, dil, a, bl, r)
    again = _run(hip, dev, x, w, b, pad, dil, a, bl, r)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    unsplit = _run(hip, dev, x, w, b, pad, dil, a, bl, r, ws_floats=None)
    assert f32_err(got, unsplit) <= 2e-5


def test_input_conv_no_snake(hip, dev, oracle):
    """64 -> 2048 channels at 252 frames, no SnakeBeta: 32 tiles, four
    splits of two K chunks."""
    x = oracle.gaussian(64 * 252, 31).reshape(64, 252)
    w = (oracle.gaussian(2048 * 64 * 7, 32) * np.float32(0.05)).reshape(2048, 64, 7)
    b = oracle.gaussian(2048, 33)
    _check(_run(hip, dev, x, w, b, 3, 1), oracle, x, w, b, 3, 1)


@pytest.mark.parametrize("c_in,c_out,t,kw,pad,dil", [(100, 70, 517, 7, 6, 2), (200, 130, 129, 7, 3, 1),
                                                    (160, 257, 1001, 1, 0, 1), (1021, 200, 999, 7, 27, 9)])
def test_partial_chunks_and_ragged_lengths(hip, dev, oracle, c_in, c_out, t, kw, pad, dil):
    """A partial last K chunk in the last split, partial channel and time
    tiles, rows not a multiple of 4 samples (padded partial rows)."""
    x, w, b, a, bl, _ = _case(oracle, c_in, c_out, t, kw, c_in + t)
    _check(_run(hip, dev, x, w, b, pad, dil, a, bl), oracle, x, w, b, pad, dil, a, bl, every=1)


def test_f16_params_in_place_residual_and_small_workspace(hip, dev, oracle):
    """F16 SnakeBeta parameters; y written over the residual (the combine
    reads each residual element before writing it); a workspace for two
    partial sums only (two splits instead of four)."""
    c_in, c_out, t = 256, 256, 1500
    x, w, b, a, bl, r = _case(oracle, c_in, c_out, t, 1, 40, residual=True)
    a16, b16 = oracle.f32_to_f16(a), oracle.f32_to_f16(bl)
    a32, b32 = oracle.f16_to_f32(a16), oracle.f16_to_f32(b16)
    got = _run(hip, dev, x, w, b, 0, 1, a16, b16, r, param_type=1, in_place=True)
    _check(got, oracle, x, w, b, 0, 1, a32, b32, r, every=4)
    two = _run(hip, dev, x, w, b, 0, 1, a16, b16, r, param_type=1, ws_floats=2 * c_out * 1500)
    _check(two, oracle, x, w, b, 0, 1, a32, b32, r, every=4)


@pytest.mark.parametrize("c_in,c_out,t,kw,ws", [(13, 7, 300, 3, -1), (128, 128, 48384, 7, -1), (1024, 1024, 2520, 7, 0),
                                                (1024, 1024, 2520, 7, 1024 * 2520)])
def test_falls_back_bit_identical(hip, dev, oracle, c_in, c_out, t, kw, ws):
    """Two K chunks (a split needs two each), a grid of 378 tiles, an empty
    workspace and a workspace below two partial sums all run the unsplit
    convolution, bit for bit."""
    pad = (kw - 1) // 2
    x, w, b, a, bl, _ = _case(oracle, c_in, c_out, t, kw, 50 + c_in)
    got = _run(hip, dev, x, w, b, pad, 1, a, bl, ws_floats=ws)
    plain = _run(hip, dev, x, w, b, pad, 1, a, bl, ws_floats=None)
    assert np.array_equal(got.view(np.uint32), plain.view(np.uint32))


def test_rejects_bad_workspace(hip, dev, binding):
    import torch
    c, t = 256, 1000
    x = torch.zeros((c, t), device=dev)
    w = torch.zeros((c, c, 7), device=dev)
    y = torch.zeros((c, t), device=dev)
    n = hip.snake_conv1d_split_workspace_floats(c, t)
    ws = torch.zeros(n + 4, device=dev)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.snake_conv1d_split(x, c, t, w, c, 7, workspace=ws[1:], workspace_floats=n, padding=3, y=y)
    big = torch.zeros(c * t + n, device=dev)
    with pytest.raises(binding.LevoHipError, match="overlaps"):
        hip.snake_conv1d_split(x, c, t, w, c, 7, workspace=big, workspace_floats=n, padding=3, y=big)
    assert hip.snake_conv1d_split_workspace_floats(0, 5) < 0
    assert hip.snake_conv1d_split_workspace_floats(3, 5) == 4 * 3 * 8


# ---- transposed convolution (levo_hip_snake_conv_transpose1d_split) --------

def _run_t(hip, dev, x, w, b, stride, pad, a=None, bl=None, param_type=0, split=True):
    import torch
    c_in, t_in = x.shape
    _, c_out, _ = w.shape
    t_out = (t_in + 1) * stride - 2 * pad
    packed = torch.empty(stride * c_out * c_in * 2, dtype=torch.float32, device=dev)
    hip.conv_transpose1d_pack_weights(to_dev(w, dev), packed, c_in, c_out, stride)
    y = torch.full((c_out, t_out), float("nan"), dtype=torch.float32, device=dev)
    kwargs = dict(alpha_log=to_dev(a, dev) if a is not None else None,
                  beta_log=to_dev(bl, dev) if bl is not None else None, param_type=param_type,
                  bias=to_dev(b, dev) if b is not None else None, padding=pad, y=y)
    if split:
        n = hip.snake_conv_transpose1d_split_workspace_floats(c_out, t_in, stride)
        ws = torch.full((n,), float("nan"), dtype=torch.float32, device=dev)
        hip.snake_conv_transpose1d_split(to_dev(x, dev), c_in, t_in, packed, c_out, stride, workspace=ws,
                                         workspace_floats=n, **kwargs)
    else:
        hip.snake_conv_transpose1d(to_dev(x, dev), c_in, t_in, packed, c_out, stride, **kwargs)
    torch.cuda.synchronize()
    return from_dev(y)


def _f64_transpose_rows(oracle, x, w, b, stride, pad, a, bl, rows):
    """ggml_conv_transpose_1d + crop + bias (src/levo-audio-ops.cpp:89-123) in
    float64 for output channels `rows`: input sample q feeds outputs
    q * stride + k - pad for k < 2 * stride."""
    xs = (oracle.snake_beta(x, a, bl, threads=8) if a is not None else x).astype(np.float64)
    t_in = x.shape[1]
    full = np.zeros((len(rows), (t_in + 1) * stride))
    for k in range(2 * stride):
        full[:, k:k + t_in * stride:stride] += w[:, rows, k].astype(np.float64).T @ xs
    t_out = (t_in + 1) * stride - 2 * pad
    y = full[:, pad:pad + t_out]
    return y + b[rows, None] if b is not None else y


def _t_case(oracle, c_in, c_out, t_in, stride, seed):
    x = oracle.gaussian(c_in * t_in, seed).reshape(c_in, t_in)
    w = (oracle.gaussian(c_in * c_out * 2 * stride, seed + 1) *
         np.float32(1.0 / np.sqrt(2 * c_in))).reshape(c_in, c_out, 2 * stride)
    b = (oracle.gaussian(c_out, seed + 2) * np.float32(0.1)).astype(np.float32)
    a, bl = _params(oracle, c_in, seed + 3)
    return x, w, b, a, bl


def test_transpose_stage1_window(hip, dev, oracle):
    """Stage 1's upsampler at a 10.08 s window (2048 -> 1024 channels, 252
    frames, stride 10: 160 workgroups, three splits): float64 rows, two calls
    bit-identical, the unsplit launch within two F32 errors."""
    c_in, c_out, t_in, s = 2048, 1024, 252, 10
    pad = (s + 1) // 2
    x, w, b, a, bl = _t_case(oracle, c_in, c_out, t_in, s, 80)
    got = _run_t(hip, dev, x, w, b, s, pad, a, bl)
    rows = np.arange(0, c_out, 16)
    assert f32_err(got[rows], _f64_transpose_rows(oracle, x, w, b, s, pad, a, bl, rows)) <= 1e-5
    again = _run_t(hip, dev, x, w, b, s, pad, a, bl)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    assert f32_err(got, _run_t(hip, dev, x, w, b, s, pad, a, bl, split=False)) <= 2e-5


@pytest.mark.parametrize("c_in,c_out,t_in,stride,pad,f16", [(2048, 1024, 60, 10, 5, False), (520, 200, 77, 3, 2, True),
                                                            (64, 130, 255, 1, 0, False), (256, 128, 103, 4, 2, True)])
def test_transpose_split_shapes(hip, dev, oracle, c_in, c_out, t_in, stride, pad, f16):
    """Against float64 (every output channel) and the oracle's
    conv_transpose_1d restatement: four splits at stage 1's channels, a
    partial last chunk (520 channels: 33 chunks of 16), stride 1, column
    counts not a multiple of 4, F16 SnakeBeta parameters."""
    x, w, b, a, bl = _t_case(oracle, c_in, c_out, t_in, stride, c_in + t_in)
    pt = 0
    if f16:
        a16, b16 = oracle.f32_to_f16(a), oracle.f32_to_f16(bl)
        got = _run_t(hip, dev, x, w, b, stride, pad, a16, b16, param_type=1)
        a, bl = oracle.f16_to_f32(a16), oracle.f16_to_f32(b16)
    else:
        got = _run_t(hip, dev, x, w, b, stride, pad, a, bl, param_type=pt)
    rows = np.arange(c_out)
    assert f32_err(got, _f64_transpose_rows(oracle, x, w, b, stride, pad, a, bl, rows)) <= 1e-5
    xs = oracle.snake_beta(x, a, bl, threads=8)
    assert f32_err(got, oracle.conv_transpose1d(xs, w, b, stride, pad)) <= 2e-5
