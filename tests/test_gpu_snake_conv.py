"""Fused SnakeBeta + Conv1d + bias + residual (levo_hip_snake_conv1d)
against the oracle's chain: lo_snake_beta_f32 (the reference's ggml chain)
then lo_conv1d_f32 (ggml_im2col + F32 mul_mat + bias,
src/levo-audio-ops.cpp:56-87), then the residual add (src/levo-vae.cpp:100).

Bar: F32 max|a - b| / max(|b|, 1) <= 1e-5 (the matrix cores sum in another
order than ggml's dot); bit-exact for delta kernels without SnakeBeta,
where every output is one product (KAT-style identity / shift / dilation).
Shapes: the decoder's residual units (k = 7 at dilation 1, 3, 9 with
padding 3d; k = 1) at the last stage's 128 channels and at 1024 channels,
the input conv 64 -> 2048 without SnakeBeta, the output conv 128 -> 2, odd
channel counts and lengths, F16 SnakeBeta parameters, strides, y written
over the residual, and inputs beyond the reduced sine's range (bit-exact
against levo_hip_snake_beta followed by the conv without SnakeBeta).
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


def _run(hip, dev, x, w, b, pad, dil, a=None, bl=None, residual=None, param_type=0):
    import torch
    c_in, t_in = x.shape
    c_out, _, kw = w.shape
    t_out = t_in + 2 * pad - dil * (kw - 1)
    y = torch.full((c_out, t_out), float("nan"), dtype=torch.float32, device=dev)
    keep = [to_dev(x, dev), to_dev(w, dev)]
    bd = to_dev(b, dev) if b is not None else None
    ad = to_dev(a, dev) if a is not None else None
    bld = to_dev(bl, dev) if bl is not None else None
    rd = to_dev(residual, dev) if residual is not None else None
    hip.snake_conv1d(keep[0], c_in, t_in, keep[1], c_out, kw, alpha_log=ad, beta_log=bld, param_type=param_type,
                     bias=bd, padding=pad, dilation=dil, residual=rd, y=y)
    return from_dev(y)


@pytest.mark.parametrize("c,t,kw,dil", [(128, 48384, 7, 1), (128, 48384, 7, 3), (128, 48384, 7, 9),
                                        (128, 48384, 1, 1), (1024, 2520, 7, 9), (512, 3000, 1, 1)])
def test_residual_unit_convs(hip, dev, oracle, c, t, kw, dil):
    """snake -> conv (k = 7, padding 3d, dilation d) and snake -> conv (k = 1)
    + residual, as run_residual builds them (src/levo-vae.cpp:91-100)."""
    pad = 3 * dil if kw == 7 else 0
    x = oracle.gaussian(c * t, c + kw + dil).reshape(c, t)
    w = (oracle.gaussian(c * c * kw, 2 * c + dil) * np.float32(1.0 / np.sqrt(c * kw))).reshape(c, c, kw)
    b = (oracle.gaussian(c, 3 * c) * np.float32(0.1)).astype(np.float32)
    a, bl = _params(oracle, c, 4 * c + dil)
    residual = oracle.gaussian(c * t, 5 * c).reshape(c, t) if kw == 1 else None
    got = _run(hip, dev, x, w, b, pad, dil, a, bl, residual)
    want = _want(oracle, x, w, b, pad, dil, a, bl, residual)
    assert f32_err(got, want) <= 1e-5


def test_input_and_output_convs(hip, dev, oracle):
    """The decoder's input conv (64 -> 2048, k = 7, padding 3, no SnakeBeta)
    and output conv (SnakeBeta, 128 -> 2, k = 7, no bias)."""
    x = oracle.gaussian(64 * 252, 11).reshape(64, 252)
    w = (oracle.gaussian(2048 * 64 * 7, 12) * np.float32(0.05)).reshape(2048, 64, 7)
    b = oracle.gaussian(2048, 13)
    assert f32_err(_run(hip, dev, x, w, b, 3, 1), _want(oracle, x, w, b, 3, 1)) <= 1e-5
    x = oracle.gaussian(128 * 20000, 14).reshape(128, 20000)
    w = (oracle.gaussian(2 * 128 * 7, 15) * np.float32(0.03)).reshape(2, 128, 7)
    a, bl = _params(oracle, 128, 16)
    assert f32_err(_run(hip, dev, x, w, None, 3, 1, a, bl), _want(oracle, x, w, None, 3, 1, a, bl)) <= 1e-5


@pytest.mark.parametrize("c_in,c_out,t,kw,pad,dil", [(13, 7, 300, 3, 1, 2), (5, 3, 9, 5, 0, 1), (1, 1, 1, 1, 0, 1),
                                                    (200, 130, 129, 7, 3, 1), (33, 257, 1000, 1, 0, 1),
                                                    (9, 4, 70, 7, 27, 9)])
def test_odd_shapes(hip, dev, oracle, c_in, c_out, t, kw, pad, dil):
    """Partial K chunks, partial channel and time tiles, scalar weight loads."""
    x = oracle.gaussian(c_in * t, c_in + t).reshape(c_in, t)
    w = (oracle.gaussian(c_out * c_in * kw, c_out + t) * np.float32(0.2)).reshape(c_out, c_in, kw)
    b = oracle.gaussian(c_out, 7)
    a, bl = _params(oracle, c_in, 8)
    assert f32_err(_run(hip, dev, x, w, b, pad, dil, a, bl), _want(oracle, x, w, b, pad, dil, a, bl)) <= 1e-5


def test_partial_chunk(hip, dev, oracle):
    """k = 7 with 100 input channels: the last chunk of 8 holds 4 (with and
    without SnakeBeta)."""
    c_in, c_out, t, pad, dil = 100, 70, 517, 6, 2
    x = oracle.gaussian(c_in * t, 140).reshape(c_in, t)
    w = (oracle.gaussian(c_out * c_in * 7, 141) * np.float32(1.0 / np.sqrt(c_in * 7))).reshape(c_out, c_in, 7)
    b = oracle.gaussian(c_out, 142)
    a, bl = _params(oracle, c_in, 143)
    assert f32_err(_run(hip, dev, x, w, b, pad, dil, a, bl), _want(oracle, x, w, b, pad, dil, a, bl)) <= 1e-5
    assert f32_err(_run(hip, dev, x, w, b, pad, dil), _want(oracle, x, w, b, pad, dil)) <= 1e-5


def test_large_arguments(hip, dev, oracle):
    """Inputs whose alpha * x lies beyond the reduced-argument sine's range
    (|alpha x| > 8192: the full sinf form) in every chunk. The fused launch
    must equal, bit for bit, levo_hip_snake_beta followed by the same conv
    without SnakeBeta (one accumulation order, one SnakeBeta definition).
    Against the oracle the bar is taken on the output's scale: summands of
    1e3 cancel to outputs near zero, where F32 sums in any two orders differ
    by ~1e-3 absolute."""
    import torch
    c_in, c_out, t, pad, dil = 100, 70, 517, 6, 2
    x = oracle.gaussian(c_in * t, 144).reshape(c_in, t)
    x[3::7] *= np.float32(3.0e4)      # whole rows, every chunk
    x[:, 100:103] *= np.float32(2.5e4)  # columns across all channels
    w = (oracle.gaussian(c_out * c_in * 7, 145) * np.float32(1.0 / np.sqrt(c_in * 7))).reshape(c_out, c_in, 7)
    b = oracle.gaussian(c_out, 146)
    a, bl = _params(oracle, c_in, 147)
    fused = _run(hip, dev, x, w, b, pad, dil, a, bl)
    xs = torch.empty((c_in, t), dtype=torch.float32, device=dev)
    hip.snake_beta(to_dev(x, dev), to_dev(a, dev), to_dev(bl, dev), xs)
    torch.cuda.synchronize()
    two_step = _run(hip, dev, from_dev(xs), w, b, pad, dil)
    assert np.array_equal(fused.view(np.uint32), two_step.view(np.uint32))
    want = _want(oracle, x, w, b, pad, dil, a, bl)
    assert np.max(np.abs(fused.astype(np.float64) - want)) <= 1e-5 * np.max(np.abs(want))


def test_delta_kernels_bit_exact(hip, dev, oracle):
    """Identity, one-sample delay and dilated advance: each output is one
    product with 1.0 (exact), plus the bias in its own rounding."""
    c, t = 130, 1000
    x = oracle.gaussian(c * t, 90).reshape(c, t)
    b = oracle.gaussian(c, 91)
    eye = np.eye(c, dtype=np.float32)
    for tap, pad, dil in ((3, 3, 1), (0, 3, 1), (6, 27, 9)):
        w = np.zeros((c, c, 7), np.float32)
        w[:, :, tap] = eye
        got = _run(hip, dev, x, w, b, pad, dil)
        want = _want(oracle, x, w, b, pad, dil)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (tap, pad, dil)


def test_f16_snake_parameters(hip, dev, oracle):
    """F16 alpha_log / beta_log are widened exactly (src/levo-audio-ops.cpp:143-144)."""
    c, t = 64, 5000
    x = oracle.gaussian(c * t, 100).reshape(c, t)
    w = (oracle.gaussian(c * c * 7, 101) * np.float32(0.05)).reshape(c, c, 7)
    a16 = oracle.f32_to_f16(_params(oracle, c, 102)[0])
    b16 = oracle.f32_to_f16(_params(oracle, c, 102)[1])
    got = _run(hip, dev, x, w, None, 3, 1, a16, b16, param_type=1)
    want = _want(oracle, x, w, None, 3, 1, oracle.f16_to_f32(a16), oracle.f16_to_f32(b16))
    assert f32_err(got, want) <= 1e-5


def test_strides_and_in_place_residual(hip, dev, oracle):
    """Row strides on x and y, and y written over the residual (the unit's
    second conv adds its input in place)."""
    import torch
    c, t = 128, 3000
    x = oracle.gaussian(c * t, 110).reshape(c, t)
    w = (oracle.gaussian(c * c, 111) * np.float32(0.1)).reshape(c, c, 1)
    b = oracle.gaussian(c, 112)
    r = oracle.gaussian(c * t, 113).reshape(c, t)
    a, bl = _params(oracle, c, 114)
    want = _want(oracle, x, w, b, 0, 1, a, bl, r)
    xs = torch.zeros((c, t + 5), dtype=torch.float32, device=dev)
    xs[:, :t] = torch.from_numpy(x).to(dev)
    rs = torch.zeros((c, t + 3), dtype=torch.float32, device=dev)
    rs[:, :t] = torch.from_numpy(r).to(dev)
    hip.snake_conv1d(xs, c, t, to_dev(w, dev), c, 1, alpha_log=to_dev(a, dev), beta_log=to_dev(bl, dev),
                     bias=to_dev(b, dev), residual=rs, y=rs, x_stride=t + 5, residual_stride=t + 3, y_stride=t + 3)
    assert f32_err(from_dev(rs)[:, :t], want) <= 1e-5


@pytest.mark.parametrize("c_in,t,kw,dil", [(1021, 33000, 7, 9), (1280, 33000, 1, 1), (1024, 33000, 7, 9)])
def test_wide_inputs_parameter_ring(hip, dev, oracle, c_in, t, kw, dil):
    """Wide inputs in a grid of more than one workgroup per CU keep only two
    chunks of SnakeBeta parameters in LDS, each computed one chunk ahead
    (1021 channels at k = 7, dilation 9: weight rows not 16-byte aligned;
    1280 channels at k = 1). 128 outputs: 258 workgroups. With 1024
    channels at k = 7 (a 40 s window's first stage) the interleaved kernel
    keeps the whole table instead, one workgroup per CU."""
    pad = 3 * dil if kw == 7 else 0
    x = oracle.gaussian(c_in * t, 130 + kw).reshape(c_in, t)
    w = (oracle.gaussian(128 * c_in * kw, 131) * np.float32(1.0 / np.sqrt(c_in * kw))).reshape(128, c_in, kw)
    b = oracle.gaussian(128, 132)
    a, bl = _params(oracle, c_in, 133)
    got = _run(hip, dev, x, w, b, pad, dil, a, bl)
    want = _want(oracle, x, w, b, pad, dil, a, bl)
    assert f32_err(got, want) <= 1e-5


@pytest.mark.parametrize("c_in,c_out,t,kw,pad,dil", [(128, 2, 483840, 7, 3, 1), (128, 1, 5000, 7, 3, 1),
                                                    (37, 3, 2049, 5, 2, 4), (8, 4, 1024, 3, 1, 1),
                                                    (17, 4, 3001, 7, 255, 85), (300, 2, 777, 1, 0, 1),
                                                    (2, 3, 40, 7, 0, 5)])
def test_narrow_outputs(hip, dev, oracle, c_in, c_out, t, kw, pad, dil):
    """c_out <= 4 (the decoder's 128 -> 2 output conv at a 10.08 s window's
    483840 samples, and ragged ones): the VAE output path. Partial channel
    chunks, tiles past t_out, padding wider than a tile's halo, the largest
    span (kernel - 1) * dilation = 510 of that path."""
    x = oracle.gaussian(c_in * t, c_in + t + kw).reshape(c_in, t)
    w = (oracle.gaussian(c_out * c_in * kw, c_out + t) * np.float32(1.0 / np.sqrt(c_in * kw))).reshape(c_out, c_in, kw)
    b = oracle.gaussian(c_out, 9) if c_out != 1 else None
    a, bl = _params(oracle, c_in, 10 + c_in)
    got = _run(hip, dev, x, w, b, pad, dil, a, bl)
    want = _want(oracle, x, w, b, pad, dil, a, bl)
    assert got.shape == want.shape
    assert f32_err(got, want) <= 1e-5


def test_narrow_delta_residual_f16(hip, dev, oracle):
    """c_out <= 4: a one-tap selector is exact (each output one product with
    1.0 plus the bias), y written over the residual, F16 SnakeBeta parameters."""
    import torch
    c_in, c_out, t = 19, 4, 3000
    x = oracle.gaussian(c_in * t, 120).reshape(c_in, t)
    b = oracle.gaussian(c_out, 121)
    w = np.zeros((c_out, c_in, 7), np.float32)
    for co, (ci, tap) in enumerate(((0, 3), (7, 0), (18, 6), (11, 2))):
        w[co, ci, tap] = 1.0
    got = _run(hip, dev, x, w, b, 9, 3)
    want = _want(oracle, x, w, b, 9, 3)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    r = oracle.gaussian(c_out * t, 122).reshape(c_out, t)
    w = (oracle.gaussian(c_out * c_in * 7, 123) * np.float32(0.1)).reshape(c_out, c_in, 7)
    a16 = oracle.f32_to_f16(_params(oracle, c_in, 124)[0])
    b16 = oracle.f32_to_f16(_params(oracle, c_in, 124)[1])
    want = _want(oracle, x, w, b, 3, 1, oracle.f16_to_f32(a16), oracle.f16_to_f32(b16), r)
    rs = to_dev(r, dev)
    hip.snake_conv1d(to_dev(x, dev), c_in, t, to_dev(w, dev), c_out, 7, alpha_log=to_dev(a16, dev),
                     beta_log=to_dev(b16, dev), param_type=1, bias=to_dev(b, dev), padding=3, residual=rs, y=rs)
    torch.cuda.synchronize()
    assert f32_err(from_dev(rs), want) <= 1e-5


def test_rejects_bad_arguments(hip, dev, binding):
    import torch
    x = torch.zeros((4, 10), device=dev)
    w = torch.zeros((4, 4, 7), device=dev)
    y = torch.zeros((4, 10), device=dev)
    with pytest.raises(binding.LevoHipError, match="kernel size"):
        hip.snake_conv1d(x, 4, 10, w, 4, 9, padding=4, y=y)
    with pytest.raises(binding.LevoHipError, match="wider than the padded input"):
        hip.snake_conv1d(x, 4, 10, w, 4, 7, padding=0, dilation=2, y=y)
    with pytest.raises(binding.LevoHipError, match="needs both"):
        hip.snake_conv1d(x, 4, 10, w, 4, 7, padding=3, alpha_log=torch.zeros(4, device=dev), y=y)


# ---- SnakeBeta + ConvTranspose1d (the decoder's upsamplers) ----------------------

def _run_transpose(hip, dev, x, w, b, stride, pad, a=None, bl=None, param_type=0):
    import torch
    c_in, t_in = x.shape
    _, c_out, k = w.shape
    assert k == 2 * stride
    t_out = (t_in + 1) * stride - 2 * pad
    packed = torch.empty(stride * c_out * c_in * 2, dtype=torch.float32, device=dev)
    wd = to_dev(w, dev)
    hip.conv_transpose1d_pack_weights(wd, packed, c_in, c_out, stride)
    y = torch.full((c_out, t_out), float("nan"), dtype=torch.float32, device=dev)
    hip.snake_conv_transpose1d(to_dev(x, dev), c_in, t_in, packed, c_out, stride,
                               alpha_log=to_dev(a, dev) if a is not None else None,
                               beta_log=to_dev(bl, dev) if bl is not None else None, param_type=param_type,
                               bias=to_dev(b, dev) if b is not None else None, padding=pad, y=y)
    return from_dev(y)


def _want_transpose(oracle, x, w, b, stride, pad, a=None, bl=None):
    xs = oracle.snake_beta(x, a, bl, threads=8) if a is not None else x
    return oracle.conv_transpose1d(xs, w, b, stride, pad)


@pytest.mark.parametrize("c_in,c_out,t_in,stride", [(2048, 1024, 40, 10), (1024, 512, 250, 6), (512, 256, 600, 4),
                                                    (256, 128, 2000, 4), (128, 128, 9000, 2)])
def test_upsample_stages(hip, dev, oracle, c_in, c_out, t_in, stride):
    """The five upsample steps of decode (strides 10, 6, 4, 4, 2, kernel
    2 * stride, padding (stride + 1) / 2; src/levo-vae.cpp:215-228) with
    SnakeBeta in front, at shortened lengths."""
    pad = (stride + 1) // 2
    x = oracle.gaussian(c_in * t_in, c_in + stride).reshape(c_in, t_in)
    w = (oracle.gaussian(c_in * c_out * 2 * stride, c_out + t_in) *
         np.float32(1.0 / np.sqrt(2 * c_in))).reshape(c_in, c_out, 2 * stride)
    b = (oracle.gaussian(c_out, 7 + stride) * np.float32(0.1)).astype(np.float32)
    a, bl = _params(oracle, c_in, 8 + stride)
    got = _run_transpose(hip, dev, x, w, b, stride, pad, a, bl)
    want = _want_transpose(oracle, x, w, b, stride, pad, a, bl)
    assert got.shape == want.shape
    assert f32_err(got, want) <= 1e-5


@pytest.mark.parametrize("c_in,c_out,t_in,stride,pad", [(3, 5, 7, 3, 2), (17, 9, 130, 5, 0), (1, 1, 1, 1, 0),
                                                        (33, 130, 255, 2, 1), (6, 4, 20, 4, 3)])
def test_transpose_odd_shapes(hip, dev, oracle, c_in, c_out, t_in, stride, pad):
    """Partial channel and time tiles, odd channel counts (scalar weight
    loads), stride 1, paddings other than the decoder's."""
    x = oracle.gaussian(c_in * t_in, 40 + c_in).reshape(c_in, t_in)
    w = (oracle.gaussian(c_in * c_out * 2 * stride, 41 + c_out) * np.float32(0.3)).reshape(c_in, c_out, 2 * stride)
    b = oracle.gaussian(c_out, 42)
    a, bl = _params(oracle, c_in, 43)
    got = _run_transpose(hip, dev, x, w, b, stride, pad, a, bl)
    want = _want_transpose(oracle, x, w, b, stride, pad, a, bl)
    assert f32_err(got, want) <= 1e-5


def test_transpose_delta_kernel_bit_exact(hip, dev, oracle):
    """A delta tap with no SnakeBeta and no bias is zero-insertion
    upsampling: every output is one product with 1.0 (exact)."""
    c, t, s = 64, 300, 4
    x = oracle.gaussian(c * t, 50).reshape(c, t)
    for tap in (0, 2, 5, 7):
        w = np.zeros((c, c, 2 * s), np.float32)
        w[:, :, tap] = np.eye(c, dtype=np.float32)
        got = _run_transpose(hip, dev, x, w, None, s, 2)
        want = _want_transpose(oracle, x, w, None, s, 2)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), tap


def test_transpose_f16_params_and_no_snake(hip, dev, oracle):
    c_in, c_out, t, s = 64, 32, 500, 6
    x = oracle.gaussian(c_in * t, 60).reshape(c_in, t)
    w = (oracle.gaussian(c_in * c_out * 2 * s, 61) * np.float32(0.1)).reshape(c_in, c_out, 2 * s)
    a16 = oracle.f32_to_f16(_params(oracle, c_in, 62)[0])
    b16 = oracle.f32_to_f16(_params(oracle, c_in, 62)[1])
    got = _run_transpose(hip, dev, x, w, None, s, 3, a16, b16, param_type=1)
    want = _want_transpose(oracle, x, w, None, s, 3, oracle.f16_to_f32(a16), oracle.f16_to_f32(b16))
    assert f32_err(got, want) <= 1e-5
    got = _run_transpose(hip, dev, x, w, None, s, 3)
    assert f32_err(got, _want_transpose(oracle, x, w, None, s, 3)) <= 1e-5


def test_transpose_wide_partial_chunk_and_large_arguments(hip, dev, oracle):
    """520 input channels (the last chunk of 16 holds 8), 200 outputs (a
    partial channel tile), stride 3: with F16 SnakeBeta parameters, without
    SnakeBeta, and with inputs beyond the reduced sine's range, where the
    fused launch must equal levo_hip_snake_beta followed by the transposed
    conv without SnakeBeta, bit for bit."""
    import torch
    c_in, c_out, t_in, s, pad = 520, 200, 77, 3, 2
    x = oracle.gaussian(c_in * t_in, 70).reshape(c_in, t_in)
    w = (oracle.gaussian(c_in * c_out * 2 * s, 71) * np.float32(1.0 / np.sqrt(2 * c_in))).reshape(c_in, c_out, 2 * s)
    b = oracle.gaussian(c_out, 72)
    a16 = oracle.f32_to_f16(_params(oracle, c_in, 73)[0])
    b16 = oracle.f32_to_f16(_params(oracle, c_in, 73)[1])
    got = _run_transpose(hip, dev, x, w, b, s, pad, a16, b16, param_type=1)
    want = _want_transpose(oracle, x, w, b, s, pad, oracle.f16_to_f32(a16), oracle.f16_to_f32(b16))
    assert f32_err(got, want) <= 1e-5
    assert f32_err(_run_transpose(hip, dev, x, w, b, s, pad), _want_transpose(oracle, x, w, b, s, pad)) <= 1e-5
    x[5::11] *= np.float32(3.0e4)
    a, bl = _params(oracle, c_in, 74)
    fused = _run_transpose(hip, dev, x, w, b, s, pad, a, bl)
    xs = torch.empty((c_in, t_in), dtype=torch.float32, device=dev)
    hip.snake_beta(to_dev(x, dev), to_dev(a, dev), to_dev(bl, dev), xs)
    torch.cuda.synchronize()
    two_step = _run_transpose(hip, dev, from_dev(xs), w, b, s, pad)
    assert np.array_equal(fused.view(np.uint32), two_step.view(np.uint32))
