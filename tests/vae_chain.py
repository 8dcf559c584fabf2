"""The VAE decoder's graph (vae_decoder::decode, src/levo-vae.cpp:172-276)
for the decoder tests: random weights of the reference's shapes, the
oracle's F32 chain of the same operations in the reference's order, and the
same graph evaluated in float64 (numpy: convolutions as im2col products,
transposed convolutions as scattered per-tap products, SnakeBeta from its
closed form x + sin^2(alpha x) / beta).

The float64 chain is the exact result the F32 implementations approximate:
it pins the oracle's chain (a wrong padding, dilation, stride or parameter
mapping moves the result by far more than F32 rounding does) and gives the
GPU decode a bar set by F32 rounding, not by the distance between two F32
summation orders.
"""
from __future__ import annotations

import numpy as np

STRIDES = (10, 6, 4, 4, 2)
DILATIONS = (1, 3, 9)


class Weights:
    """Host copies of one decoder's weights, drawn from a seeded generator."""

    def __init__(self, binding, seed):
        rng = np.random.default_rng(seed)
        f32 = lambda a: np.ascontiguousarray(a, np.float32)

        def conv(c_out, c_in, k, bias=True, gain=0.5):
            w = f32(rng.standard_normal((c_out, c_in, k)) * (gain / np.sqrt(c_in * k)))
            b = f32(rng.standard_normal(c_out) * 0.05) if bias else None
            return w, b

        def snake(c):
            return f32(rng.standard_normal(c) * 0.3), f32(rng.standard_normal(c) * 0.3)

        self.input = conv(2048, 64, 7)
        self.stages = []
        for s, (ci, co) in enumerate(zip(binding.VAE_IN_WIDTH, binding.VAE_OUT_WIDTH)):
            st = binding.VAE_STRIDES[s]
            up_w = f32(rng.standard_normal((ci, co, 2 * st)) * (0.5 / np.sqrt(2 * ci)))
            up_b = f32(rng.standard_normal(co) * 0.05)
            res = [dict(pre=snake(co), conv0=conv(co, co, 7), post=snake(co), conv1=conv(co, co, 1, gain=0.3))
                   for _ in range(3)]
            self.stages.append(dict(act=snake(ci), up=(up_w, up_b), res=res))
        self.out_act = snake(128)
        self.out_w = conv(2, 128, 7, bias=False)[0]


def oracle_decode(oracle, w, latent, dilations=DILATIONS, tap_order=1):
    """vae_decoder::decode's graph with the oracle's F32 operations.
    dilations and tap_order (-1 reverses the upsamplers' taps) exist to plant
    mistakes in tests of the float64 chain's sensitivity."""
    h = oracle.conv1d(latent, w.input[0], w.input[1], 3, 1, threads=8)
    for s, sg in enumerate(w.stages):
        st = STRIDES[s]
        x = oracle.snake_beta(h, *sg["act"], threads=8)
        y = oracle.conv_transpose1d(x, sg["up"][0][:, :, ::tap_order], sg["up"][1], st, (st + 1) // 2)
        for r, d in enumerate(dilations):
            ru = sg["res"][r]
            t = oracle.conv1d(oracle.snake_beta(y, *ru["pre"], threads=8), ru["conv0"][0], ru["conv0"][1], 3 * d, d,
                              threads=8)
            t = oracle.conv1d(oracle.snake_beta(t, *ru["post"], threads=8), ru["conv1"][0], ru["conv1"][1], 0, 1,
                              threads=8)
            y = (y + t).astype(np.float32)
        h = y
    return oracle.conv1d(oracle.snake_beta(h, *w.out_act, threads=8), w.out_w, None, 3, 1, threads=8)


# ---- the same graph in float64 ------------------------------------------------------

def snake_f64(x, alpha_log, beta_log):
    """x + sin^2(alpha x) / (beta + 1e-9), alpha = e^alpha_log, beta = e^beta_log
    (src/levo-audio-ops.cpp:146-151)."""
    a = np.exp(alpha_log.astype(np.float64))[:, None]
    b = (np.exp(beta_log.astype(np.float64)) + 1e-9)[:, None]
    return x + np.sin(a * x) ** 2 / b


def conv1d_f64(x, w, bias, padding, dilation):
    """Stride-1 Conv1d, x [c_in][t], w [c_out][c_in][k], as one im2col product."""
    c_in, t = x.shape
    c_out, _, k = w.shape
    xp = np.pad(x, ((0, 0), (padding, padding)))
    t_out = t + 2 * padding - dilation * (k - 1)
    cols = np.stack([xp[:, j * dilation: j * dilation + t_out] for j in range(k)], axis=1)
    y = w.astype(np.float64).reshape(c_out, c_in * k) @ cols.reshape(c_in * k, t_out)
    return y if bias is None else y + bias.astype(np.float64)[:, None]


def conv_transpose1d_f64(x, w, bias, stride, padding):
    """ConvTranspose1d, x [c_in][t], w [c_in][c_out][k]: input sample i adds
    w[:, :, j] . x[:, i] to output sample i * stride + j, then the crop."""
    c_in, t = x.shape
    _, c_out, k = w.shape
    taps = np.tensordot(w.astype(np.float64), x, axes=([0], [0]))  # [c_out][k][t]
    full = np.zeros((c_out, (t - 1) * stride + k))
    for i in range(t):
        full[:, i * stride: i * stride + k] += taps[:, :, i]
    return full[:, padding: full.shape[1] - padding] + bias.astype(np.float64)[:, None]


def decode_f64(w, latent):
    h = conv1d_f64(latent.astype(np.float64), w.input[0], w.input[1], 3, 1)
    for s, sg in enumerate(w.stages):
        st = STRIDES[s]
        y = conv_transpose1d_f64(snake_f64(h, *sg["act"]), sg["up"][0], sg["up"][1], st, (st + 1) // 2)
        for r, d in enumerate(DILATIONS):
            ru = sg["res"][r]
            t = conv1d_f64(snake_f64(y, *ru["pre"]), ru["conv0"][0], ru["conv0"][1], 3 * d, d)
            y = y + conv1d_f64(snake_f64(t, *ru["post"]), ru["conv1"][0], ru["conv1"][1], 0, 1)
        h = y
    return conv1d_f64(snake_f64(h, *w.out_act), w.out_w, None, 3, 1)


def scaled_err(actual, exact):
    """max |actual - exact| over max |exact|: the error at the signal's scale."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(exact, np.float64)
    return float(np.max(np.abs(a - e)) / max(np.max(np.abs(e)), 1e-30))
