"""The whole VAE decoder (levo_hip_vae_decode) against the oracle's chain of
the same operations in the reference's order (vae_decoder::decode,
src/levo-vae.cpp:172-276): input conv, five stages of SnakeBeta +
ConvTranspose1d upsample and three residual units, SnakeBeta + output conv.

Random weights of the reference's shapes (no checkpoint is available); one
and two latent frames, as the reference's own first VAE fixtures use
(docs/renderer-parity.md). Two bars, both 1e-5:
- against the oracle's F32 chain, max |gpu - oracle| / max(|oracle|, 1)
  (measured 1.2e-7 to 1.9e-7; the decoder's outputs are below 1, so this is
  an absolute error);
- against the same graph in float64 (tests/vae_chain.py), the error at the
  signal's scale, max |gpu - exact| / max |exact| (measured 1.2e-6 to
  1.5e-6, as close as the oracle's own F32 chain, 1.3e-6 to 1.6e-6).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev
from vae_chain import Weights, decode_f64, oracle_decode, scaled_err

pytestmark = pytest.mark.gpu


def to_f16_params(oracle, w):
    """The same weights with every SnakeBeta parameter stored as F16 (the
    reference's F16 artifacts keep them so; they widen exactly)."""
    narrow = lambda pair: tuple(oracle.f32_to_f16(a) for a in pair)
    widen = lambda pair: tuple(oracle.f16_to_f32(a) for a in pair)
    w16, w32 = Weights.__new__(Weights), Weights.__new__(Weights)
    for dst, f in ((w16, narrow), (w32, lambda pr: widen(narrow(pr)))):
        dst.input, dst.out_w = w.input, w.out_w
        dst.out_act = f(w.out_act)
        dst.stages = [dict(act=f(sg["act"]), up=sg["up"],
                           res=[dict(pre=f(r["pre"]), conv0=r["conv0"], post=f(r["post"]), conv1=r["conv1"])
                                for r in sg["res"]]) for sg in w.stages]
    return w16, w32


def device_weights(hip, binding, dev, w):
    import torch
    keep = []

    def put(a):
        if a is None:
            return None
        t = to_dev(a, dev)
        keep.append(t)
        return t.data_ptr()

    dw = binding.VaeDecoderWeights()
    dw.input.weight, dw.input.bias = put(w.input[0]), put(w.input[1])
    for s, sg in enumerate(w.stages):
        st = binding.VAE_STRIDES[s]
        ci, co = binding.VAE_IN_WIDTH[s], binding.VAE_OUT_WIDTH[s]
        stage = dw.stage[s]
        stage.activation.alpha_log, stage.activation.beta_log = put(sg["act"][0]), put(sg["act"][1])
        packed = torch.empty(st * co * ci * 2, dtype=torch.float32, device=dev)
        keep.append(packed)
        raw = to_dev(sg["up"][0], dev)
        hip.conv_transpose1d_pack_weights(raw, packed, ci, co, st)
        keep.append(raw)
        stage.upsample.weight, stage.upsample.bias = packed.data_ptr(), put(sg["up"][1])
        for r in range(3):
            ru, dr = sg["res"][r], stage.residual[r]
            dr.pre.alpha_log, dr.pre.beta_log = put(ru["pre"][0]), put(ru["pre"][1])
            dr.conv_0.weight, dr.conv_0.bias = put(ru["conv0"][0]), put(ru["conv0"][1])
            dr.post.alpha_log, dr.post.beta_log = put(ru["post"][0]), put(ru["post"][1])
            dr.conv_1.weight, dr.conv_1.bias = put(ru["conv1"][0]), put(ru["conv1"][1])
    dw.output_activation.alpha_log, dw.output_activation.beta_log = put(w.out_act[0]), put(w.out_act[1])
    dw.output_weight = put(w.out_w)
    dw.param_type = 1 if w.out_act[0].dtype == np.uint16 else 0
    return dw, keep


@pytest.mark.parametrize("frames", [1, 2])
def test_decoder_matches_oracle_chain(hip, binding, dev, oracle, frames):
    import torch
    w = Weights(binding, 1234 + frames)
    latent = oracle.gaussian(64 * frames, 99 + frames).reshape(64, frames)
    want = oracle_decode(oracle, w, latent)
    dw, keep = device_weights(hip, binding, dev, w)
    nbytes = hip.vae_decode_workspace_bytes(frames)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    audio = torch.full((2, frames * 1920), float("nan"), dtype=torch.float32, device=dev)
    hip.vae_decode(dw, to_dev(latent, dev), frames, audio, ws, nbytes)
    got = from_dev(audio)
    exact = decode_f64(w, latent)
    err = f32_err(got, want)
    e_gpu, e_orc = scaled_err(got, exact), scaled_err(want, exact)
    print(f"frames {frames}: max|y| {np.abs(exact).max():.3g}, err vs oracle {err:.3g}, "
          f"scaled err vs float64: gpu {e_gpu:.3g}, oracle {e_orc:.3g}")
    assert got.shape == (2, frames * 1920)
    assert np.isfinite(got).all()
    assert err <= 1e-5
    assert e_gpu <= 1e-5


def test_decoder_f16_snake_parameters(hip, binding, dev, oracle):
    """F16 SnakeBeta parameters (param_type F16) widen exactly: the decode
    equals the oracle chain over the widened values to the same bar."""
    import torch
    frames = 1
    w16, w32 = to_f16_params(oracle, Weights(binding, 4321))
    latent = oracle.gaussian(64 * frames, 17).reshape(64, frames)
    want = oracle_decode(oracle, w32, latent)
    dw, keep = device_weights(hip, binding, dev, w16)
    assert dw.param_type == 1
    nbytes = hip.vae_decode_workspace_bytes(frames)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    audio = torch.full((2, frames * 1920), float("nan"), dtype=torch.float32, device=dev)
    hip.vae_decode(dw, to_dev(latent, dev), frames, audio, ws, nbytes)
    got = from_dev(audio)
    assert np.isfinite(got).all()
    err = f32_err(got, want)
    e_gpu = scaled_err(got, decode_f64(w32, latent))
    print(f"f16 parameters: err vs oracle {err:.3g}, scaled err vs float64 {e_gpu:.3g}")
    assert err <= 1e-5
    assert e_gpu <= 1e-5


def fill_pointers(struct, address):
    """Every pointer field of a VaeDecoderWeights (nested) set to address."""
    import ctypes
    for name, kind in struct._fields_:
        value = getattr(struct, name)
        if isinstance(value, ctypes.Array):
            for item in value:
                fill_pointers(item, address)
        elif isinstance(value, ctypes.Structure):
            fill_pointers(value, address)
        elif kind is ctypes.c_void_p:
            setattr(struct, name, address)


def test_decoder_rejects_bad_arguments(hip, binding, dev):
    """validate_weights (src/levo-vae.cpp:56-78) and the frame / workspace
    checks, each before any launch."""
    import torch
    dw = binding.VaeDecoderWeights()
    ws = torch.empty(16, dtype=torch.float32, device=dev)
    lat = torch.zeros(64, device=dev)
    audio = torch.zeros(2 * 1920, device=dev)
    with pytest.raises(binding.LevoHipError, match="convolution weight must be present"):
        hip.vae_decode(dw, lat, 1, audio, ws, hip.vae_decode_workspace_bytes(1))
    fill_pointers(dw, ws.data_ptr())
    hip.vae_validate_weights(dw)
    dw.stage[3].residual[2].pre.alpha_log = None
    with pytest.raises(binding.LevoHipError, match="SnakeBeta alpha must be present"):
        hip.vae_validate_weights(dw)
    dw.stage[3].residual[2].pre.alpha_log = ws.data_ptr()
    dw.param_type = 8
    with pytest.raises(binding.LevoHipError, match="F32 or F16"):
        hip.vae_validate_weights(dw)
    dw.param_type = 0
    with pytest.raises(binding.LevoHipError, match="workspace smaller"):
        hip.vae_decode(dw, lat, 1, audio, ws, 64)
    with pytest.raises(binding.LevoHipError, match="frame count"):
        hip.vae_decode(dw, lat, 0, audio, ws, 64)
    assert hip.vae_decode_workspace_bytes(1) == 3 * 128 * 1920 * 4
    assert hip.vae_decode_workspace_bytes(0) < 0


def test_decoder_stage_outputs(hip, binding, dev, oracle):
    """Stage capture: stage s's output equals the oracle chain's, and the
    audio is bit-identical to a decode without capture."""
    import torch
    frames = 1
    w = Weights(binding, 77)
    latent = oracle.gaussian(64 * frames, 5).reshape(64, frames)
    dw, keep = device_weights(hip, binding, dev, w)
    nbytes = hip.vae_decode_workspace_bytes(frames)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    lat = to_dev(latent, dev)
    plain = torch.empty(2, 1920 * frames, device=dev)
    hip.vae_decode(dw, lat, frames, plain, ws, nbytes)
    lens = np.cumprod(binding.VAE_STRIDES) * frames
    stages = [torch.full((c, n), float("nan"), device=dev) for c, n in zip(binding.VAE_OUT_WIDTH, lens)]
    stages[2] = None
    audio = torch.empty_like(plain)
    hip.vae_decode(dw, lat, frames, audio, ws, nbytes, stage_outputs=stages)
    torch.cuda.synchronize()
    assert torch.equal(audio, plain)
    # the oracle's stage outputs, recomputed stage by stage
    h = oracle.conv1d(latent, w.input[0], w.input[1], 3, 1, threads=8)
    for s, sg in enumerate(w.stages):
        st = binding.VAE_STRIDES[s]
        y = oracle.conv_transpose1d(oracle.snake_beta(h, *sg["act"], threads=8), sg["up"][0], sg["up"][1], st,
                                    (st + 1) // 2)
        for r, d in enumerate(binding.VAE_DILATIONS):
            ru = sg["res"][r]
            t = oracle.conv1d(oracle.snake_beta(y, *ru["pre"], threads=8), ru["conv0"][0], ru["conv0"][1], 3 * d, d,
                              threads=8)
            t = oracle.conv1d(oracle.snake_beta(t, *ru["post"], threads=8), ru["conv1"][0], ru["conv1"][1], 0, 1,
                              threads=8)
            y = (y + t).astype(np.float32)
        h = y
        if stages[s] is not None:
            err = f32_err(from_dev(stages[s]), y)
            print(f"stage {s}: err {err:.3g}")
            assert err <= 1e-5


# ---- one residual unit (levo_hip_vae_residual_unit, run_residual) -------------

def _unit_weights(rng, c, bias=True):
    f32 = lambda a: np.ascontiguousarray(a, np.float32)
    snake = lambda: (f32(rng.standard_normal(c) * 0.3), f32(rng.standard_normal(c) * 0.3))
    w0 = f32(rng.standard_normal((c, c, 7)) * (0.5 / np.sqrt(c * 7)))
    w1 = f32(rng.standard_normal((c, c, 1)) * (0.3 / np.sqrt(c)))
    b0 = f32(rng.standard_normal(c) * 0.05) if bias else None
    b1 = f32(rng.standard_normal(c) * 0.05) if bias else None
    return dict(pre=snake(), conv0=(w0, b0), post=snake(), conv1=(w1, b1))


def _unit_oracle(oracle, ru, x, d):
    t = oracle.conv1d(oracle.snake_beta(x, *ru["pre"], threads=8), ru["conv0"][0], ru["conv0"][1], 3 * d, d, threads=8)
    t = oracle.conv1d(oracle.snake_beta(t, *ru["post"], threads=8), ru["conv1"][0], ru["conv1"][1], 0, 1, threads=8)
    return (x + t).astype(np.float32)


def _unit_struct(binding, dev, ru, misalign_w0=False):
    import torch
    keep = []

    def put(a, shift=0):
        if a is None:
            return None
        t = torch.empty(a.size + shift, dtype=torch.float32 if a.dtype == np.float32 else torch.int16, device=dev)
        t[shift:] = torch.from_numpy(a.view(np.float32 if a.dtype == np.float32 else np.int16).ravel()).to(dev)
        keep.append(t)
        return t.data_ptr() + shift * t.element_size()

    u = binding.VaeResidual()
    u.pre.alpha_log, u.pre.beta_log = put(ru["pre"][0]), put(ru["pre"][1])
    u.conv_0.weight, u.conv_0.bias = put(ru["conv0"][0], 1 if misalign_w0 else 0), put(ru["conv0"][1])
    u.post.alpha_log, u.post.beta_log = put(ru["post"][0]), put(ru["post"][1])
    u.conv_1.weight, u.conv_1.bias = put(ru["conv1"][0]), put(ru["conv1"][1])
    return u, keep


def _run_unit(hip, dev, u, x, d, param_type=0):
    import torch
    c, t = x.shape
    y = torch.full((c, t), float("nan"), dtype=torch.float32, device=dev)
    h = torch.full((c, t), float("nan"), dtype=torch.float32, device=dev)
    hip.vae_residual_unit(to_dev(x, dev), c, t, u, d, y, h, param_type=param_type)
    return from_dev(y)


@pytest.mark.parametrize("c,t,d", [(128, 3000, 1), (128, 1001, 3), (128, 517, 9), (128, 128, 9), (128, 1, 1),
                                   (64, 700, 3), (256, 300, 9)])
def test_residual_unit(hip, binding, dev, oracle, c, t, d):
    """128 channels run as one launch (the k = 1 conv in the k = 7 conv's
    epilogue); other widths as the two fused SnakeBeta + conv launches.
    Lengths off the 128-sample tile and off 4 (the scalar epilogue)."""
    rng = np.random.default_rng(c + t + d)
    ru = _unit_weights(rng, c)
    x = oracle.gaussian(c * t, 7 * t + d).reshape(c, t)
    u, keep = _unit_struct(binding, dev, ru)
    assert f32_err(_run_unit(hip, dev, u, x, d), _unit_oracle(oracle, ru, x, d)) <= 1e-5


def test_residual_unit_f16_params_no_bias_and_unfused_twin(hip, binding, dev, oracle):
    """F16 SnakeBeta parameters (widened exactly), null biases, and the same
    128-channel unit with a misaligned conv_0 weight, which takes the
    two-launch path: both agree with the oracle."""
    rng = np.random.default_rng(77)
    c, t, d = 128, 2000, 3
    ru = _unit_weights(rng, c, bias=False)
    x = oracle.gaussian(c * t, 78).reshape(c, t)
    want = _unit_oracle(oracle, ru, x, d)
    u, keep = _unit_struct(binding, dev, ru)
    fused = _run_unit(hip, dev, u, x, d)
    assert f32_err(fused, want) <= 1e-5
    u2, keep2 = _unit_struct(binding, dev, ru, misalign_w0=True)
    assert f32_err(_run_unit(hip, dev, u2, x, d), want) <= 1e-5
    ru16 = dict(ru, pre=tuple(oracle.f32_to_f16(a) for a in ru["pre"]),
                post=tuple(oracle.f32_to_f16(a) for a in ru["post"]))
    ru16w = dict(ru, pre=tuple(oracle.f16_to_f32(a) for a in ru16["pre"]),
                 post=tuple(oracle.f16_to_f32(a) for a in ru16["post"]))
    u3, keep3 = _unit_struct(binding, dev, ru16)
    assert f32_err(_run_unit(hip, dev, u3, x, d, param_type=1), _unit_oracle(oracle, ru16w, x, d)) <= 1e-5


def test_residual_unit_rejects(hip, binding, dev):
    import torch
    rng = np.random.default_rng(5)
    ru = _unit_weights(rng, 128)
    u, keep = _unit_struct(binding, dev, ru)
    x = torch.zeros((128, 256), device=dev)
    h = torch.zeros((128, 256), device=dev)
    with pytest.raises(binding.LevoHipError, match="must not overlap"):
        hip.vae_residual_unit(x, 128, 256, u, 1, x, h)
    with pytest.raises(binding.LevoHipError, match="must not overlap"):
        hip.vae_residual_unit(x, 128, 256, u, 1, x[:, 4:], h)
    with pytest.raises(binding.LevoHipError, match="null tensor"):
        hip.vae_residual_unit(x, 128, 256, u, 1, torch.zeros((128, 256), device=dev), None)
    with pytest.raises(binding.LevoHipError, match="dilation"):
        hip.vae_residual_unit(x, 128, 256, u, 0, torch.zeros((128, 256), device=dev), h)
    with pytest.raises(binding.LevoHipError, match="invalid shape"):  # checked before any access
        hip.vae_residual_unit(x, 128, 1 << 37, u, 1, torch.zeros((128, 256), device=dev), h)
    for channels in (128, 64):  # one-launch and two-launch widths reject it alike
        with pytest.raises(binding.LevoHipError, match="F32 or F16"):
            hip.vae_residual_unit(x[:channels], channels, 256, u, 1, torch.zeros((channels, 256), device=dev),
                                  h[:channels], param_type=8)


# ---- the decode as its public steps ------------------------------------------

def _compose_decode(hip, binding, dev, w, latent):
    """decode through the public entry points, in the decoder's order:
    levo_hip_snake_conv1d_split (input conv; each two-launch unit's conv_0,
    then conv_1 with the post SnakeBeta and the residual),
    levo_hip_snake_conv_transpose1d_split, levo_hip_vae_residual_unit (the
    one-launch 128-channel units) and levo_hip_snake_conv1d (output conv).
    Each split call gets the workspace the decoder gives it: the free tail of
    the workspace buffer its output lives in (a third of
    levo_hip_vae_decode_workspace_bytes, after the output rounded up to 64
    floats), so both split alike."""
    import torch
    frames = latent.shape[1]
    n_buf = hip.vae_decode_workspace_bytes(frames) // 4 // 3
    tail = lambda out_floats: n_buf - (out_floats + 63) // 64 * 64
    keep = []

    def d(a):
        if a is None:
            return None
        t = to_dev(a, dev)
        keep.append(t)
        return t

    def conv(x, ci, t, wb, co, k, pad, dil, act=None, res=None):
        t_out = t + 2 * pad - dil * (k - 1)
        y = torch.empty((co, t_out), dtype=torch.float32, device=dev)
        n = tail(co * t_out)
        ws = torch.empty(n, dtype=torch.float32, device=dev)
        keep.extend([y, ws])
        hip.snake_conv1d_split(x, ci, t, d(wb[0]), co, k, workspace=ws, workspace_floats=n,
                               alpha_log=d(act[0]) if act else None, beta_log=d(act[1]) if act else None,
                               bias=d(wb[1]), padding=pad, dilation=dil, residual=res, y=y)
        return y

    x = conv(d(latent), 64, frames, w.input, 2048, 7, 3, 1)
    length = frames
    for s, sg in enumerate(w.stages):
        st = binding.VAE_STRIDES[s]
        ci, co = binding.VAE_IN_WIDTH[s], binding.VAE_OUT_WIDTH[s]
        packed = torch.empty(st * co * ci * 2, dtype=torch.float32, device=dev)
        hip.conv_transpose1d_pack_weights(d(sg["up"][0]), packed, ci, co, st)
        y = torch.empty((co, length * st), dtype=torch.float32, device=dev)
        n = tail(co * length * st)
        ws = torch.empty(n, dtype=torch.float32, device=dev)
        keep.extend([packed, y, ws])
        hip.snake_conv_transpose1d_split(x, ci, length, packed, co, st, workspace=ws, workspace_floats=n,
                                         alpha_log=d(sg["act"][0]), beta_log=d(sg["act"][1]), bias=d(sg["up"][1]),
                                         padding=(st + 1) // 2, y=y)
        x, length = y, length * st
        for r, dil in enumerate((1, 3, 9)):
            ru = sg["res"][r]
            if co == 128:
                u, k2 = _unit_struct(binding, dev, ru)
                keep.extend(k2)
                y = torch.empty((co, length), dtype=torch.float32, device=dev)
                h = torch.empty((co, length), dtype=torch.float32, device=dev)
                keep.extend([y, h])
                hip.vae_residual_unit(x, co, length, u, dil, y, h)
            else:
                h = conv(x, co, length, ru["conv0"], co, 7, 3 * dil, dil, act=ru["pre"])
                y = conv(h, co, length, ru["conv1"], co, 1, 0, 1, act=ru["post"], res=x)
            x = y
    audio = torch.empty((2, length), dtype=torch.float32, device=dev)
    hip.snake_conv1d(x, 128, length, d(w.out_w), 2, 7, alpha_log=d(w.out_act[0]), beta_log=d(w.out_act[1]),
                     padding=3, y=audio)
    torch.cuda.synchronize()
    return from_dev(audio)


@pytest.mark.parametrize("frames", [1, 3])
def test_decoder_equals_its_public_steps(hip, binding, dev, oracle, frames):
    """Bit for bit: the decoder stores each two-launch unit's conv_0 output
    through the post SnakeBeta (one evaluation per sample in the epilogue or
    the split combine) where the public steps apply it in conv_1's staging;
    both compute snake(h) from the same F32 h with the same parameters."""
    import torch
    w = Weights(binding, 4321 + frames)
    latent = oracle.gaussian(64 * frames, 17 + frames).reshape(64, frames)
    dw, keep = device_weights(hip, binding, dev, w)
    nbytes = hip.vae_decode_workspace_bytes(frames)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    audio = torch.full((2, frames * 1920), float("nan"), dtype=torch.float32, device=dev)
    hip.vae_decode(dw, to_dev(latent, dev), frames, audio, ws, nbytes)
    got = from_dev(audio)
    want = _compose_decode(hip, binding, dev, w, latent)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
