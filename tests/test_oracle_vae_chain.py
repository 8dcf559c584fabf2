"""The oracle's F32 chain of the VAE decoder (vae_decoder::decode,
src/levo-vae.cpp:172-276) against the same graph in float64: at one and two
latent frames the F32 chain stays within 1e-5 of the output's scale of the
exact result. A wrong padding, dilation, crop, stride or SnakeBeta parameter
mapping in either chain moves the output by orders of magnitude more."""
from __future__ import annotations

import numpy as np
import pytest

from vae_chain import Weights, decode_f64, oracle_decode, scaled_err


@pytest.mark.parametrize("frames", [1, 2])
def test_oracle_chain_matches_float64(oracle, binding, frames):
    w = Weights(binding, 1234 + frames)
    latent = oracle.gaussian(64 * frames, 99 + frames).reshape(64, frames)
    got = oracle_decode(oracle, w, latent)
    exact = decode_f64(w, latent)
    assert got.shape == exact.shape == (2, 1920 * frames)
    err = scaled_err(got, exact)
    print(f"frames {frames}: max|y| {np.abs(exact).max():.3g}, scaled err {err:.3g}")
    assert err <= 1e-5


@pytest.mark.parametrize("mistake", [dict(dilations=(1, 1, 1)), dict(tap_order=-1)])
def test_float64_chain_detects_planted_mistakes(oracle, binding, mistake):
    """A chain with the residual units' dilations all 1, or with the
    upsamplers' taps reversed (same shapes), lands far outside the bar."""
    w = Weights(binding, 1235)
    latent = oracle.gaussian(64, 100).reshape(64, 1)
    wrong = oracle_decode(oracle, w, latent, **mistake)
    assert scaled_err(wrong, decode_f64(w, latent)) > 1e-2
