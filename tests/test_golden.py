"""The oracle against the reference's own outputs stored in
tests/golden/reference_sampling.npz (written by tests/golden/make_golden.py
from src/levo-sampling.cpp and src/levo-renderer-pattern.cpp compiled from the
reference checkout). Runs without the reference: the fixture is data."""
from __future__ import annotations

import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_sampling.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("scale", [1.5, 2.0, 0.0])
def test_cfg_matches_reference_bit_for_bit(oracle, gold, scale):
    key = str(scale).replace(".", "p")
    c, u = gold["cfg_cond"], gold["cfg_uncond"]
    got = oracle.apply_cfg(c, u, scale)
    assert np.array_equal(_bits(got), _bits(gold[f"cfg_apply_{key}"]))
    # combine_renderer_cfg(uncond, cond, g) is the same two-rounding formula
    assert np.array_equal(_bits(got), _bits(gold[f"cfg_renderer_{key}"]))


def test_single_row_sampler_tokens_and_cursor(oracle, gold):
    rows = gold["one_rows"].astype(np.float32)
    rng, draws = oracle.mt(int(gold["one_seed"][0])), 0
    for i in range(rows.shape[0]):
        tok, draws = oracle.sample_top_k(rows[i], int(gold["one_k"][i]), float(gold["one_t"][i]),
                                         bool(gold["one_use"][i]), rng, draws)
        assert tok == gold["one_tokens"][i], i
        assert draws == gold["one_draws"][i], i


@pytest.mark.parametrize("seed", [77, 78, 79])
def test_stream_generation_loop(oracle, gold, seed):
    cond, uncond = gold["streams_cond"].astype(np.float32), gold["streams_uncond"].astype(np.float32)
    P, S, V = cond.shape
    temp, use = gold[f"streams_params_{seed}"]
    window = int(gold["streams_window"][0])
    penalty = float(gold["streams_penalty"][0])
    rng, draws = oracle.mt(seed), 0
    history = [[] for _ in range(S)]
    for p in range(P):
        adjusted = oracle.apply_cfg(cond[p], uncond[p], 1.5)
        width = min(window, len(history[0]))
        recent = None
        if width:
            recent = np.array([h[-width:] for h in history], np.int64)
        toks, draws = oracle.sample_streams(adjusted, use_sampling=bool(use), temperature=float(temp),
                                            top_k_mixed=50, top_k_detail=1, repetition_penalty=penalty,
                                            recent=recent, ignore=gold["streams_ignore"], rng=rng, draws=draws)
        assert toks.tolist() == gold[f"streams_tokens_{seed}"][p].tolist(), p
        assert draws == gold[f"streams_draws_{seed}"][p], p
        for q in range(S):
            history[q].append(int(toks[q]))


@pytest.mark.parametrize("steps", [1, 2, 3, 7, 50])
def test_euler_time_grid(oracle, gold, steps):
    """The oracle's Euler step at t = step * dt with dt = 1.0f / steps: driving
    lo_flow_incontext over the reference's grid reproduces its noise-scale
    interpolation for a unit noise and zero context."""
    times, dt = gold[f"euler_times_{steps}"], np.float32(gold[f"euler_dt_{steps}"][0])
    assert dt == np.float32(1.0) / np.float32(steps)
    for i in range(steps + 1):
        t = np.float32(i) * dt
        assert t.view(np.uint32) == times[i].view(np.uint32)
        state = np.zeros(4, np.float32)
        oracle.flow_incontext(state, np.ones(4, np.float32), np.zeros(4, np.float32), 4, float(t), 0.1)
        want = np.float32(1.0) - np.float32(1.0 - np.float32(0.1)) * t
        assert state[0].view(np.uint32) == np.float32(want).view(np.uint32)


def test_repetition_penalty(oracle, gold):
    got = oracle.repetition_penalty(gold["pen_logits"], gold["pen_recent"], 1.1, 0)
    assert np.array_equal(_bits(got), _bits(gold["pen_out_full"]))
    got = oracle.repetition_penalty(gold["pen_logits"], gold["pen_recent"], 2.0, 299)
    assert np.array_equal(_bits(got), _bits(gold["pen_out_limit"]))
