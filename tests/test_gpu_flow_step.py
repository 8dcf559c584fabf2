"""Device-resident Flow step: levo_hip_flow_assemble_input and
levo_hip_flow_step against the oracle's Euler solver loop
(src/levo-flow-renderer.cpp:57-120 with the CFG lambda :283-310,
append_model_row :35-53, the estimator's velocity slice
src/levo-flow-estimator.cpp:390-399 and denormalize_latents
src/levo-flow-conditioning.cpp:124-133).

The estimator is replaced by an elementwise stand-in that torch (on the GPU)
and numpy compute with the same F32 roundings: velocity =
(state_column * 0.5 - t) + conditioning_column * 0.25. Every output column
outside the velocity slice is NaN, so reading anything else trips the
finiteness flags. The bar is bit-exact: state after every step (the
reference's checkpoint), the next estimator input, the denormalized latents.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


class Window:
    """One Flow window's tensors (host copies) and their layout."""

    def __init__(self, oracle, frames, latent, mask_dim, cond_width, prefix, seed):
        self.F, self.L, self.M, self.C, self.P = frames, latent, mask_dim, cond_width, prefix
        self.H = mask_dim + 2 * latent + cond_width
        g = lambda n, s, scale=1.0: (oracle.gaussian(n, seed * 100 + s) * np.float32(scale)).astype(np.float32)
        self.mask = g(frames * mask_dim, 1).reshape(frames, mask_dim)
        self.ctx = g(frames * latent, 2).reshape(frames, latent)
        self.cond = g(frames * cond_width, 3).reshape(frames, cond_width)
        self.noise = g(frames * latent, 4).reshape(frames, latent)
        self.mean = g(latent, 5, 0.1)
        self.stddev = (np.abs(g(latent, 6)) * np.float32(0.5) + np.float32(0.5)).astype(np.float32)

    def model_input(self, state, batch):
        """append_model_row for every row (src/levo-flow-renderer.cpp:35-53, :287-295)."""
        rows = []
        for b in range(batch):
            cond = np.zeros_like(self.cond) if (batch == 2 and b == 0) else self.cond
            rows.append(np.concatenate([self.mask, self.ctx, cond, state], axis=1))
        return np.stack(rows).astype(np.float32)

    def velocity_np(self, mi, t):
        xs = mi[:, :, self.H - self.L:]
        xc = mi[:, :, self.M + self.L:self.M + 2 * self.L]
        return ((xs * np.float32(0.5)) - np.float32(t)) + (xc * np.float32(0.25))

    def solve_oracle(self, oracle, steps, guidance, batch, start=0, state0=None):
        """solve_flow_euler with the stand-in estimator; returns the state
        after every step, the estimator input of every step, the final state
        and the denormalized latents."""
        state = (self.noise if state0 is None else state0).copy().reshape(-1)
        dt = np.float32(1.0) / np.float32(steps)
        states, inputs = [], []
        for k in range(start, steps):
            t = float(np.float32(k) * dt)
            oracle.flow_incontext(state, self.noise.reshape(-1), self.ctx.reshape(-1), self.P * self.L, t, 1e-4)
            mi = self.model_input(state.reshape(self.F, self.L), batch)
            inputs.append(mi)
            v = self.velocity_np(mi, t)
            vu = np.ascontiguousarray(v[0]).reshape(-1)
            vc = np.ascontiguousarray(v[1]).reshape(-1) if batch == 2 else None
            oracle.flow_cfg_euler(state, vu, vc, guidance, float(dt))
            states.append(state.copy())
        final = state.copy()
        final[: self.P * self.L] = self.ctx.reshape(-1)[: self.P * self.L]
        denorm = (final.reshape(self.F, self.L) * self.stddev + self.mean).astype(np.float32)
        return states, inputs, final, denorm


def _assemble(hip, binding, w, dev, d, batch, step, steps, state_dev):
    a = binding.FlowInputArgs()
    a.model_input, a.batch, a.frames = d["mi"].data_ptr(), batch, w.F
    a.mask_embedding, a.mask_dim = d["mask"].data_ptr(), w.M
    a.context, a.latent = d["ctx"].data_ptr(), w.L
    a.conditioning, a.condition_width = d["cond"].data_ptr(), w.C
    a.state, a.noise, a.prefix_frames = state_dev.data_ptr(), d["noise"].data_ptr(), w.P
    a.step, a.steps, a.sigma_min = step, steps, 1e-4
    hip.flow_assemble_input(a)


def _step_args(binding, w, d, batch, step, steps, guidance, state_dev, flags):
    a = binding.FlowStepArgs()
    a.state, a.output, a.out_pitch, a.vel_col = state_dev.data_ptr(), d["out"].data_ptr(), w.H, w.H - w.L
    a.batch, a.guidance, a.frames, a.latent = batch, guidance, w.F, w.L
    a.step, a.steps = step, steps
    a.noise, a.context, a.prefix_frames, a.sigma_min = d["noise"].data_ptr(), d["ctx"].data_ptr(), w.P, 1e-4
    a.next_input, a.in_pitch, a.state_col = d["mi"].data_ptr(), w.H, w.H - w.L
    a.mean, a.stddev, a.denormalized = d["mean"].data_ptr(), d["std"].data_ptr(), d["denorm"].data_ptr()
    a.nonfinite = flags.data_ptr()
    return a


def _device(w, dev, batch):
    import torch
    d = {k: to_dev(v, dev) for k, v in (("mask", w.mask), ("ctx", w.ctx), ("cond", w.cond), ("noise", w.noise),
                                          ("mean", w.mean), ("std", w.stddev))}
    d["mi"] = torch.full((batch, w.F, w.H), float("nan"), dtype=torch.float32, device=dev)
    d["out"] = torch.full((batch, w.F, w.H), float("nan"), dtype=torch.float32, device=dev)
    d["denorm"] = torch.full((w.F, w.L), float("nan"), dtype=torch.float32, device=dev)
    return d


def _estimate(w, d, t):
    """The stand-in estimator on the GPU, op by op (each op one rounding)."""
    mi = d["mi"]
    xs = mi[:, :, w.H - w.L:]
    xc = mi[:, :, w.M + w.L:w.M + 2 * w.L]
    d["out"][:, :, w.H - w.L:] = ((xs * 0.5) - t) + (xc * 0.25)


def _run_window(hip, binding, oracle, dev, w, steps, guidance, batch, start=0, state0=None):
    import torch
    states, inputs, final, denorm = w.solve_oracle(oracle, steps, guidance, batch, start, state0)
    d = _device(w, dev, batch)
    state = to_dev((w.noise if state0 is None else state0).reshape(-1).copy(), dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    _assemble(hip, binding, w, dev, d, batch, start, steps, state)
    dt = np.float32(1.0) / np.float32(steps)
    for i, k in enumerate(range(start, steps)):
        assert _eq(from_dev(d["mi"]), inputs[i]), f"estimator input of step {k}"
        t = float(np.float32(k) * dt)
        _estimate(w, d, t)
        hip.flow_step(_step_args(binding, w, d, batch, k, steps, guidance, state, flags))
        if k + 1 < steps:
            assert _eq(from_dev(state), states[i]), f"state after step {k}"
    assert int(from_dev(flags)[0]) == 0
    assert _eq(from_dev(state), final)
    assert _eq(from_dev(d["denorm"]), denorm)


def test_window_fifty_steps_cfg(hip, binding, dev, oracle):
    """LeVo's window: 1000 frames x 64 latent, rows of 24 | 64 | 2048 | 64 =
    2200, 250 in-context frames, 50 steps, guidance 1.5 (batch 2)."""
    w = Window(oracle, 1000, 64, 24, 2048, 250, seed=1)
    _run_window(hip, binding, oracle, dev, w, 50, 1.5, 2)


def test_window_without_cfg(hip, binding, dev, oracle):
    """guidance <= 1: batch 1, the estimator output is the velocity (:301)."""
    w = Window(oracle, 1000, 64, 24, 2048, 250, seed=2)
    _run_window(hip, binding, oracle, dev, w, 10, 1.0, 1)


def test_window_resumed_mid_solve(hip, binding, dev, oracle):
    """Resume at step 17 of 25 from a saved state (:75-86): the assembled
    input re-interpolates the prefix for step 17 and the rest matches."""
    w = Window(oracle, 1000, 64, 24, 2048, 250, seed=3)
    states, _, _, _ = w.solve_oracle(oracle, 25, 1.5, 2)
    _run_window(hip, binding, oracle, dev, w, 25, 1.5, 2, start=17, state0=states[16].reshape(w.F, w.L))


@pytest.mark.parametrize("frames,latent,mask_dim,cond_width,prefix", [
    (7, 5, 3, 6, 2),      # odd widths: one element per thread
    (33, 64, 24, 128, 0),  # no in-context prefix
    (9, 8, 4, 8, 9),       # every frame in context
])
def test_odd_shapes(hip, binding, dev, oracle, frames, latent, mask_dim, cond_width, prefix):
    w = Window(oracle, frames, latent, mask_dim, cond_width, prefix, seed=frames)
    _run_window(hip, binding, oracle, dev, w, 6, 1.5, 2)


@pytest.mark.parametrize("where", ["velocity", "state"])
def test_flags_nonfinite(hip, binding, dev, oracle, where):
    """A NaN velocity sets the velocity bit (and the state bit: the NaN
    reaches the state); an overflowing update sets only the state bit
    (:104, :106)."""
    import torch
    w = Window(oracle, 100, 64, 24, 2048, 25, seed=5)
    d = _device(w, dev, 2)
    state = to_dev(w.noise.reshape(-1).copy(), dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    _assemble(hip, binding, w, dev, d, 2, 0, 50, state)
    _estimate(w, d, 0.0)
    if where == "velocity":
        d["out"][1, 60, w.H - 3] = float("nan")
        want = 3
    else:
        state[70 * 64 + 5] = 3.4e38                 # frame 70 is past the prefix
        d["out"][:, 70, w.H - w.L + 5] = 3.0e38     # finite velocity; 3.4e38 + 0.02 * 3e38 overflows
        want = 2
    hip.flow_step(_step_args(binding, w, d, 2, 0, 50, 1.5, state, flags))
    assert int(from_dev(flags)[0]) == want


def test_rejects_bad_layouts(hip, binding, dev, oracle):
    w = Window(oracle, 10, 8, 4, 8, 2, seed=6)
    d = _device(w, dev, 2)
    state = to_dev(w.noise.reshape(-1).copy(), dev)
    import torch
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    a = _step_args(binding, w, d, 2, 0, 4, 1.5, state, flags)
    a.vel_col = w.H - w.L + 1
    with pytest.raises(binding.LevoHipError, match="velocity columns exceed"):
        hip.flow_step(a)
    a = _step_args(binding, w, d, 2, 4, 4, 1.5, state, flags)
    with pytest.raises(binding.LevoHipError, match="step out of range"):
        hip.flow_step(a)
    a = _step_args(binding, w, d, 2, 0, 4, 1.5, state, flags)
    a.prefix_frames = w.F + 1
    with pytest.raises(binding.LevoHipError, match="in-context length exceeds"):
        hip.flow_step(a)


@pytest.mark.parametrize("frames,latent,offset", [(1000, 64, 0), (37, 5, 0), (10, 64, 1)])
def test_normalize_denormalize(hip, dev, oracle, frames, latent, offset):
    """normalize_latents / denormalize_latents (src/levo-flow-conditioning.cpp:
    113-133): (x - mean) / stddev and x * stddev + mean, bit-exact; a
    non-finite input sets the flag (require_finite, :116, :128)."""
    import torch
    x = oracle.gaussian(frames * latent, 900 + latent).reshape(frames, latent)
    mean = (oracle.gaussian(latent, 901) * np.float32(0.1)).astype(np.float32)
    sd = (np.abs(oracle.gaussian(latent, 902)) + np.float32(0.5)).astype(np.float32)
    base = torch.zeros(frames * latent + offset, dtype=torch.float32, device=dev)
    xd = base[offset:]
    xd.copy_(torch.from_numpy(x.reshape(-1)))
    md, sdd = to_dev(mean, dev), to_dev(sd, dev)
    out = torch.empty(frames * latent + offset, dtype=torch.float32, device=dev)[offset:]
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.flow_normalize(xd, md, sdd, out, frames, latent, flags)
    assert _eq(from_dev(out).reshape(frames, latent), ((x - mean) / sd).astype(np.float32))
    hip.flow_denormalize(xd, md, sdd, out, frames, latent, flags)
    assert _eq(from_dev(out).reshape(frames, latent), (x * sd + mean).astype(np.float32))
    assert int(from_dev(flags)[0]) == 0
    xd[frames * latent // 2] = float("inf")
    hip.flow_denormalize(xd, md, sdd, out, frames, latent, flags)
    assert int(from_dev(flags)[0]) == 2
