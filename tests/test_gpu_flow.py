"""Flow Euler/CFG update and the CFG combine on the GPU.

The reference computes every product and sum here with two F32 roundings
(src/levo-flow-renderer.cpp:94-105, :307; src/levo-sampling.cpp:22-28), which
the kernels reproduce, so the bar is bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _eq(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_flow_euler_reference_kat(hip, dev):
    """tests/test-flow-renderer.cpp:33-65 driven through the device entry points."""
    import torch
    noise = to_dev(np.array([1, 2, 10, 20, 30, 40], np.float32), dev)
    ctx = to_dev(np.array([4, 8, 0, 0, 0, 0], np.float32), dev)
    ones = torch.ones(6, dtype=torch.float32, device=dev)
    state = noise.clone()
    steps, incontext, dim, sigma = 2, 1, 2, 0.1
    dt = np.float32(1.0) / np.float32(steps)
    seen = []
    for step in range(steps):
        t = float(np.float32(step) * dt)
        hip.flow_incontext(state, noise, ctx, incontext * dim, t, sigma)
        seen.append(from_dev(state).copy())
        hip.flow_cfg_euler(state, ones, None, 6, 1.0, float(dt))
    state[: incontext * dim] = ctx[: incontext * dim]
    out = from_dev(state)
    assert np.allclose(seen[0][:2], [1.0, 2.0], atol=1e-6)
    assert np.allclose(seen[1][:2], [2.55, 5.10], atol=1e-6)
    assert np.allclose(out, [4, 8, 11, 21, 31, 41], atol=1e-6)


def test_config_fifty_steps_bit_exact(hip, dev, oracle):
    """[1,64,2520] F32, dt = 1/50, g = 1.5, fresh seeded v_c, v_u every step."""
    n, steps, g = 64 * 2520, 50, 1.5
    dt = float(np.float32(1.0) / np.float32(steps))
    x0 = oracle.gaussian(n, 4242)
    want = x0.copy()
    state = to_dev(x0, dev)
    for s in range(steps):
        vu = oracle.gaussian(n, 10_000 + 2 * s)
        vc = oracle.gaussian(n, 10_001 + 2 * s)
        hip.flow_cfg_euler(state, to_dev(vu, dev), to_dev(vc, dev), n, g, dt)
        oracle.flow_cfg_euler(want, vu, vc, g, dt)
    assert _eq(from_dev(state), want)


@pytest.mark.parametrize("n,offset", [(1, 0), (3, 0), (7, 0), (4099, 0), (1000, 1), (4097, 3)])
def test_odd_sizes_and_unaligned(hip, dev, oracle, n, offset):
    import torch
    base = oracle.gaussian(n + offset, 8)
    vu = oracle.gaussian(n + offset, 9)
    vc = oracle.gaussian(n + offset, 10)
    sd, ud, cd = to_dev(base, dev), to_dev(vu, dev), to_dev(vc, dev)
    hip.flow_cfg_euler(sd[offset:], ud[offset:], cd[offset:], n, 1.5, 0.02)
    want = base[offset:].copy()
    oracle.flow_cfg_euler(want, vu[offset:].copy(), vc[offset:].copy(), 1.5, 0.02)
    got = from_dev(sd)
    assert _eq(got[offset:], want) and _eq(got[:offset], base[:offset])
    # no CFG: state += dt * v
    sd = to_dev(base, dev)
    hip.flow_cfg_euler(sd[offset:], ud[offset:], None, n, 1.5, 0.02)
    want = base[offset:].copy()
    oracle.flow_cfg_euler(want, vu[offset:].copy(), None, 1.5, 0.02)
    assert _eq(from_dev(sd)[offset:], want)
    del torch


def test_incontext_bit_exact(hip, dev, oracle):
    n, prefix = 64 * 1000, 64 * 250
    state0 = oracle.gaussian(n, 1)
    noise = oracle.gaussian(n, 2)
    ctx = oracle.gaussian(n, 3)
    for step in (0, 7, 49):
        t = float(np.float32(step) * (np.float32(1) / np.float32(50)))
        sd = to_dev(state0, dev)
        hip.flow_incontext(sd, to_dev(noise, dev), to_dev(ctx, dev), prefix, t, 1e-4)
        want = state0.copy()
        oracle.flow_incontext(want, noise, ctx, prefix, t, 1e-4)
        assert _eq(from_dev(sd), want)


def test_cfg_combine_kats_and_reference(hip, dev, oracle, ref):
    import torch
    out = torch.empty(2, dtype=torch.float32, device=dev)
    hip.cfg_combine(out, to_dev(np.array([1, 1], np.float32), dev), to_dev(np.array([2, 4], np.float32), dev), 2, 1.5)
    assert from_dev(out).tolist() == [2.5, 5.5]           # tests/test-sampling.cpp:8
    hip.cfg_combine(out, to_dev(np.array([1, 2], np.float32), dev), to_dev(np.array([3, 6], np.float32), dev), 2, 1.5)
    assert from_dev(out).tolist() == [4.0, 8.0]           # tests/test-renderer-pattern.cpp:88-90
    n = 3 * 16384 + 3
    c = oracle.gaussian(n, 31) * 3
    u = oracle.gaussian(n, 32) * 3
    out = torch.empty(n, dtype=torch.float32, device=dev)
    hip.cfg_combine(out, to_dev(u, dev), to_dev(c, dev), n, 1.5)
    got = from_dev(out)
    assert _eq(got, ref.apply_cfg(c, u, 1.5))
    assert _eq(got, ref.combine_renderer_cfg(u, c, 1.5))
    out2 = torch.empty(n + 1, dtype=torch.float32, device=dev)
    ud, cd = to_dev(np.concatenate([[0], u]).astype(np.float32), dev), to_dev(np.concatenate([[0], c]).astype(np.float32), dev)
    hip.cfg_combine(out2[1:], ud[1:], cd[1:], n, 1.5)   # unaligned scalar path
    assert _eq(from_dev(out2)[1:], got)


def test_fp16_row_converters(hip, dev, oracle):
    import torch
    bits = np.arange(0, 2**32, 65537 * 13, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)].copy()
    h = torch.empty(f.size, dtype=torch.int16, device=dev)
    hip.fp32_to_fp16_row(to_dev(f, dev), h, f.size)
    assert np.array_equal(from_dev(h).view(np.uint16), oracle.f32_to_f16(f))
    allh = np.arange(65536, dtype=np.uint16)
    out = torch.empty(65536, dtype=torch.float32, device=dev)
    hip.fp16_to_fp32_row(to_dev(allh.view(np.int16), dev), out, 65536)
    got, want = from_dev(out), oracle.f16_to_f32(allh)
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32)) and np.all(np.isnan(got[~ok]))
    # rows that start off the 16-byte grid (the scalar path) and a ragged tail
    fd = to_dev(np.concatenate([[0], f]).astype(np.float32), dev)
    h2 = torch.empty(f.size + 1, dtype=torch.int16, device=dev)
    hip.fp32_to_fp16_row(fd[1:], h2[1:], f.size - 3)
    assert np.array_equal(from_dev(h2)[1:f.size - 2].view(np.uint16), oracle.f32_to_f16(f[:f.size - 3]))
    hd = to_dev(np.concatenate([np.zeros(1, np.uint16), allh]).view(np.int16), dev)
    out2 = torch.empty(65537, dtype=torch.float32, device=dev)
    hip.fp16_to_fp32_row(hd[1:], out2[1:], 65533)
    got2 = from_dev(out2)[1:65534]
    assert np.array_equal(got2[ok[:65533]].view(np.uint32), want[:65533][ok[:65533]].view(np.uint32))


@pytest.mark.parametrize("n", [4096 * 1536, 4096 * 1536 + 8 * 1023 + 5, 8 * 1024 * 3 + 8])
def test_fp16_row_converters_large(hip, dev, oracle, n):
    """Rows spanning many workgroups, each thread converting four groups of
    eight a grid apart; sizes that leave the last pass ragged."""
    import torch
    f = oracle.gaussian(n, 2024 + n % 97) * 3.0
    h = torch.empty(n, dtype=torch.int16, device=dev)
    hip.fp32_to_fp16_row(to_dev(f, dev), h, n)
    hb = from_dev(h).view(np.uint16)
    assert np.array_equal(hb, oracle.f32_to_f16(f))
    out = torch.empty(n, dtype=torch.float32, device=dev)
    hip.fp16_to_fp32_row(h, out, n)
    assert np.array_equal(from_dev(out).view(np.uint32), oracle.f16_to_f32(hb).view(np.uint32))


@pytest.mark.parametrize("n,offset", [(64 * 2520, 0), (4099, 0), (1001, 1)])
def test_checked_euler_matches_unchecked_and_stays_clear(hip, dev, oracle, n, offset):
    """The checked entry point updates bit-identically and leaves the flag 0."""
    import torch
    x0 = oracle.gaussian(n + offset, 31)
    vu = oracle.gaussian(n + offset, 32)
    vc = oracle.gaussian(n + offset, 33)
    a, b = to_dev(x0, dev), to_dev(x0, dev)
    du, dc = to_dev(vu, dev), to_dev(vc, dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.flow_cfg_euler(a[offset:], du[offset:], dc[offset:], n, 1.5, 0.02)
    hip.flow_cfg_euler_checked(b[offset:], du[offset:], dc[offset:], n, 1.5, 0.02, flags)
    assert _eq(from_dev(a), from_dev(b))
    assert int(flags.item()) == 0


VEL, STATE = 1, 2


@pytest.mark.parametrize("where", ["vector", "tail"])
def test_checked_euler_flags_nonfinite_velocity_and_state(hip, dev, where):
    """src/levo-flow-renderer.cpp:104, :106: a NaN/inf velocity or an
    overflowing state is reported through the flag word."""
    import torch
    n = 4099
    pos = 1234 if where == "vector" else n - 1
    state = torch.zeros(n, dtype=torch.float32, device=dev)
    vu = torch.ones(n, dtype=torch.float32, device=dev)
    vc = torch.ones(n, dtype=torch.float32, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.flow_cfg_euler_checked(state, vu, vc, n, 1.5, 0.02, flags)
    assert int(flags.item()) == 0
    vc[pos] = float("nan")
    hip.flow_cfg_euler_checked(state, vu, vc, n, 1.5, 0.02, flags)
    assert int(flags.item()) & VEL
    vc[pos] = 1.0
    flags.zero_()
    state[pos] = 3.0e38
    vu[pos] = 3.0e38
    vc[pos] = 3.0e38
    hip.flow_cfg_euler_checked(state, vu, vc, n, 1.5, 1.0, flags)  # finite v, state overflows
    assert int(flags.item()) == STATE
    flags.zero_()
    hip.flow_cfg_euler_checked(state, vu, None, n, 1.5, 0.02, flags)  # inf state stays inf
    assert int(flags.item()) == STATE


@pytest.mark.parametrize("n,offset", [(1, 0), (5, 0), (4096, 0), (161_283, 0), (1003, 1), (10_000_000, 0)])
def test_check_finite(hip, dev, n, offset):
    import torch
    x = torch.randn(n + offset, dtype=torch.float32, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    hip.check_finite(x[offset:], n, flags, 4)
    assert int(flags.item()) == 0
    for pos, bad in [(0, float("nan")), (n // 2, float("inf")), (n - 1, float("-inf"))]:
        flags.zero_()
        keep = float(x[offset + pos].item())
        x[offset + pos] = bad
        hip.check_finite(x[offset:], n, flags, 4)
        assert int(flags.item()) == 4, (pos, bad)
        x[offset + pos] = keep
