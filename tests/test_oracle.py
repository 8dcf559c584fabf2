"""Pins the CPU oracle (the checker) before it is trusted.

Each oracle function is checked against the reference's own known-answer
tests (cited file:line), the reference's own sources compiled from the
checkout (oracle/_ref), and what the mathematics fixes (closed forms,
invariants, independent numpy restatements) — chosen so that a plausible
mistake (dropped term, wrong sign or index, FMA where the reference rounds
twice) fails at least one of them. CPU only.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import f16_ulp, f32_err

LN = math.log


# ---------------------------------------------------------------- F16 conversion

def test_fp16_matches_numpy_rne(oracle):
    bits = np.arange(0, 2**32, 997, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    with np.errstate(over="ignore"):
        expect = f.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(f), expect)


def test_fp16_edge_cases(oracle):
    # subnormal boundaries, ties to even, overflow threshold, signed zero
    cases = np.array([0.0, -0.0, 2.0**-24, 2.0**-25, 1.5 * 2.0**-25, 2.0**-25 * 1.0000001, 65504.0,
                      65519.99, 65520.0, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 6.1035156e-05,
                      2.0**-14 - 2.0**-25, np.inf, -np.inf, 1e-40], dtype=np.float32)
    with np.errstate(over="ignore"):
        expect = cases.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(cases), expect)


def test_fp16_widening_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].view(np.uint32), want[ok].view(np.uint32))
    assert np.all(np.isnan(got[~ok]))


# ---------------------------------------------------------------- SnakeBeta

SNAKE_X = np.array([[-1.0, 0.0, 1.0], [-0.5, 0.5, 1.5]], dtype=np.float32)
SNAKE_A = np.array([LN(2.0), LN(0.5)], dtype=np.float32)
SNAKE_B = np.array([LN(1.5), LN(0.75)], dtype=np.float32)


def snake_expected_kat():
    """tests/test-audio-ops.cpp:203-213: value + sin(value*alpha)^2 / (exp(b)+1e-9) in float."""
    out = np.empty_like(SNAKE_X)
    for c in range(2):
        alpha = np.float32(math.exp(np.float32(SNAKE_A[c])))
        beta = np.float32(np.float32(math.exp(np.float32(SNAKE_B[c]))) + np.float32(1e-9))
        for t in range(3):
            v = SNAKE_X[c, t]
            s = np.float32(math.sin(np.float32(v * alpha)))
            out[c, t] = np.float32(v + np.float32(s * s) / beta)
    return out


def test_snake_reference_kat(oracle):
    y = oracle.snake_beta(SNAKE_X, SNAKE_A, SNAKE_B)
    # reference CPU tolerance (tests/test-audio-ops.cpp:214-215)
    assert np.max(np.abs(y - snake_expected_kat())) <= 1e-6


def test_snake_f16_params_kat(oracle):
    # F16 parameters promoted to F32 (src/levo-audio-ops.cpp:143-144), gate 2e-3 (:220-221)
    a = oracle.f16_to_f32(oracle.f32_to_f16(SNAKE_A))
    b = oracle.f16_to_f32(oracle.f32_to_f16(SNAKE_B))
    y = oracle.snake_beta(SNAKE_X, a, b)
    assert np.max(np.abs(y - snake_expected_kat())) <= 2e-3


def snake_f64(x, a, b):
    x = x.astype(np.float64)
    alpha = np.exp(a.astype(np.float64))[:, None]
    beta = (np.exp(b.astype(np.float64)) + 1e-9)[:, None]
    return x + np.sin(x * alpha) ** 2 / beta


def test_snake_against_float64_closed_form(oracle):
    C, T = 64, 3000
    x = oracle.gaussian(C * T, 11).reshape(C, T)
    rng = np.random.default_rng(3)
    a = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, C).astype(np.float32)
    y = oracle.snake_beta(x, a, b, threads=4)
    assert f32_err(y, snake_f64(x, a, b)) <= 1e-6
    # a dropped 1/beta or a missing square is far outside this
    assert f32_err(x + np.sin(x * np.exp(a)[:, None]) ** 2, snake_f64(x, a, b)) > 1e-3


def test_snake_special_cases(oracle):
    x = np.zeros((3, 8), dtype=np.float32)
    a = np.array([0.3, -0.2, 0.0], dtype=np.float32)
    b = np.array([0.1, 0.0, -0.4], dtype=np.float32)
    assert np.array_equal(oracle.snake_beta(x, a, b), x)  # sin(0) = 0 -> y = x exactly
    # sign symmetry of sin^2: y(-x) + x = y(x) - x
    x = oracle.gaussian(3 * 64, 5).reshape(3, 64)
    yp = oracle.snake_beta(x, a, b)
    ym = oracle.snake_beta(-x, a, b)
    assert np.max(np.abs((yp - x) - (ym + x))) <= 1e-6


def test_snake_threads_do_not_change_results(oracle):
    x = oracle.gaussian(37 * 101, 9).reshape(37, 101)
    a = np.linspace(-0.5, 0.5, 37, dtype=np.float32)
    b = np.linspace(0.5, -0.5, 37, dtype=np.float32)
    assert np.array_equal(oracle.snake_beta(x, a, b, threads=1), oracle.snake_beta(x, a, b, threads=5))


# ---------------------------------------------------------------- norms

def _f16(oracle, x):
    return oracle.f32_to_f16(np.asarray(x, dtype=np.float32))


def test_layer_norm_constant_row_gives_beta_exactly(oracle):
    D = 2048
    x = np.full((3, D), 0.7, dtype=np.float32)
    g = oracle.gaussian(D, 1) * 0.02 + 1
    bta = oracle.gaussian(D, 2) * 0.02
    _, y = oracle.layer_norm(x, None, g.astype(np.float32), bta.astype(np.float32), 1e-6)
    assert np.array_equal(y, np.broadcast_to(bta, y.shape))


def test_layer_norm_alternating_row(oracle):
    D = 1536
    x = np.tile(np.array([1.0, -1.0], dtype=np.float32), (2, D // 2))
    g = (oracle.gaussian(D, 4) * 0.02 + 1).astype(np.float32)
    bta = (oracle.gaussian(D, 5) * 0.02).astype(np.float32)
    eps = 1e-6
    _, y = oracle.layer_norm(x, None, g, bta, eps)
    want = x.astype(np.float64) / math.sqrt(1 + eps) * g + bta
    assert f32_err(y, want) <= 2e-7


def test_rms_norm_constant_row(oracle):
    D, c, eps = 2048, 0.25, 1e-6
    x = np.full((2, D), c, dtype=np.float32)
    w = (oracle.gaussian(D, 6) * 0.02 + 1).astype(np.float32)
    _, y = oracle.rms_norm(x, None, w, eps)
    want = w.astype(np.float64) * c / math.sqrt(c * c + eps)
    assert f32_err(y, np.broadcast_to(want, y.shape)) <= 2e-7


def norm_f64(h, w, b, eps, layer):
    h = h.astype(np.float64)
    if layer:
        v = h - h.mean(axis=1, keepdims=True)
        return v / np.sqrt((v * v).mean(axis=1, keepdims=True) + eps) * w + b
    return h / np.sqrt((h * h).mean(axis=1, keepdims=True) + eps) * w


@pytest.mark.parametrize("layer", [False, True])
def test_norm_f32_against_float64(oracle, layer):
    rows, D, eps = 37, 2200, 1e-5
    x = oracle.gaussian(rows * D, 7).reshape(rows, D)
    d = oracle.gaussian(rows * D, 8).reshape(rows, D)
    w = (oracle.gaussian(D, 9) * 0.02 + 1).astype(np.float32)
    b = (oracle.gaussian(D, 10) * 0.02).astype(np.float32)
    if layer:
        h, y = oracle.layer_norm(x, d, w, b, eps, threads=3)
    else:
        h, y = oracle.rms_norm(x, d, w, eps, threads=3)
    assert np.array_equal(h, x + d)
    assert f32_err(y, norm_f64(x + d, w, b, eps, layer)) <= 1e-5
    # the residual must enter the statistics: normalising x alone is far off
    assert f32_err(norm_f64(x, w, b, eps, layer), norm_f64(x + d, w, b, eps, layer)) > 1e-2


@pytest.mark.parametrize("layer", [False, True])
def test_norm_f16_rounding_points(oracle, layer):
    """numpy float16 pipeline with the same rounding points (src/levo-kv.cpp:153-160)."""
    rows, D, eps = 16, 2048, 1e-6
    xh = _f16(oracle, oracle.gaussian(rows * D, 12).reshape(rows, D))
    dh = _f16(oracle, oracle.gaussian(rows * D, 13).reshape(rows, D))
    wh = _f16(oracle, oracle.gaussian(D, 14) * 0.02 + 1)
    bh = _f16(oracle, oracle.gaussian(D, 15) * 0.02)
    if layer:
        h, y = oracle.layer_norm(xh, dh, wh, bh, eps)
    else:
        h, y = oracle.rms_norm(xh, dh, wh, eps)
    x16, d16 = xh.view(np.float16), dh.view(np.float16)
    w32, b32 = wh.view(np.float16).astype(np.float32), bh.view(np.float16).astype(np.float32)
    h16 = (x16.astype(np.float32) + d16.astype(np.float32)).astype(np.float16)
    assert np.array_equal(h, h16.view(np.uint16))
    hf = h16.astype(np.float32)
    if layer:
        mean = (hf.astype(np.float64).sum(axis=1) / D).astype(np.float32)[:, None]
        v = hf - mean
        var = ((v * v).astype(np.float64).sum(axis=1) / D).astype(np.float32)[:, None]
        scale = np.float32(1) / np.sqrt(var + np.float32(eps))
        y16 = ((v * scale) * w32 + b32).astype(np.float16)
    else:
        ms = ((hf * hf).astype(np.float64).sum(axis=1) / D).astype(np.float32)[:, None]
        scale = np.float32(1) / np.sqrt(ms + np.float32(eps))
        n16 = (hf * scale).astype(np.float16)
        y16 = (n16.astype(np.float32) * w32).astype(np.float16)
    assert f16_ulp(y, y16.view(np.uint16)) <= 1


# ---------------------------------------------------------------- CFG

def test_cfg_reference_kats(oracle, ref):
    # tests/test-sampling.cpp:8 and tests/test-renderer-pattern.cpp:88-90
    assert oracle.apply_cfg([2, 4], [1, 1], 1.5).tolist() == [2.5, 5.5]
    assert oracle.apply_cfg([3, 6], [1, 2], 1.5).tolist() == [4.0, 8.0]
    assert ref.apply_cfg([2, 4], [1, 1], 1.5).tolist() == [2.5, 5.5]
    assert ref.combine_renderer_cfg([1, 2], [3, 6], 1.5).tolist() == [4.0, 8.0]


def test_cfg_bit_exact_vs_reference_and_not_fused(oracle, ref):
    c = (oracle.gaussian(1 << 16, 21) * 3).astype(np.float32)
    u = (oracle.gaussian(1 << 16, 22) * 3).astype(np.float32)
    got = oracle.apply_cfg(c, u, 1.5)
    assert np.array_equal(got.view(np.uint32), ref.apply_cfg(c, u, 1.5).view(np.uint32))
    assert np.array_equal(got.view(np.uint32), ref.combine_renderer_cfg(u, c, 1.5).view(np.uint32))
    # the reference rounds s*(c-u) before the add: a fused a*b+c differs somewhere
    fused = (u.astype(np.float64) + np.float64(1.5) * (c - u).astype(np.float64)).astype(np.float32)
    assert np.count_nonzero(fused.view(np.uint32) != got.view(np.uint32)) > 0


# ---------------------------------------------------------------- RNG / sampling

def test_mt19937_64_standard_value(oracle, ref):
    rng = oracle.mt(5489)
    for _ in range(9999):
        oracle.mt_next(rng)
    assert oracle.mt_next(rng) == 9981545732273789042  # C++ [rand.predef]
    for seed in (0, 1, 1234, 2**63 + 5):
        r = oracle.mt(seed)
        vals = [oracle.mt_next(r) for _ in range(700)]
        assert vals[699] == ref.mt_after(seed, 699)
        assert vals[0] == ref.mt_after(seed, 0)


def test_repetition_penalty_kat(oracle, ref):
    # tests/test-sampling.cpp:9-11: unique ids, not frequencies
    assert oracle.repetition_penalty([10, 8, 6], [0, 0, 1], 2.0).tolist() == [5, 4, 6]
    x = oracle.gaussian(300, 31)
    rec = np.array([5, 5, 299, 298, -1, 17, 400, 17], dtype=np.int64)
    for limit in (0, 299, 10):
        assert np.array_equal(oracle.repetition_penalty(x, rec, 1.1, limit), ref.repetition_penalty(x, rec, 1.1, limit))


def test_sampler_reference_kats(oracle):
    # tests/test-sampling.cpp:12-15: penalised token 2, EOS (last logit) excluded
    toks, d = oracle.sample_streams(np.array([[9, 8, 10, 7]], np.float32), use_sampling=False, temperature=0.9,
                                    top_k_mixed=50, top_k_detail=1, repetition_penalty=2.0,
                                    recent=np.array([[2, 3]]), rng=oracle.mt(0))
    assert toks.tolist() == [0] and d == 0
    # :33-37 greedy picks and no draws
    g = oracle.mt(12)
    assert oracle.sample_top_k([0, 1, 2], 3, 1.0, False, g)[0] == 2
    assert oracle.sample_top_k([0, 1, 2], 3, 0.0, True, g)[0] == 2
    toks, d = oracle.sample_streams(np.array([[0, 2, 1], [1, 4, 0]], np.float32), use_sampling=False,
                                    temperature=0.9, top_k_mixed=50, top_k_detail=1, rng=g)
    assert toks.tolist() == [1, 1] and d == 0
    # :38 top-1 of {-1,3,-2}
    assert oracle.sample_top_k([-1, 3, -2], 1, 1.0, True, oracle.mt(1))[0] == 1
    # :41-48 k=1 keeps both tied maxima
    r = oracle.mt(7)
    seen = {oracle.sample_top_k([5, 5, 0], 1, 1.0, True, r)[0] for _ in range(64)}
    assert seen == {0, 1}


def test_sampler_cursor_matches_reference(oracle, ref):
    # tests/test-sampling.cpp:18-32
    s = ref.sampler(1234)
    full = [s.sample([0, 1, 2, 3], 4, 0.8, True) for _ in range(20)]
    r, d = oracle.mt(1234), 0
    mine = []
    for _ in range(20):
        t, d = oracle.sample_top_k([0, 1, 2, 3], 4, 0.8, True, r, d)
        mine.append(t)
    assert mine == full and d == 20 == s.draw_count


def _tie_heavy_logits(oracle, n, vocab, seed):
    x = oracle.gaussian(n * vocab, seed).reshape(n, vocab) * 3
    return oracle.f16_to_f32(oracle.f32_to_f16(x))  # F16-rounded like src/levo-kv.cpp:735-738


@pytest.mark.parametrize("top_k", [1, 2, 50, 100, 0])
def test_top_k_candidates_brute_force(oracle, top_k):
    lg = _tie_heavy_logits(oracle, 40, 2048, 41 + top_k)
    lg[3, :] = 1.0                      # everything tied
    lg[4, 100:160] = lg[4].max() + 1    # 60 tied maxima
    lg[5, :] = -np.inf
    lg[6, 7] = -0.0
    lg[6, 9] = 0.0
    for row in lg:
        best, cand = oracle.top_k_candidates(row, top_k)
        order = np.argsort(-row.astype(np.float64), kind="stable")
        if 0 < top_k < row.size:
            thr = row[order[top_k - 1]]
            want = np.nonzero(row >= thr)[0]
        else:
            want = np.arange(row.size)
        assert np.array_equal(cand, want)
        assert best == int(np.argmax(row))  # numpy argmax also keeps the first maximum


def test_sampler_tokens_match_reference(oracle, ref):
    V = 4096
    for seed in range(6):
        lg = _tie_heavy_logits(oracle, 3 * 30, V, 100 + seed).reshape(30, 3, V)
        s = ref.sampler(seed)
        r, d = oracle.mt(seed), 0
        recent = np.full((3, 50), -1, dtype=np.int64)
        for pos in range(30):
            cfg = dict(use_sampling=seed != 5, temperature=0.9 if seed != 4 else 0.3, top_k_mixed=50,
                       top_k_detail=1 if seed % 2 == 0 else 7)
            want = s.sample_streams(lg[pos], repetition_penalty=1.1, recent=recent, ignore=(3, 9, V - 1), **cfg)
            got, d = oracle.sample_streams(lg[pos], repetition_penalty=1.1, recent=recent, ignore=(3, 9, V - 1),
                                           rng=r, draws=d, **cfg)
            assert got.tolist() == want.tolist()
            recent = np.concatenate([recent[:, 1:], got[:, None]], axis=1)
        assert d == s.draw_count


def test_sampler_rejects_nan(oracle, ref):
    with pytest.raises(ValueError):
        oracle.sample_top_k([0.0, float("nan"), 1.0], 2, 1.0, True, oracle.mt(0))
    s = ref.sampler(0)
    with pytest.raises(ValueError, match="NaN"):
        s.sample([0.0, float("nan"), 1.0], 2, 1.0, True)


# ---------------------------------------------------------------- Flow Euler

def _solve(oracle, noise, ctx, frames, dim, incontext, sigma_min, steps, velocity):
    state = noise.copy()
    dt = np.float32(1.0) / np.float32(steps)
    seen = []
    for step in range(steps):
        t = np.float32(step) * dt
        oracle.flow_incontext(state, noise, ctx, incontext * dim, float(t), sigma_min)
        seen.append(state.copy())
        v_u, v_c, g = velocity(state, t)
        oracle.flow_cfg_euler(state, v_u, v_c, g, float(dt))
    state[: incontext * dim] = ctx[: incontext * dim]
    return state, seen


def test_flow_euler_reference_kat(oracle):
    # tests/test-flow-renderer.cpp:33-65
    noise = np.array([1, 2, 10, 20, 30, 40], np.float32)
    ctx = np.array([4, 8, 0, 0, 0, 0], np.float32)
    ones = np.ones(6, np.float32)
    out, seen = _solve(oracle, noise, ctx, 3, 2, 1, 0.1, 2, lambda s, t: (ones, None, 1.0))
    assert np.allclose(seen[0][:2], [1.0, 2.0], atol=1e-6)
    assert np.allclose(seen[1][:2], [2.55, 5.10], atol=1e-6)
    assert np.allclose(out, [4, 8, 11, 21, 31, 41], atol=1e-6)


def test_flow_euler_schedule_matches_reference(ref):
    times, dt = ref.euler_schedule(50)
    t = np.arange(51, dtype=np.float32) * np.float32(1.0 / np.float32(50))
    assert dt == np.float32(1.0) / np.float32(50)
    assert np.array_equal(times[:50], (np.arange(50, dtype=np.float32) * np.float32(dt)).astype(np.float32))
    assert times[-1] == 1.0 and t[0] == 0.0


def test_flow_cfg_euler_closed_form(oracle):
    n, steps = 64 * 2520, 50
    x0 = oracle.gaussian(n, 51)
    state = x0.copy()
    g, dt = np.float32(1.5), np.float32(1.0) / np.float32(steps)
    want = x0.copy()
    for s in range(steps):
        vu = oracle.gaussian(n, 1000 + 2 * s)
        vc = oracle.gaussian(n, 1001 + 2 * s)
        oracle.flow_cfg_euler(state, vu, vc, float(g), float(dt))
        v = vu + g * (vc - vu)            # numpy float32: two roundings each
        want = want + dt * v
    assert np.array_equal(state.view(np.uint32), want.view(np.uint32))
    # constant velocity: x0 + steps * dt * v, within the 50 half-ulp roundings of the sum
    state = x0.copy()
    one = np.full(n, 0.5, np.float32)
    for _ in range(steps):
        oracle.flow_cfg_euler(state, one, None, 1.5, float(dt))
    assert f32_err(state, x0.astype(np.float64) + 0.5) <= steps * 2.0**-23


# ---------------------------------------------------------------- Q8_0 / Q4_0

def q8_numpy(x):
    """ggml quantize_row_q8_0_ref restated in numpy (independent of the C)."""
    b = x.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    v = (b * idv[:, None]).astype(np.float32)
    q = np.where(np.abs(v - np.trunc(v)) >= 0.5, np.trunc(v) + np.sign(v), np.trunc(v)).astype(np.int8)
    out = np.empty((b.shape[0], 34), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def q4_numpy(x):
    """ggml quantize_row_q4_0_ref restated in numpy."""
    b = x.reshape(-1, 32).astype(np.float32)
    first = np.argmax(np.abs(b) == np.max(np.abs(b), axis=1, keepdims=True), axis=1)
    vmax = b[np.arange(b.shape[0]), first]
    vmax = np.where(np.max(np.abs(b), axis=1) == 0, np.float32(0), vmax).astype(np.float32)
    d = (vmax / np.float32(-8)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    q = np.trunc((b * idv[:, None]).astype(np.float32) + np.float32(8.5)).astype(np.int32)
    q = np.minimum(q, 15).astype(np.uint8)
    out = np.empty((b.shape[0], 18), np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.ravel()


def test_q8_0_reference_kat(oracle):
    # tests/test-quantization.cpp:46-75: padded 4x32 matrix, Q8_0 product within 0.015
    m = np.zeros((4, 32), np.float32)
    for r in range(4):
        for c in range(6):
            m[r, c] = 0.03125 * (r + 1) * (c + 1)
    q = oracle.quantize(8, m)
    deq = oracle.dequantize(8, q, 128).reshape(4, 32)
    inp = np.zeros(32, np.float32)
    inp[:6] = [0.25, -0.5, 0.75, -1.0, 1.25, -1.5]
    assert np.all(np.abs(deq @ inp - m @ inp) < 0.015)


def test_q8_0_invariants_and_numpy_restatement(oracle):
    x = (oracle.gaussian(4096 * 64, 61) * 0.02).reshape(4096, 64)
    x[0, :32] = 0.0
    x[1, :32] = np.arange(32) - 16.0          # amax 16 -> d = 16/127
    x[2, :32] = 0.0
    x[2, 0], x[2, 1], x[2, 2] = 127.0, 2.5, -2.5   # d = 1, id = 1: ties round away from zero
    x[3, :32] = 1e-6 * np.arange(32)          # F16-subnormal scale
    q = oracle.quantize(8, x)
    assert np.array_equal(q, q8_numpy(x))
    blocks = q.reshape(-1, 34)
    qs = blocks[:, 2:].view(np.int8).astype(np.int32)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    xb = x.reshape(-1, 32)
    assert np.all(np.abs(qs) <= 127)
    amax_pos = np.argmax(np.abs(xb), axis=1)
    nz = np.max(np.abs(xb), axis=1) > 0
    assert np.all(np.abs(qs[np.arange(len(qs)), amax_pos][nz]) == 127)
    assert np.all(blocks[0] == 0)
    assert qs[4, 1] == 3 and qs[4, 2] == -3   # block 4 = first block of row 2
    deq = oracle.dequantize(8, q, x.size).reshape(-1, 32)
    dd = (np.max(np.abs(xb), axis=1) / np.float32(127)).astype(np.float32)
    assert np.all(np.abs(deq - xb) <= dd[:, None] * 0.5001 + np.abs(d - dd)[:, None] * 127.0 + 1e-12)
    assert np.array_equal(deq, (qs * d[:, None]).astype(np.float32))


def test_q4_0_invariants_and_numpy_restatement(oracle):
    x = (oracle.gaussian(2048 * 64, 71) * 0.02).reshape(2048, 64)
    x[0, :32] = 0.0
    x[1, :32] = 0.0
    x[1, 1], x[1, 3] = -0.5, 0.5               # equal |x|: the first (negative) one wins
    q = oracle.quantize(2, x)
    assert np.array_equal(q, q4_numpy(x))
    blocks = q.reshape(-1, 18)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    assert d[2] == np.float32(0.5 / 8)          # d = max/-8 with max = -0.5
    nib = np.concatenate([blocks[:, 2:] & 15, blocks[:, 2:] >> 4], axis=1).astype(np.int32)
    assert nib.max() <= 15
    xb = x.reshape(-1, 32)
    first = np.argmax(np.abs(xb) == np.max(np.abs(xb), axis=1, keepdims=True), axis=1)
    nz = np.max(np.abs(xb), axis=1) > 0
    assert np.all(nib[np.arange(len(nib)), first][nz] == 0)   # the signed max maps to q = 0
    deq = oracle.dequantize(2, q, x.size).reshape(-1, 32)
    assert np.array_equal(deq, ((nib - 8) * d[:, None]).astype(np.float32))


def test_quantize_padding_matches_chunk_of_padded_rows(oracle):
    rows, src_cols, dst_cols = 5, 2200, 2208   # Flow hidden 2200 -> 2208 (src/levo-quantization.h:120-130)
    xh = oracle.f32_to_f16(oracle.gaussian(rows * src_cols, 81).reshape(rows, src_cols) * 0.02)
    for qt in (8, 2):
        padded = np.zeros((rows, dst_cols), np.float32)
        padded[:, :src_cols] = oracle.f16_to_f32(xh)
        assert np.array_equal(oracle.quantize_f16_padded(qt, xh, dst_cols), oracle.quantize(qt, padded))


# ---------------------------------------------------------------- Q8_0 mat-vec

def _q8_parts(blocks, nblocks):
    """(d as float32, quants as int32 [nblocks][32]) of packed Q8_0 blocks."""
    b = np.ascontiguousarray(blocks, np.uint8).reshape(nblocks, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32).reshape(nblocks)
    q = b[:, 2:].view(np.int8).astype(np.int32)
    return d, q


@pytest.mark.parametrize("rows,k,n_vec", [(64, 1536, 2), (7, 8960, 1), (33, 32, 3)])
def test_mul_mat_q8_0_matches_block_terms(oracle, rows, k, n_vec):
    """ggml_vec_dot_q8_0_q8_0 semantics: y = sum_b sumi_b * (d_w * d_x) with
    the activation quantized by the reference quantizer. Checked against the
    float64 sum of independently built block terms, within the error bound of
    a sequential F32 sum ((nb - 1) * 2^-24 * sum |term|). A dropped or
    transposed term, a wrong scale or an unquantized activation fails it."""
    nb = k // 32
    w = (oracle.gaussian(rows * k, 1000 + k) * np.float32(0.02)).reshape(rows, k)
    x = oracle.gaussian(n_vec * k, 2000 + k).reshape(n_vec, k)
    wb = oracle.quantize(8, w)
    y = oracle.mul_mat_q8_0(wb, x, rows, k)
    dw, qw = _q8_parts(wb, rows * nb)
    for v in range(n_vec):
        dx, qx = _q8_parts(oracle.quantize(8, x[v].reshape(1, k)), nb)
        sumi = (qw.reshape(rows, nb, 32) * qx.reshape(1, nb, 32)).sum(axis=2)
        terms = sumi.astype(np.float32) * (dw.reshape(rows, nb) * dx.reshape(1, nb)).astype(np.float32)
        exact = terms.astype(np.float64).sum(axis=1)
        bound = (nb - 1) * 2.0 ** -24 * np.abs(terms).astype(np.float64).sum(axis=1) + 1e-30
        assert np.all(np.abs(y[v].astype(np.float64) - exact) <= bound)
        # and close to the unquantized product (quantization error only)
        assert np.max(np.abs(y[v] - w @ x[v])) < 0.05 * np.sqrt(k) * 0.02


def test_mul_mat_q8_0_integer_blocks_exact(oracle):
    """Blocks whose largest |value| is 127 quantize with d = 1 and q = value:
    the product is the exact integer product (every partial sum < 2^24)."""
    rng = np.random.default_rng(5)
    rows, k, n_vec = 40, 640, 2
    w = rng.integers(-127, 128, (rows, k)).astype(np.float32)
    x = rng.integers(-127, 128, (n_vec, k)).astype(np.float32)
    w[:, ::32] = 127.0
    x[:, 5::32] = -127.0
    y = oracle.mul_mat_q8_0(oracle.quantize(8, w), x, rows, k)
    want = (w.astype(np.int64) @ x.astype(np.int64).T).T
    assert np.array_equal(y, want.astype(np.float32))


# ---------------------------------------------------------------- Conv1d

def _conv64(x, w, bias, pad, dil):
    c_in, t_in = x.shape
    c_out, _, kw = w.shape
    t_out = t_in + 2 * pad - dil * (kw - 1)
    xp = np.zeros((c_in, t_in + 2 * pad + dil * kw), np.float64)
    xp[:, pad:pad + t_in] = x
    y = np.zeros((c_out, t_out), np.float64)
    absum = np.zeros((c_out, t_out), np.float64)
    for k in range(kw):
        win = xp[:, k * dil:k * dil + t_out]
        y += w[:, :, k].astype(np.float64) @ win
        absum += np.abs(w[:, :, k]).astype(np.float64) @ np.abs(win)
    return y, absum


@pytest.mark.parametrize("c_in,c_out,t_in,kw,pad,dil", [(16, 24, 300, 7, 3, 1), (8, 8, 200, 7, 27, 9),
                                                       (32, 16, 100, 1, 0, 1), (5, 3, 40, 3, 2, 2)])
def test_conv1d_matches_float64(oracle, c_in, c_out, t_in, kw, pad, dil):
    """conv_1d_f32's im2col + dot + bias against a float64 direct convolution:
    within the error bound of a sequential F32 sum plus the bias rounding.
    A wrong tap offset, padding side or dilation fails it."""
    x = oracle.gaussian(c_in * t_in, 70 + kw).reshape(c_in, t_in)
    w = (oracle.gaussian(c_out * c_in * kw, 71 + kw) * np.float32(0.3)).reshape(c_out, c_in, kw)
    b = oracle.gaussian(c_out, 72)
    y = oracle.conv1d(x, w, b, pad, dil, threads=2)
    exact, absum = _conv64(x, w, None, pad, dil)
    exact += b[:, None]
    bound = c_in * kw * 2.0 ** -24 * absum + 2.0 ** -24 * np.abs(exact) + 1e-30
    assert y.shape == exact.shape
    assert np.all(np.abs(y - exact) <= bound)


def test_conv1d_identity_shift_and_dilation_kernels(oracle):
    """Delta kernels move samples exactly: the centre tap is the identity,
    tap 0 with padding 1 delays by one, tap 2 at dilation 2 with padding 2
    advances by two; zeros come in from the padding."""
    c, t = 6, 50
    x = oracle.gaussian(c * t, 80).reshape(c, t)
    eye = np.eye(c, dtype=np.float32)
    for tap, pad, dil, shift in ((1, 1, 1, 0), (0, 1, 1, -1), (2, 2, 2, 2)):
        w = np.zeros((c, c, 3), np.float32)
        w[:, :, tap] = eye
        y = oracle.conv1d(x, w, None, pad, dil)
        want = np.zeros_like(y)
        for i in range(y.shape[1]):
            if 0 <= i + shift < t:
                want[:, i] = x[:, i + shift]
        assert np.array_equal(y, want), (tap, pad, dil)
    b = oracle.gaussian(c, 81)
    w = np.zeros((c, c, 3), np.float32)
    w[:, :, 1] = eye
    assert np.array_equal(oracle.conv1d(x, w, b, 1, 1), (x + b[:, None]).astype(np.float32))


@pytest.mark.parametrize("c_in,c_out,t_in,stride", [(16, 8, 30, 10), (8, 16, 50, 6), (12, 12, 40, 4),
                                                    (6, 5, 90, 2), (3, 2, 7, 3)])
def test_conv_transpose1d_matches_float64(oracle, c_in, c_out, t_in, stride):
    """ggml_conv_transpose_1d (kernel 2 * stride) + crop (stride + 1) / 2 +
    bias against a float64 scatter-form transposed convolution, within the
    error bound of the per-tap F32 dots and the two F32 additions."""
    k = 2 * stride
    pad = (stride + 1) // 2
    x = oracle.gaussian(c_in * t_in, 300 + stride).reshape(c_in, t_in)
    w = (oracle.gaussian(c_in * c_out * k, 301 + stride) * np.float32(0.3)).reshape(c_in, c_out, k)
    b = oracle.gaussian(c_out, 302)
    y = oracle.conv_transpose1d(x, w, b, stride, pad)
    t_full = (t_in - 1) * stride + k
    full = np.zeros((c_out, t_full))
    absf = np.zeros((c_out, t_full))
    for i in range(t_in):
        for kk in range(k):
            full[:, i * stride + kk] += w[:, :, kk].astype(np.float64).T @ x[:, i].astype(np.float64)
            absf[:, i * stride + kk] += np.abs(w[:, :, kk]).astype(np.float64).T @ np.abs(x[:, i]).astype(np.float64)
    exact = full[:, pad:t_full - pad] + b[:, None]
    bound = (c_in + 2) * 2.0 ** -24 * absf[:, pad:t_full - pad] + 2.0 ** -24 * np.abs(exact) + 1e-30
    assert y.shape == exact.shape
    assert np.all(np.abs(y - exact) <= bound)


def test_conv_transpose1d_delta_kernel_upsamples(oracle):
    """A delta at tap k of a stride-s kernel places x[ci][i] at output
    i * s + k - padding: zero-insertion upsampling, exactly."""
    c, t, s = 4, 20, 4
    x = oracle.gaussian(c * t, 310).reshape(c, t)
    for tap in (0, 3, 5, 7):
        w = np.zeros((c, c, 2 * s), np.float32)
        w[:, :, tap] = np.eye(c, dtype=np.float32)
        pad = (s + 1) // 2
        y = oracle.conv_transpose1d(x, w, None, s, pad)
        want = np.zeros_like(y)
        for i in range(t):
            o = i * s + tap - pad
            if 0 <= o < y.shape[1]:
                want[:, o] = x[:, i]
        assert np.array_equal(y, want), tap


def test_f16_residual_single_rounding_equals_f32_chain():
    """The F16 residual kernels add packed halves (one rounding of the exact
    sum) where the reference rounds f32(x) + f32(d) to F32 and then to F16
    (src/levo-kv.cpp:462, 507). Equal by Figueroa's double-rounding bound (24
    >= 2 * 11 + 2); checked here for every finite F16 x against 96 d each:
    64 random halves and 32 placed at, just inside and just outside the
    rounding midpoints of x (including binade edges and subnormals). The
    correctly rounded sum is the exact float64 sum rounded to F16."""
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x16 = bits.view(np.float16)
    x16 = x16[np.isfinite(x16)]
    rng = np.random.default_rng(5)
    rand = rng.integers(0, 1 << 16, size=(x16.size, 64), dtype=np.uint32).astype(np.uint16).view(np.float16)
    with np.errstate(over="ignore"):  # spacing of the largest finite half is inf in F16
        ulp = np.spacing(np.abs(x16)).astype(np.float64)
    half = np.concatenate([ulp[:, None] * f for f in (0.5, 0.25)], axis=1)
    near = []
    for h in (half[:, :1], half[:, 1:2]):
        for m in (1.0, 1.0 + 2.0 ** -9, 1.0 - 2.0 ** -9, 1.0 + 2.0 ** -3, 1.0 - 2.0 ** -3, 3.0, 2.0 ** -5, 2.0 ** -12):
            near.append(h * m)
            near.append(-h * m)
    with np.errstate(over="ignore", invalid="ignore"):
        placed = np.concatenate(near, axis=1).astype(np.float16)
    d16 = np.concatenate([rand, placed], axis=1)
    d16 = np.where(np.isfinite(d16), d16, np.float16(0))
    for lo in range(0, x16.size, 4096):
        xs, ds = x16[lo:lo + 4096, None], d16[lo:lo + 4096]
        with np.errstate(over="ignore", invalid="ignore"):
            chain = (xs.astype(np.float32) + ds.astype(np.float32)).astype(np.float16)
            direct = (xs.astype(np.float64) + ds.astype(np.float64)).astype(np.float16)
        same = (chain.view(np.uint16) == direct.view(np.uint16)) | (np.isnan(chain) & np.isnan(direct))
        assert same.all(), (lo, np.argwhere(~same)[:5])


# ---- gated residual + LayerNorm + AdaLN modulation (Flow estimator blocks) ----------

def _modulation(rng, batches, dim, stride, scale=0.3):
    """(dynamic [batches][stride], learned [dim]) as modulation_chunk reads them."""
    dyn = (rng.standard_normal((batches, stride)) * scale).astype(np.float32)
    learned = (rng.standard_normal(dim) * scale).astype(np.float32)
    return dyn, learned


def _chain_f64(x, d, gate, gamma, beta, scale, shift, rpb, eps):
    """The ggml chain of src/levo-flow-estimator.cpp:89-109, 221-261 evaluated
    in float64 throughout (a brute force: no F32 rounding anywhere)."""
    rows, dim = x.shape
    b = np.arange(rows) // rpb

    def vec(v):
        dyn, learned = v
        out = dyn[:, :dim].astype(np.float64)
        return out + (0.0 if learned is None else learned.astype(np.float64))

    x64 = x.astype(np.float64)
    cur = x64 if d is None else (x64 + d.astype(np.float64) * (vec(gate)[b] if gate else 1.0))
    mean = cur.mean(axis=1, keepdims=True)
    var = ((cur - mean) ** 2).mean(axis=1, keepdims=True)
    t = (cur - mean) / np.sqrt(var + eps) * gamma.astype(np.float64) + beta.astype(np.float64)
    if scale is not None:
        t = t * (vec(scale)[b] + 1.0) + vec(shift)[b]
    return cur, t


def test_modulated_norm_without_gate_or_modulation_is_the_layer_norm(oracle):
    """No gate and no modulation: bit-identical to lo_residual_layer_norm_f32
    (itself pinned above), with and without delta."""
    rng = np.random.default_rng(21)
    x = rng.standard_normal((12, 2200)).astype(np.float32)
    d = rng.standard_normal((12, 2200)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(2200)).astype(np.float32)
    b = (0.02 * rng.standard_normal(2200)).astype(np.float32)
    for delta in (d, None):
        h, y = oracle.layer_norm_modulated(x, delta, None, g, b, None, None, 6, 1e-5)
        h2, y2 = oracle.layer_norm(x, delta, g, b, 1e-5)
        assert np.array_equal(h, h2) and np.array_equal(y, y2)


def test_modulated_norm_identity_modulation(oracle):
    """gate = 1, scale = 0, shift = 0 (dynamic parts zero, learned parts 1 /
    0 / 0) change no value: d * 1 + x = x + d and t * (0 + 1) + 0 = t."""
    rng = np.random.default_rng(22)
    rows, dim = 8, 1024
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    b = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    zeros = np.zeros((2, dim), np.float32)
    gate = (zeros, np.ones(dim, np.float32))
    zero = (zeros, np.zeros(dim, np.float32))
    h, y = oracle.layer_norm_modulated(x, d, gate, g, b, zero, zero, 4, 1e-5)
    h2, y2 = oracle.layer_norm(x, d, g, b, 1e-5)
    assert np.array_equal(h, h2) and np.array_equal(y, y2)


@pytest.mark.parametrize("learned", [True, False])
def test_modulated_norm_against_float64_chain(oracle, learned):
    """Three batch entries of distinct gate / scale / shift (modulation rows
    6 * dim apart, as the time modulation's chunks are) against the chain in
    float64: within the F32 bar everywhere, and far outside it for the plausible
    slips (a row taking another entry's vectors, scale used without the + 1,
    gate on x instead of delta, the modulation before beta)."""
    rng = np.random.default_rng(23 + learned)
    rows, dim, rpb, eps = 3 * 5, 2200, 5, 1e-5
    x = rng.standard_normal((rows, dim)).astype(np.float32)
    d = rng.standard_normal((rows, dim)).astype(np.float32)
    gamma = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    beta = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    vecs = []
    for _ in range(3):
        dyn, lrn = _modulation(rng, 3, dim, 6 * dim)
        vecs.append((dyn, lrn if learned else None))
    gate, scale, shift = vecs
    h, y = oracle.layer_norm_modulated(x, d, gate, gamma, beta, scale, shift, rpb, eps)
    h64, y64 = _chain_f64(x, d, gate, gamma, beta, scale, shift, rpb, eps)
    assert f32_err(h, h64) <= 1e-6
    assert f32_err(y, y64) <= 1e-5
    # the slips a restatement could make all land far outside the bar
    wrong_batch = _chain_f64(x, d, gate, gamma, beta, scale, shift, rows, eps)[1]
    no_plus_one = _chain_f64(x, d, gate, gamma, beta, (scale[0] - 1.0, scale[1]), shift, rpb, eps)[1]
    gate_on_x = _chain_f64(d, x, gate, gamma, beta, scale, shift, rpb, eps)[1]
    for slip in (wrong_batch, no_plus_one, gate_on_x):
        assert f32_err(y, slip) > 1e-2


def test_modulated_norm_constant_rows(oracle):
    """A constant row normalizes to 0, so y = (beta * (scale + 1)) + shift,
    each F32 operation rounded once (closed form)."""
    rng = np.random.default_rng(24)
    rows, dim = 6, 512
    x = np.repeat(rng.standard_normal((rows, 1)), dim, axis=1).astype(np.float32)
    gamma = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    beta = (0.5 * rng.standard_normal(dim)).astype(np.float32)
    scale = _modulation(rng, 2, dim, dim)
    shift = _modulation(rng, 2, dim, dim)
    _, y = oracle.layer_norm_modulated(x, None, None, gamma, beta, scale, shift, 3, 1e-5)
    for r in range(rows):
        b = r // 3
        ops = (scale[0][b] + scale[1]).astype(np.float32) + np.float32(1)
        sh = (shift[0][b] + shift[1]).astype(np.float32)
        want = (beta * ops).astype(np.float32) + sh
        assert np.array_equal(y[r], want)
