"""CFG + temperature softmax + argmax / top-k on the GPU vs the oracle and
the compiled reference sampler (src/levo-sampling.cpp).

Bars: argmax ids, candidate ids (top-k with ties) and candidate logits are
bit-exact; probabilities and the log-sum-exp are F32 outputs (<= 1e-5);
sampled tokens drawn on the host from the GPU candidates, and those drawn
on the GPU by levo_hip_sample_draw, equal the reference Sampler's tokens
and its draw cursor.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev

pytestmark = pytest.mark.gpu


def run_sample(hip, binding, dev, cond, uncond, *, top_k, n_streams, temperature=0.9, scale=1.5, capacity=64,
               vocab=None, pitch=None, recent=None, penalty=1.1, penalty_limit=0, ignore=None, lse=True):
    import torch
    rows = cond.shape[0]
    V = vocab if vocab is not None else cond.shape[1]
    P = pitch if pitch is not None else cond.shape[1]
    cd = to_dev(cond, dev)
    ud = to_dev(uncond, dev) if uncond is not None else None
    a = binding.SampleArgs()
    a.cond = cd.data_ptr()
    a.uncond = ud.data_ptr() if ud is not None else None
    a.rows, a.vocab, a.row_pitch = rows, V, P
    a.cfg_scale, a.temperature, a.n_streams = scale, temperature, n_streams
    for i, k in enumerate(top_k):
        a.top_k[i] = k
    keep = []
    if recent is not None:
        rd = to_dev(np.ascontiguousarray(recent, np.int64), dev)
        keep.append(rd)
        a.recent, a.n_recent, a.repetition_penalty, a.penalty_limit = rd.data_ptr(), recent.shape[1], penalty, penalty_limit
    if ignore is not None and len(ignore):
        idd = to_dev(np.asarray(ignore, np.int64), dev)
        keep.append(idd)
        a.ignore, a.n_ignore = idd.data_ptr(), len(ignore)
    best = torch.empty(rows, dtype=torch.int32, device=dev)
    count = torch.empty(rows, dtype=torch.int32, device=dev)
    ids = torch.full((rows, capacity), -7, dtype=torch.int32, device=dev)
    lg = torch.empty((rows, capacity), dtype=torch.float32, device=dev)
    pr = torch.empty((rows, capacity), dtype=torch.float32, device=dev)
    mx = torch.empty(rows, dtype=torch.float32, device=dev)
    ls = torch.empty(rows, dtype=torch.float32, device=dev) if lse else None
    a.best, a.count, a.cand_ids, a.cand_logits, a.cand_probs = (best.data_ptr(), count.data_ptr(), ids.data_ptr(),
                                                                lg.data_ptr(), pr.data_ptr())
    a.row_max = mx.data_ptr()
    a.row_lse = ls.data_ptr() if lse else None
    a.capacity = capacity
    hip.cfg_sample(a)
    out = dict(best=from_dev(best), count=from_dev(count), ids=from_dev(ids), logits=from_dev(lg),
               probs=from_dev(pr), max=from_dev(mx),
               dev=dict(best=best, count=count, ids=ids, logits=lg, max=mx, capacity=capacity))
    if lse:
        out["lse"] = from_dev(ls)
    return out


def weights_f64(vals, m, t):
    """src/levo-sampling.cpp:102-107: exp((double)((v - max) / T)), -inf -> 0."""
    v = np.asarray(vals, np.float32)
    w = np.where(np.isneginf(v), 0.0, np.exp(((v - np.float32(m)) / np.float32(t)).astype(np.float64)))
    return w


def check_rows(out, adjusted, top_ks, oracle, temperature, rows=None, lse=True):
    R = adjusted.shape[0]
    for r in (range(R) if rows is None else rows):
        row = adjusted[r]
        k = top_ks[r]
        best, cand = oracle.top_k_candidates(row, k)
        assert out["best"][r] == best, r
        assert out["count"][r] == cand.size, (r, out["count"][r], cand.size)
        n = min(cand.size, out["ids"].shape[1])
        assert np.array_equal(out["ids"][r, :n], cand[:n]), r
        assert np.array_equal(out["logits"][r, :n].view(np.uint32), row[cand[:n]].view(np.uint32)), r
        # max_logit of the reference: std::max over the candidates in id order
        # keeps the first of equal values, i.e. the value at `best` (sign of a 0 tie)
        m = np.float32(row[best])
        assert out["max"][r].view(np.uint32) == m.view(np.uint32)
        w = weights_f64(row[cand], m, temperature)
        if w.sum() > 0 and np.isfinite(w.sum()):
            assert f32_err(out["probs"][r, :n], w[:n] / w.sum()) <= 1e-5, r
        if lse:
            z = row.astype(np.float64) / temperature
            want = z.max() + math.log(np.exp(z - z.max()).sum())
            assert f32_err(out["lse"][r:r + 1], np.array([want])) <= 1e-5, r


def test_config_batch_750_positions(hip, binding, dev, oracle):
    """cond/uncond [750][3][16384] ~N(0,3), s = 1.5, T = 0.9, top-50; argmax ids bit-exact."""
    P, S, V = 750, 3, 16384
    cond = (oracle.gaussian(P * S * V, 501) * 3).reshape(P * S, V)
    uncond = (oracle.gaussian(P * S * V, 502) * 3).reshape(P * S, V)
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 50, 50], n_streams=3)
    adjusted = oracle.apply_cfg(cond, uncond, 1.5)
    check_rows(out, adjusted, [50] * (P * S), oracle, 0.9)


def _f16_logits(oracle, rows, V, seed):
    return oracle.f16_to_f32(oracle.f32_to_f16((oracle.gaussian(rows * V, seed) * 3).reshape(rows, V)))


@pytest.mark.parametrize("k", [1, 2, 50, 64, 65, 100, 300, 0, 16383, 16384])
def test_ties_and_k(hip, binding, dev, oracle, k):
    V, R = 16384, 24
    cond = _f16_logits(oracle, R, V, 600 + k)
    # plant ties: at the max, at the k-th value, whole row equal, -0 / +0
    cond[1, 5000:5040] = cond[1].max() + 1.0
    srt = np.sort(cond[2])[::-1]
    if 0 < k < V:
        cond[2, :40] = srt[k - 1]
    cond[3, :] = 0.5
    cond[4, :] = 0.0
    cond[4, ::3] = -0.0
    out = run_sample(hip, binding, dev, cond, None, top_k=[k], n_streams=1, capacity=512)
    check_rows(out, cond, [k] * R, oracle, 0.9)


def test_reference_stream_config_with_ties(hip, binding, dev, oracle):
    """sampling_config defaults: mixed stream top-50, vocal/BGM top-1 (src/levo-sampling.h:17-25)."""
    P, S, V = 120, 3, 16384
    cond = _f16_logits(oracle, P * S, V, 700)
    uncond = _f16_logits(oracle, P * S, V, 701)
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 1, 1], n_streams=3)
    adjusted = oracle.apply_cfg(cond, uncond, 1.5)
    check_rows(out, adjusted, [50, 1, 1] * P, oracle, 0.9)


def test_vocab_16385_packed_rows(hip, binding, dev, oracle):
    """The real LeLM rows hold 16384 codes + EOS (src/levo-model.h:121): unaligned pitch."""
    R, V = 30, 16385
    cond = _f16_logits(oracle, R, V, 800)
    uncond = _f16_logits(oracle, R, V, 801)
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 1, 1], n_streams=3)
    check_rows(out, oracle.apply_cfg(cond, uncond, 1.5), [50, 1, 1] * 10, oracle, 0.9)
    # the same rows at a padded, 16-byte aligned pitch take the vector path
    pad = np.zeros((R, 16388), np.float32)
    padu = np.zeros((R, 16388), np.float32)
    pad[:, :V], padu[:, :V] = cond, uncond
    out2 = run_sample(hip, binding, dev, pad, padu, top_k=[50, 1, 1], n_streams=3, vocab=V, pitch=16388)
    for key in ("best", "count", "max"):
        assert np.array_equal(out[key], out2[key])
    for r in range(R):
        n = out["count"][r]
        assert np.array_equal(out["ids"][r, :n], out2["ids"][r, :n])
        assert np.array_equal(out["logits"][r, :n].view(np.uint32), out2["logits"][r, :n].view(np.uint32))


@pytest.mark.parametrize("V", [1, 3, 4, 100, 1000, 5000])
def test_small_vocabularies(hip, binding, dev, oracle, V):
    R = 12
    cond = _f16_logits(oracle, R, V, 900 + V)
    ks = [1, 2, 3, 0]
    out = run_sample(hip, binding, dev, cond, None, top_k=ks, n_streams=4, capacity=max(V, 1))
    check_rows(out, cond, ks * (R // 4), oracle, 0.9)


def test_penalty_and_ignore_lists(hip, binding, dev, oracle):
    P, S, V = 40, 3, 16385
    cond = _f16_logits(oracle, P * S, V, 1000)
    uncond = _f16_logits(oracle, P * S, V, 1001)
    rng = np.random.default_rng(5)
    recent = rng.integers(-1, V, size=(P * S, 50))
    recent[:, :10] = rng.integers(0, 40, size=(P * S, 10))   # repeats: divided once
    recent[0, :] = V - 1                                        # EOS is excluded by the limit
    ignore = [3, 9, 77, 16000, V + 5, -2]
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 1, 1], n_streams=3, recent=recent,
                     penalty=1.1, penalty_limit=V - 1, ignore=ignore)
    adjusted = oracle.apply_cfg(cond, uncond, 1.5)
    for r in range(P * S):
        adjusted[r] = oracle.repetition_penalty(adjusted[r], recent[r], 1.1, V - 1)
        if r % 3 == 0:
            for t in ignore:
                if 0 <= t < V:
                    adjusted[r, t] = -np.inf
    check_rows(out, adjusted, [50, 1, 1] * P, oracle, 0.9)


def test_nan_and_degenerate_rows(hip, binding, dev, oracle):
    V = 4096
    cond = _f16_logits(oracle, 6, V, 1100)
    cond[0, 17] = np.nan                 # rejected like the reference ("logits contain NaN")
    cond[1, 3] = np.nan                  # stream-1 row: the ignore list does not apply, NaN stays
    cond[2, :] = -np.inf                 # everything -inf: all ids stay candidates
    cond[3, :] = np.inf
    cond[3, 10:] = 0.0                   # +inf maxima
    out = run_sample(hip, binding, dev, cond, None, top_k=[50, 50], n_streams=2, ignore=[3], capacity=V)
    assert out["best"][0] == -1 and out["count"][0] == -1
    adjusted = cond.copy()
    adjusted[[2, 4], 3] = -np.inf        # ignore list applies to stream-0 rows only (2, 4)
    adjusted[1, 3] = np.nan              # row 1 is stream 1: its NaN stays
    assert out["count"][1] == -1
    check_rows(out, adjusted, [50] * 6, oracle, 0.9, rows=[2, 3, 4, 5], lse=False)
    assert out["count"][2] == V and out["best"][2] == 0
    assert out["probs"][2, 0] == 1.0 and np.all(out["probs"][2, 1:] == 0.0)  # falls back to best


@pytest.mark.parametrize("V,pitch", [(20000, 20000), (32768, 32768), (24001, 24001), (18432, 18432),
                                     (16896, 16897)])
def test_large_vocabularies(hip, binding, dev, oracle, V, pitch):
    """Rows above the LeLM codebook up to the 32768-id limit: the vector path
    with 64 logits per thread (full and padded), the largest 36-per-thread
    shape, and the scalar path (unaligned pitch) at its two largest shapes;
    with CFG, top-k 50 / 1 and planted ties at the maximum."""
    R = 6
    cond = np.zeros((R, pitch), np.float32)
    uncond = np.zeros((R, pitch), np.float32)
    cond[:, :V] = _f16_logits(oracle, R, V, 1300 + V)
    uncond[:, :V] = _f16_logits(oracle, R, V, 1400 + V)
    cond[1, [5, V - 3]] = 40.0   # tied maxima after CFG (u + 1.5 (c - u) equal only if u equal)
    uncond[1, [5, V - 3]] = 0.0
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 1], n_streams=2, vocab=V, pitch=pitch)
    adjusted = oracle.apply_cfg(cond[:, :V].copy(), uncond[:, :V].copy(), 1.5)
    check_rows(out, adjusted, [50, 1] * (R // 2), oracle, 0.9)
    assert out["best"][1] == 5 and out["count"][1] == 2


@pytest.mark.parametrize("V", [4096, 5000, 16384])
def test_special_values_without_lists(hip, binding, dev, oracle, V):
    """NaN, +inf and -inf runs on rows with no penalty or ignore list: the
    streamed softmax statistics must send NaN and +inf rows to the exact check,
    and -inf or very low first groups must not poison the log-sum-exp. A
    thread's first group is ids 4t .. 4t + 3 (512 threads x 4 ids per chunk,
    so the first chunk is ids 0 .. 2047); its maximum is the thread's fixed
    shift. V = 4096 / 16384 fill every item; 5000 leaves padding."""
    cond = _f16_logits(oracle, 10, V, 1200 + V)
    cond[0, V // 2] = np.nan
    cond[1, [7, V - 1]] = np.inf
    cond[2, :2000] = -np.inf
    cond[3, :] = -np.inf
    ids = np.arange(V)
    cond[4, ids < 2048] = -np.inf          # every thread's first group all -inf
    cond[5, 0] = -np.inf
    cond[7, (ids < 2048) & (ids % 4 == 0)] = -np.inf   # one -inf in every first group
    cond[8, ids < 2048] = -200.0           # shift so low that later terms overflow
    cond[9, ids < 2048] = -30.0            # shift 2^48 terms below the later values
    out = run_sample(hip, binding, dev, cond, None, top_k=[50], n_streams=1, capacity=V)
    assert out["best"][0] == -1 and out["count"][0] == -1
    check_rows(out, cond, [50] * 10, oracle, 0.9, rows=[2, 4, 5, 6, 7, 8, 9])
    check_rows(out, cond, [50] * 10, oracle, 0.9, rows=[1, 3], lse=False)
    assert out["lse"][1] == np.inf and out["lse"][3] == -np.inf
    assert out["count"][3] == V and out["best"][3] == 0


def test_capacity_overflow_reports_full_count(hip, binding, dev, oracle):
    V = 3000
    cond = _f16_logits(oracle, 2, V, 1200)
    out = run_sample(hip, binding, dev, cond, None, top_k=[0], n_streams=1, capacity=64)
    assert np.all(out["count"] == V)
    assert np.array_equal(out["ids"][0], np.arange(64))


def host_draw(oracle, rng, draws, ids, logits, best, count, temperature, use_sampling):
    """The host half of sample_top_k_counted (src/levo-sampling.cpp:97-115):
    returns (token, draws) from the GPU candidate list."""
    if not use_sampling or temperature == 0.0:
        return best, draws
    cand = np.asarray(logits[:count], np.float32)
    m = np.float32(cand.max())
    w = weights_f64(cand, m, temperature)
    total = 0.0
    for x in w:
        total += float(x)
    if not (total > 0.0) or not math.isfinite(total):
        return best, draws
    u = ((oracle.mt_next(rng) >> 11) + 0.5) / 9007199254740992.0
    target = u * total
    cum = 0.0
    for i, x in enumerate(w):
        cum += float(x)
        if target < cum:
            return int(ids[i]), draws + 1
    return int(ids[count - 1]), draws + 1


def test_sampled_tokens_match_reference_sampler(hip, binding, dev, oracle, ref):
    P, S, V = 60, 3, 16385
    cond = _f16_logits(oracle, P * S, V, 1300)
    uncond = _f16_logits(oracle, P * S, V, 1301)
    for seed, temp, use in ((11, 0.9, True), (12, 0.3, True), (13, 0.9, False)):
        s = ref.sampler(seed)
        rng, draws = oracle.mt(seed), 0
        recent = np.full((S, 50), -1, np.int64)
        adjusted = oracle.apply_cfg(cond, uncond, 1.5)
        for pos in range(P):
            rows = slice(pos * S, pos * S + S)
            want = s.sample_streams(adjusted[rows], use_sampling=use, temperature=temp, top_k_mixed=50,
                                    top_k_detail=1, repetition_penalty=1.1, recent=recent, ignore=(3, 9))
            out = run_sample(hip, binding, dev, cond[rows], uncond[rows], top_k=[50, 1, 1], n_streams=3,
                             temperature=temp, capacity=256, recent=recent, penalty=1.1, penalty_limit=V - 1,
                             ignore=(3, 9), lse=False)
            got = []
            for q in range(S):
                assert 0 <= out["count"][q] <= 256
                tok, draws = host_draw(oracle, rng, draws, out["ids"][q], out["logits"][q], int(out["best"][q]),
                                       int(out["count"][q]), temp, use)
                got.append(tok)
            assert got == want.tolist(), (seed, pos)
            recent = np.concatenate([recent[:, 1:], np.array(got, np.int64)[:, None]], axis=1)
        assert draws == s.draw_count


@pytest.mark.parametrize("vocab,limit", [(16385, 16384), (16385, 0), (5, 3), (600_000, 0)])
def test_standalone_repetition_penalty_matches_oracle(hip, dev, oracle, vocab, limit):
    """levo_hip_repetition_penalty == apply_unique_token_repetition_penalty
    (src/levo-sampling.cpp:39-47): duplicates divide once, ids outside
    [0, limit) are ignored. 600,000 ids exercises the first-occurrence scan."""
    import torch
    rng = np.random.default_rng(vocab + limit)
    logits = (rng.standard_normal(vocab) * 3).astype(np.float32)
    top = limit if limit else vocab
    recent = np.concatenate([rng.integers(0, top, 40), rng.integers(0, top, 10),
                             [-1, -7, vocab, vocab + 5, top - 1, top - 1, 0, 0]]).astype(np.int64)
    recent[45:50] = recent[0:5]  # forced duplicates
    want = oracle.repetition_penalty(logits.copy(), recent, 1.1, limit)
    d = to_dev(logits, dev)
    r = torch.from_numpy(recent).to(dev)
    hip.repetition_penalty(d, vocab, r, len(recent), 1.1, limit)
    got = from_dev(d)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_standalone_repetition_penalty_reference_kat(hip, dev, binding):
    """tests/test-sampling.cpp:9-11: {10,8,6} with {0,0,1}, penalty 2 -> {5,4,6};
    a non-positive penalty is rejected with the reference's message."""
    import torch
    d = torch.tensor([10.0, 8.0, 6.0], device=dev)
    r = torch.tensor([0, 0, 1], dtype=torch.int64, device=dev)
    hip.repetition_penalty(d, 3, r, 3, 2.0)
    assert from_dev(d).tolist() == [5.0, 4.0, 6.0]
    with pytest.raises(binding.LevoHipError, match="repetition penalty must be finite and positive"):
        hip.repetition_penalty(d, 3, r, 3, 0.0)


# ---- levo_hip_sample_draw -------------------------------------------------------

def run_draw(hip, binding, dev, out, bits, *, temperature, use_sampling=True):
    """levo_hip_sample_draw over the device outputs of run_sample; bits are
    the raw engine values handed to the rows in order."""
    import torch
    d = out["dev"]
    rows = d["best"].numel()
    b = torch.tensor(np.asarray(bits, np.uint64).view(np.int64), dtype=torch.int64, device=dev)
    tokens = torch.full((rows,), -99, dtype=torch.int64, device=dev)
    draws = torch.full((rows,), -99, dtype=torch.int32, device=dev)
    a = binding.DrawArgs()
    a.best, a.count, a.cand_ids = d["best"].data_ptr(), d["count"].data_ptr(), d["ids"].data_ptr()
    a.cand_logits, a.row_max = d["logits"].data_ptr(), d["max"].data_ptr()
    a.rows, a.capacity, a.temperature, a.use_sampling = rows, d["capacity"], temperature, int(use_sampling)
    a.bits, a.tokens, a.draws = b.data_ptr(), tokens.data_ptr(), draws.data_ptr()
    hip.sample_draw(a)
    return from_dev(tokens), from_dev(draws)


def peek_bits(oracle, seed, consumed, n):
    """The next n raw mt19937_64 values after `consumed` draws from `seed`."""
    rng = oracle.mt(seed)
    oracle.lib.lo_mt_discard(__import__("ctypes").byref(rng), consumed)
    return np.array([oracle.mt_next(rng) for _ in range(n)], np.uint64)


def test_device_draw_matches_reference_sampler(hip, binding, dev, oracle, ref):
    """Sampler::sample_streams (src/levo-sampling.cpp:129-152) over 60
    positions of 3 streams with CFG, penalty windows and the ignore list: the
    ids drawn on the GPU and the engine cursor equal the reference's."""
    P, S, V = 60, 3, 16385
    cond = _f16_logits(oracle, P * S, V, 1400)
    uncond = _f16_logits(oracle, P * S, V, 1401)
    adjusted = oracle.apply_cfg(cond, uncond, 1.5)
    for seed, temp in ((21, 0.9), (22, 0.25), (23, 2.0)):
        s = ref.sampler(seed)
        consumed = 0
        recent = np.full((S, 50), -1, np.int64)
        for pos in range(P):
            rows = slice(pos * S, pos * S + S)
            want = s.sample_streams(adjusted[rows], use_sampling=True, temperature=temp, top_k_mixed=50,
                                    top_k_detail=1, repetition_penalty=1.1, recent=recent, ignore=(3, 9))
            out = run_sample(hip, binding, dev, cond[rows], uncond[rows], top_k=[50, 1, 1], n_streams=3,
                             temperature=temp, capacity=64, recent=recent, penalty=1.1, penalty_limit=V - 1,
                             ignore=(3, 9), lse=False)
            tokens, draws = run_draw(hip, binding, dev, out, peek_bits(oracle, seed, consumed, S), temperature=temp)
            assert tokens.tolist() == want.tolist(), (seed, pos)
            assert draws.tolist() == [1, 2, 3]
            consumed += int(draws[-1])
            recent = np.concatenate([recent[:, 1:], tokens[:, None]], axis=1)
        assert consumed == s.draw_count


def test_device_draw_batch_750_positions(hip, binding, dev, oracle):
    """The [750][3][16384] batch, top-50, T = 0.9: row r draws bits[r]; every
    id equals the host draw of sample_top_k_counted over the same candidates."""
    P, S, V = 750, 3, 16384
    cond = (oracle.gaussian(P * S * V, 511) * 3).reshape(P * S, V)
    uncond = (oracle.gaussian(P * S * V, 512) * 3).reshape(P * S, V)
    out = run_sample(hip, binding, dev, cond, uncond, top_k=[50, 50, 50], n_streams=3, lse=False)
    bits = peek_bits(oracle, 77, 0, P * S)
    tokens, draws = run_draw(hip, binding, dev, out, bits, temperature=0.9)
    assert np.array_equal(draws, np.arange(1, P * S + 1))
    rng, consumed = oracle.mt(77), 0
    want = []
    for r in range(P * S):
        tok, consumed = host_draw(oracle, rng, consumed, out["ids"][r], out["logits"][r], int(out["best"][r]),
                                  int(out["count"][r]), 0.9, True)
        want.append(tok)
    assert tokens.tolist() == want


def test_device_draw_special_rows(hip, binding, dev, oracle):
    """Rows that do not draw: NaN (token -1, the reference throws), all -inf
    and +inf maxima (the first maximum, no draw, :108), greedy and T = 0;
    an overflowing candidate set reports -2 but still counts its draw."""
    V = 4096
    cond = _f16_logits(oracle, 6, V, 1500)
    cond[1, 17] = np.nan
    cond[2, :] = -np.inf
    cond[3, 10] = np.inf
    cond[5, :] = 1.0                      # 4096 tied candidates, capacity 64
    out = run_sample(hip, binding, dev, cond, None, top_k=[50], n_streams=1, capacity=64, lse=False)
    bits = peek_bits(oracle, 5, 0, 6)
    tokens, draws = run_draw(hip, binding, dev, out, bits, temperature=0.9)
    rng, consumed = oracle.mt(5), 0
    t0, consumed = host_draw(oracle, rng, consumed, out["ids"][0], out["logits"][0], int(out["best"][0]),
                             int(out["count"][0]), 0.9, True)
    assert tokens[0] == t0 and draws[0] == 1
    assert tokens[1] == binding.TOKEN_NAN and draws[1] == 1
    assert tokens[2] == out["best"][2] == 0 and draws[2] == 1
    assert tokens[3] == out["best"][3] == 10 and draws[3] == 1
    t4, consumed = host_draw(oracle, rng, consumed, out["ids"][4], out["logits"][4], int(out["best"][4]),
                             int(out["count"][4]), 0.9, True)
    assert tokens[4] == t4 and draws[4] == 2
    assert tokens[5] == binding.TOKEN_OVERFLOW and draws[5] == 3
    for temp, use in ((0.9, False), (0.0, True)):
        tokens, draws = run_draw(hip, binding, dev, out, bits, temperature=temp, use_sampling=use)
        assert tokens[[0, 2, 3, 4, 5]].tolist() == out["best"][[0, 2, 3, 4, 5]].tolist()
        assert tokens[1] == binding.TOKEN_NAN and np.all(draws == 0)


def test_device_draw_flags_targets_at_a_boundary(hip, binding, dev, oracle):
    """Two equal candidates: weights 1, 1, total 2. The raw value 2^52 << 11
    gives u = (2^52 + 0.5) / 2^53, which rounds to 0.5, so the target is 1.0,
    exactly the first cumulative boundary, where a last-bit difference
    between device and host exp could flip the pick: the row is flagged -3
    (draw on the host). 2^30 raw steps to either side the pick is made on the
    device: candidate 40 above the boundary, 7 below."""
    V = 64
    cond = np.full((1, V), -50.0, np.float32)
    cond[0, 7] = cond[0, 40] = 2.5
    out = run_sample(hip, binding, dev, cond, None, top_k=[2], n_streams=1, capacity=64, lse=False)
    assert out["count"][0] == 2
    tokens, draws = run_draw(hip, binding, dev, out, np.array([(1 << 52) << 11], np.uint64), temperature=0.9)
    assert tokens[0] == binding.TOKEN_RECHECK and draws[0] == 1
    for raw, want in ((((1 << 52) + (1 << 30)) << 11, 40), (((1 << 52) - (1 << 30)) << 11, 7)):
        tokens, draws = run_draw(hip, binding, dev, out, np.array([raw], np.uint64), temperature=0.9)
        assert tokens[0] == want and draws[0] == 1
