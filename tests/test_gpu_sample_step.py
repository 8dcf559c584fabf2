"""levo_hip_sample_step (CFG, penalty, ignore list, top-k candidates and the
draw of a decode step; rows split over one-wave parts of 512 ids that hand
over the ids above a bound, joined, selected and drawn in a second launch)
against
levo_hip_cfg_sample + levo_hip_sample_draw on the same inputs, against the
oracle, and against the compiled reference Sampler (src/levo-sampling.cpp).

Bars: best, count, candidate ids and logits, row max, tokens and draw counts
bit-exact; probabilities and the log-sum-exp F32 outputs (<= 1e-5; their
double / float sums run in another order than the two-launch path's).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import f32_err, from_dev, to_dev
from test_gpu_sampling import _f16_logits, check_rows, peek_bits

pytestmark = pytest.mark.gpu


class Case:
    """Device inputs of one sampling call and two sets of outputs."""

    def __init__(self, binding, dev, cond, uncond, *, top_k, n_streams, temperature=0.9, scale=1.5, capacity=64,
                 pitch=None, recent=None, penalty=1.1, penalty_limit=0, ignore=None, lse=True, probs=True):
        import torch
        self.torch, self.binding, self.dev = torch, binding, dev
        rows, V = cond.shape[0], cond.shape[1]
        P = pitch if pitch is not None else V
        if P != V:
            padc = np.zeros((rows, P), np.float32)
            padc[:, :V] = cond
            cond_p = padc
            if uncond is not None:
                padu = np.zeros((rows, P), np.float32)
                padu[:, :V] = uncond
                uncond = padu
        else:
            cond_p = cond
        self.keep = [to_dev(cond_p, dev)]
        if uncond is not None:
            self.keep.append(to_dev(uncond, dev))
        self.rows, self.V, self.capacity, self.lse, self.probs = rows, V, capacity, lse, probs
        self.temperature = temperature
        a = binding.SampleArgs()
        a.cond = self.keep[0].data_ptr()
        a.uncond = self.keep[1].data_ptr() if uncond is not None else None
        a.rows, a.vocab, a.row_pitch = rows, V, P
        a.cfg_scale, a.temperature, a.n_streams = scale, temperature, n_streams
        for i, k in enumerate(top_k):
            a.top_k[i] = k
        if recent is not None:
            rd = to_dev(np.ascontiguousarray(recent, np.int64), dev)
            self.keep.append(rd)
            a.recent, a.n_recent = rd.data_ptr(), recent.shape[1]
            a.repetition_penalty, a.penalty_limit = penalty, penalty_limit
        if ignore is not None and len(ignore):
            idd = to_dev(np.asarray(ignore, np.int64), dev)
            self.keep.append(idd)
            a.ignore, a.n_ignore = idd.data_ptr(), len(ignore)
        a.capacity = capacity
        self.args = a

    def outputs(self):
        t, dev, rows, cap = self.torch, self.dev, self.rows, self.capacity
        o = dict(best=t.full((rows,), -9, dtype=t.int32, device=dev), count=t.full((rows,), -9, dtype=t.int32, device=dev),
                 ids=t.full((rows, cap), -7, dtype=t.int32, device=dev), logits=t.full((rows, cap), -7.0, device=dev),
                 probs=t.full((rows, cap), -7.0, device=dev), max=t.full((rows,), -7.0, device=dev),
                 lse=t.full((rows,), -7.0, device=dev), tokens=t.full((rows,), -99, dtype=t.int64, device=dev),
                 draws=t.full((rows,), -99, dtype=t.int32, device=dev))
        a = self.binding.SampleArgs.from_buffer_copy(self.args)
        a.best, a.count, a.cand_ids = o["best"].data_ptr(), o["count"].data_ptr(), o["ids"].data_ptr()
        a.cand_logits, a.row_max = o["logits"].data_ptr(), o["max"].data_ptr()
        a.cand_probs = o["probs"].data_ptr() if self.probs else None
        a.row_lse = o["lse"].data_ptr() if self.lse else None
        return a, o

    def draw_args(self, o, bits, temperature, use_sampling):
        d = self.binding.DrawArgs()
        d.best, d.count, d.cand_ids = o["best"].data_ptr(), o["count"].data_ptr(), o["ids"].data_ptr()
        d.cand_logits, d.row_max = o["logits"].data_ptr(), o["max"].data_ptr()
        d.rows, d.capacity, d.temperature, d.use_sampling = self.rows, self.capacity, temperature, int(use_sampling)
        b = self.torch.tensor(np.asarray(bits, np.uint64).view(np.int64), dtype=self.torch.int64, device=self.dev)
        self.keep.append(b)
        d.bits, d.tokens, d.draws = b.data_ptr(), o["tokens"].data_ptr(), o["draws"].data_ptr()
        return d

    def two_launch(self, hip, bits=None, temperature=0.9, use_sampling=True):
        a, o = self.outputs()
        hip.cfg_sample(a)
        if bits is not None:
            hip.sample_draw(self.draw_args(o, bits, temperature, use_sampling))
        return {k: from_dev(v) for k, v in o.items()}

    def step(self, hip, ws=None, bits=None, temperature=0.9, use_sampling=True):
        a, o = self.outputs()
        if ws is None:
            ws = workspace(hip, self.dev, self.rows, self.V)
        d = self.draw_args(o, bits, temperature, use_sampling) if bits is not None else None
        hip.sample_step(a, d, ws[0], ws[1])
        return {k: from_dev(v) for k, v in o.items()}


def workspace(hip, dev, rows, V):
    import torch
    n = hip.sample_step_workspace_bytes(rows, V)
    return torch.zeros((n + 15) // 16 * 4, dtype=torch.float32, device=dev), n


def same_outputs(got, want, case, *, draws=False):
    for r in range(case.rows):
        assert got["best"][r] == want["best"][r], r
        assert got["count"][r] == want["count"][r], r
        n = max(0, min(int(want["count"][r]), case.capacity))
        assert np.array_equal(got["ids"][r, :n], want["ids"][r, :n]), r
        assert np.array_equal(got["logits"][r, :n].view(np.uint32), want["logits"][r, :n].view(np.uint32)), r
        assert got["max"][r].view(np.uint32) == want["max"][r].view(np.uint32) or (
            np.isnan(got["max"][r]) and np.isnan(want["max"][r])), r
        if case.probs and want["best"][r] >= 0:
            assert f32_err(got["probs"][r, :n], want["probs"][r, :n]) <= 1e-6, r
        if case.lse and want["best"][r] >= 0:
            if np.isfinite(want["lse"][r]):
                assert f32_err(got["lse"][r:r + 1], want["lse"][r:r + 1]) <= 1e-6, r
            else:
                assert got["lse"][r] == want["lse"][r], r
    if draws:
        assert np.array_equal(got["tokens"], want["tokens"])
        assert np.array_equal(got["draws"], want["draws"])


def test_decode_step_matches_two_launches_and_oracle(hip, binding, dev, oracle):
    """LeVo's decode step: 3 streams x 16385 ids (unaligned rows, the scalar
    loads), CFG 1.5, a 50-id penalty window, ignore list on stream 0, top-k
    50 / 1 / 1, T = 0.9, drawn: every output equals the two-launch path's and
    the oracle's."""
    S, V = 3, 16385
    for seed in range(4):
        cond = _f16_logits(oracle, S, V, 2000 + seed)
        uncond = _f16_logits(oracle, S, V, 2100 + seed)
        rng = np.random.default_rng(seed)
        recent = rng.integers(-1, V, (S, 50)).astype(np.int64)
        recent[:, :5] = recent[:, 5:10]  # duplicates divide once
        c = Case(binding, dev, cond, uncond, top_k=[50, 1, 1], n_streams=3, recent=recent, penalty_limit=V - 1,
                 ignore=(3, 9, 16384))
        bits = peek_bits(oracle, 40 + seed, 0, S)
        want = c.two_launch(hip, bits)
        got = c.step(hip, bits=bits)
        same_outputs(got, want, c, draws=True)
        adjusted = oracle.apply_cfg(cond, uncond, 1.5)
        for r in range(S):
            adjusted[r] = oracle.repetition_penalty(adjusted[r].copy(), recent[r], 1.1, V - 1)
        adjusted[0, [3, 9, 16384]] = -np.inf
        check_rows(got, adjusted, [50, 1, 1], oracle, 0.9)


@pytest.mark.parametrize("V,pitch", [(16384, 16384), (16385, 16388), (2048, 2048), (2049, 2049), (7, 7),
                                     (5000, 5000), (32768, 32768)])
def test_shapes_match_two_launches(hip, binding, dev, oracle, V, pitch):
    """Aligned (vector loads) and unaligned rows, one part, a partial last
    part of one id, tiny and maximal vocabularies; several rows and streams
    with different k."""
    rows = 8
    cond = _f16_logits(oracle, rows, V, 2200 + V)
    uncond = _f16_logits(oracle, rows, V, 2300 + V)
    c = Case(binding, dev, cond, uncond, top_k=[50, 1, 2, 64], n_streams=4, pitch=pitch)
    bits = peek_bits(oracle, V, 0, rows)
    want = c.two_launch(hip, bits)
    got = c.step(hip, bits=bits)
    same_outputs(got, want, c, draws=True)
    check_rows(got, oracle.apply_cfg(cond, uncond, 1.5), [50, 1, 2, 64] * 2, oracle, 0.9)


@pytest.mark.parametrize("rows", [9, 24])
def test_more_rows_than_the_join_draws(hip, binding, dev, oracle, rows):
    """Past 8 rows the join launch leaves the draw to a launch of its own (the
    C++ Sampler takes this entry point up to 4095 rows): candidates, tokens
    and draw counts equal the two-launch path's and the oracle's."""
    V = 16385
    cond = _f16_logits(oracle, rows, V, 2400 + rows)
    uncond = _f16_logits(oracle, rows, V, 2500 + rows)
    c = Case(binding, dev, cond, uncond, top_k=[50, 1, 1], n_streams=3)
    bits = peek_bits(oracle, 60 + rows, 0, rows)
    want = c.two_launch(hip, bits)
    got = c.step(hip, bits=bits)
    same_outputs(got, want, c, draws=True)
    check_rows(got, oracle.apply_cfg(cond, uncond, 1.5), [50, 1, 1] * (rows // 3), oracle, 0.9)


@pytest.mark.parametrize("k", [1, 2, 50, 100, 300, 512, 513, 0, 16383, 16384])
def test_ties_and_k(hip, binding, dev, oracle, k):
    """Ties at the maximum and at the k-th value, +-0, a constant row (more
    ids at a part's bound than a part hands over: the row is selected again
    from its logits), k = 0 and k >= V (keep every id)."""
    V, R = 16384, 6
    cond = _f16_logits(oracle, R, V, 2400 + k)
    cond[0, [5, 900, 15000]] = cond[0].max() + 1.0
    srt = np.sort(cond[1])[::-1]
    kth = srt[min(k, V) - 1] if k else srt[0]
    cond[1, [11, 4000, 9000]] = kth
    cond[2, :] = 0.5
    cond[3, [100, 200]] = 0.0
    cond[3, 300] = -0.0
    cond[3, :100] = -5.0
    cond[4, ::3] = 2.0
    c = Case(binding, dev, cond, None, top_k=[k], n_streams=1, capacity=V)
    want = c.two_launch(hip)
    got = c.step(hip)
    same_outputs(got, want, c)
    check_rows(got, cond, [k] * R, oracle, 0.9)


def test_many_survivors(hip, binding, dev, oracle):
    """A row whose handed-over ids at or above the largest part bound number
    about 290 (the join's second tier, 8 survivors per lane): every part of
    512 ids holds 20 large, distinct values in 20 lanes, so its bound (the
    10th largest lane maximum at k = 50) hands over 10 of them, and the
    largest bound keeps 9 per part. The second row is ordinary."""
    V, R = 16385, 2
    cond = _f16_logits(oracle, R, V, 3300)
    for p in range(V // 512 + 1):
        for l in range(20):
            i = 512 * p + l
            if i < V:
                cond[0, i] = np.float32(100 + 0.01 * l + 1e-5 * p)
    c = Case(binding, dev, cond, None, top_k=[50], n_streams=1, capacity=64)
    bits = peek_bits(oracle, 33, 0, R)
    want = c.two_launch(hip, bits)
    got = c.step(hip, bits=bits)
    same_outputs(got, want, c, draws=True)
    check_rows(got, cond, [50] * R, oracle, 0.9)
    assert got["count"][0] == 50


def test_special_rows(hip, binding, dev, oracle):
    """NaN rows (best = count = -1, token -1), all -inf and +inf maxima (no
    draw), NaN in the last, partial part."""
    V = 4097
    cond = _f16_logits(oracle, 6, V, 2500)
    cond[1, 17] = np.nan
    cond[2, :] = -np.inf
    cond[3, 10] = np.inf
    cond[5, V - 1] = np.nan
    c = Case(binding, dev, cond, None, top_k=[50], n_streams=1, capacity=64)
    bits = peek_bits(oracle, 9, 0, 6)
    want = c.two_launch(hip, bits)
    got = c.step(hip, bits=bits)
    same_outputs(got, want, c, draws=True)
    assert got["best"][1] == -1 and got["best"][5] == -1
    assert got["tokens"][1] == binding.TOKEN_NAN


def test_greedy_and_no_draw(hip, binding, dev, oracle):
    """use_sampling 0 and T = 0: tokens are the first maxima, no draws; no
    draw block: only the candidate outputs."""
    V = 16385
    cond = _f16_logits(oracle, 3, V, 2600)
    c = Case(binding, dev, cond, None, top_k=[50, 1, 1], n_streams=3)
    bits = peek_bits(oracle, 3, 0, 3)
    for temp, use in ((0.9, False), (0.0, True)):
        want = c.two_launch(hip, bits, temperature=temp, use_sampling=use)
        got = c.step(hip, bits=bits, temperature=temp, use_sampling=use)
        same_outputs(got, want, c, draws=True)
        assert np.all(got["draws"] == 0)
    got = c.step(hip)
    assert np.all(got["tokens"] == -99)
    same_outputs(got, c.two_launch(hip), c)


def test_reference_sampler_decode_loop(hip, binding, dev, oracle, ref):
    """Sampler::sample_streams (src/levo-sampling.cpp:129-152) over 40
    positions of 3 streams with CFG, penalty windows and the ignore list, one
    levo_hip_sample_step per position and one workspace reused throughout:
    ids and the engine cursor equal the reference's."""
    P, S, V = 40, 3, 16385
    cond = _f16_logits(oracle, P * S, V, 2700)
    uncond = _f16_logits(oracle, P * S, V, 2701)
    adjusted = oracle.apply_cfg(cond, uncond, 1.5)
    ws = workspace(hip, dev, S, V)
    for seed, temp in ((31, 0.9), (32, 0.3)):
        s = ref.sampler(seed)
        consumed = 0
        recent = np.full((S, 50), -1, np.int64)
        for pos in range(P):
            rows = slice(pos * S, pos * S + S)
            want = s.sample_streams(adjusted[rows], use_sampling=True, temperature=temp, top_k_mixed=50,
                                    top_k_detail=1, repetition_penalty=1.1, recent=recent, ignore=(3, 9))
            c = Case(binding, dev, cond[rows], uncond[rows], top_k=[50, 1, 1], n_streams=3, temperature=temp,
                     recent=recent, penalty_limit=V - 1, ignore=(3, 9), lse=False, probs=False)
            got = c.step(hip, ws=ws, bits=peek_bits(oracle, seed, consumed, S), temperature=temp)
            assert got["tokens"].tolist() == want.tolist(), (seed, pos)
            assert got["draws"].tolist() == [1, 2, 3]
            consumed += int(got["draws"][-1])
            recent = np.concatenate([recent[:, 1:], got["tokens"][:, None]], axis=1)
        assert consumed == s.draw_count


def test_workspace_reused_across_shapes(hip, binding, dev, oracle):
    """One workspace, sized for the largest call and never cleared (it starts
    full of NaN bytes), serves calls of other row counts and vocabularies in
    any order."""
    ws = workspace(hip, dev, 40, 16385)
    ws[0].fill_(float("nan"))
    for rows, V in ((3, 16385), (40, 16385), (5, 2049), (40, 4096), (1, 7), (3, 16385)):
        cond = _f16_logits(oracle, rows, V, 2900 + rows + V)
        c = Case(binding, dev, cond, None, top_k=[50, 1, 3], n_streams=3)
        bits = peek_bits(oracle, rows + V, 0, rows)
        same_outputs(c.step(hip, ws=ws, bits=bits), c.two_launch(hip, bits), c, draws=True)


def test_rejects_bad_arguments(hip, binding, dev, oracle):
    import torch
    V = 2048
    cond = _f16_logits(oracle, 2, V, 2800)
    c = Case(binding, dev, cond, None, top_k=[5], n_streams=1)
    a, o = c.outputs()
    ws, n = workspace(hip, dev, 2, V)
    with pytest.raises(binding.LevoHipError, match="workspace smaller"):
        hip.sample_step(a, None, ws, n - 4)
    with pytest.raises(binding.LevoHipError, match="16-byte aligned"):
        hip.sample_step(a, None, ws.data_ptr() + 4, n)
    d = c.draw_args(o, [1, 2], 0.9, True)
    d.capacity = 32
    with pytest.raises(binding.LevoHipError, match="own candidate outputs"):
        hip.sample_step(a, d, ws, n)
    with pytest.raises(binding.LevoHipError):
        hip.sample_step_workspace_bytes(2, 40000)
    torch.cuda.synchronize()


def test_decode_step_replayed_from_a_graph(hip, binding, dev, oracle):
    """The decode step captured once into a HIP graph (torch.cuda.graph) and
    replayed at 4 positions, each with new logits and raw values copied into
    the graph's fixed input buffers, and eager calls between the replays:
    every replay's tokens, draw counts and candidate sets equal the eager
    calls' on the same inputs. Captured three ways: cfg_sample + sample_draw,
    sample_step on a workspace, and sample_step_static (the entry point for
    callers that cannot allocate, graph capture among them)."""
    import torch
    S, V, P = 3, 16385, 4
    cond = _f16_logits(oracle, P * S, V, 3100)
    uncond = _f16_logits(oracle, P * S, V, 3101)
    recent = np.stack([np.arange(50, dtype=np.int64) * (7 + q) % (V - 1) for q in range(S)])
    case = Case(binding, dev, cond[:S], uncond[:S], top_k=[50, 1, 1], n_streams=3, recent=recent,
                penalty_limit=V - 1, ignore=(3, 9))
    a, o = case.outputs()
    d = case.draw_args(o, peek_bits(oracle, 7, 0, S), 0.9, True)
    bits_t = case.keep[-1]
    ws = workspace(hip, dev, S, V)
    variants = {
        "cfg_sample + sample_draw": lambda: (hip.cfg_sample(a), hip.sample_draw(d)),
        "sample_step": lambda: hip.sample_step(a, d, ws[0], ws[1]),
        "sample_step_static": lambda: hip.sample_step_static(a, d),
    }
    for name, fn in variants.items():
        fn()  # eager first call (the static variant's per-device set-up)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=side):
            fn()
        torch.cuda.synchronize()
        for pos in range(P):
            rows = slice(pos * S, pos * S + S)
            case.keep[0].copy_(to_dev(cond[rows], dev))
            case.keep[1].copy_(to_dev(uncond[rows], dev))
            bits = peek_bits(oracle, 7, S * pos, S)
            bits_t.copy_(torch.tensor(bits.view(np.int64), device=dev))
            want = case.two_launch(hip, bits=bits, temperature=0.9)  # eager, on the same inputs
            for t in o.values():
                t.fill_(-5)
            graph.replay()
            torch.cuda.synchronize()
            got = {k: from_dev(v) for k, v in o.items()}
            print(f"{name}, position {pos}: tokens {got['tokens'].tolist()}")
            same_outputs(got, want, case, draws=True)
