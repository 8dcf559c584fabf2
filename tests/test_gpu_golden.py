"""The HIP path against the reference's own outputs in
tests/golden/reference_sampling.npz (see tests/golden/make_golden.py): CFG bit
for bit, sampled tokens and the mt19937_64 cursor token for token (kernel
candidate set + the host draw of sample_top_k_counted), the standalone
repetition penalty bit for bit."""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import from_dev, to_dev
from test_gpu_sampling import host_draw, run_sample

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_sampling.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("scale", [1.5, 2.0, 0.0])
def test_cfg_combine(hip, dev, gold, scale):
    import torch
    key = str(scale).replace(".", "p")
    c, u = gold["cfg_cond"], gold["cfg_uncond"]
    out = torch.empty(c.size, dtype=torch.float32, device=dev)
    hip.cfg_combine(out, to_dev(u, dev), to_dev(c, dev), c.size, scale)
    assert np.array_equal(from_dev(out).view(np.uint32), gold[f"cfg_apply_{key}"].view(np.uint32))


def test_single_row_sampler(hip, binding, dev, oracle, gold):
    rows = gold["one_rows"].astype(np.float32)
    V = rows.shape[1]
    rng, draws = oracle.mt(int(gold["one_seed"][0])), 0
    for i in range(rows.shape[0]):
        k, t, use = int(gold["one_k"][i]), float(gold["one_t"][i]), bool(gold["one_use"][i])
        out = run_sample(hip, binding, dev, rows[i:i + 1], None, top_k=[k], n_streams=1,
                         temperature=t if t > 0 else 1.0, capacity=V, lse=False)
        tok, draws = host_draw(oracle, rng, draws, out["ids"][0], out["logits"][0], int(out["best"][0]),
                               int(out["count"][0]), t, use)
        assert tok == gold["one_tokens"][i], i
        assert draws == gold["one_draws"][i], i


@pytest.mark.parametrize("seed", [77, 78, 79])
def test_stream_generation_loop(hip, binding, dev, oracle, gold, seed):
    """CFG fused in the kernel (cond / uncond in, adjusted logits never leave
    the GPU), penalty window of the fed-back ids, stream-0 ignore list."""
    cond, uncond = gold["streams_cond"].astype(np.float32), gold["streams_uncond"].astype(np.float32)
    P, S, V = cond.shape
    temp, use = gold[f"streams_params_{seed}"]
    window = int(gold["streams_window"][0])
    rng, draws = oracle.mt(seed), 0
    history = [[] for _ in range(S)]
    for p in range(P):
        width = min(window, len(history[0]))
        recent = np.array([h[-width:] for h in history], np.int64) if width else None
        out = run_sample(hip, binding, dev, cond[p], uncond[p], top_k=[50, 1, 1], n_streams=S,
                         temperature=float(temp), capacity=V, recent=recent,
                         penalty=float(gold["streams_penalty"][0]), penalty_limit=V - 1,
                         ignore=gold["streams_ignore"], lse=False)
        toks = []
        for q in range(S):
            tok, draws = host_draw(oracle, rng, draws, out["ids"][q], out["logits"][q], int(out["best"][q]),
                                   int(out["count"][q]), float(temp), bool(use))
            toks.append(tok)
            history[q].append(tok)
        assert toks == gold[f"streams_tokens_{seed}"][p].tolist(), p
        assert draws == gold[f"streams_draws_{seed}"][p], p


def test_repetition_penalty(hip, dev, gold):
    import torch
    for penalty, limit, key in ((1.1, 0, "pen_out_full"), (2.0, 299, "pen_out_limit")):
        d = to_dev(gold["pen_logits"], dev)
        r = torch.from_numpy(gold["pen_recent"]).to(dev)
        hip.repetition_penalty(d, d.numel(), r, r.numel(), penalty, limit)
        assert np.array_equal(from_dev(d).view(np.uint32), gold[key].view(np.uint32))
