"""Writes tests/golden/reference_sampling.npz from the reference's own sources.

Runs the reference's src/levo-sampling.cpp and src/levo-renderer-pattern.cpp,
compiled from the read-only checkout into oracle/_ref/libref_levo.so by
oracle/Makefile (`make -C oracle ref`), on seeded inputs, and stores the inputs
with the reference's outputs:

  cfg_*       levo::apply_cfg and combine_renderer_cfg (src/levo-sampling.cpp:22-28,
              src/levo-renderer-pattern.cpp:123-135), incl. values where an FMA
              would round differently
  one_*       Sampler::sample over single rows with ties, every top-k regime,
              greedy and sampled, one engine (tokens and draw cursor after each)
  streams_*   Sampler::sample_streams over 3 streams x 20 positions with the
              sampled ids fed back as the repetition window and a prompt ignore list
  euler_*     the renderer's Euler time grid (ref_euler_schedule)
  pen_*       apply_unique_token_repetition_penalty

The fixture is data only; the test suites read it without the reference.
Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.levo_oracle import Reference, have_reference  # noqa: E402

OUT = os.path.join(HERE, "reference_sampling.npz")


def f16_grid(rng, shape, scale):
    """Random values that are exact F16 numbers (stored as float16)."""
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def main() -> int:
    if not have_reference():
        sys.stderr.write("oracle/_ref is not built: run `make -C oracle ref REF=/root/reference`\n")
        return 1
    ref = Reference()
    rng = np.random.default_rng(20261201)
    fx = {}

    # ---- CFG ---------------------------------------------------------------------
    c = (rng.standard_normal(4096) * 3).astype(np.float32)
    u = (rng.standard_normal(4096) * 3).astype(np.float32)
    c[:8] = [np.inf, -np.inf, 0.0, -0.0, 1e38, -1e38, 1e-40, 3.0]
    u[:8] = [1.0, 2.0, -0.0, 0.0, -1e38, 1e38, 2e-40, 3.0]
    fx["cfg_cond"], fx["cfg_uncond"] = c, u
    for s in (1.5, 2.0, 0.0):
        key = str(s).replace(".", "p")
        fx[f"cfg_apply_{key}"] = ref.apply_cfg(c, u, s)
        fx[f"cfg_renderer_{key}"] = ref.combine_renderer_cfg(u, c, s)

    # ---- Sampler::sample over single rows -----------------------------------------
    V1, N1 = 512, 96
    rows = f16_grid(rng, (N1, V1), 3.0).astype(np.float32)
    ks = np.array([0, 1, 2, 3, 50, 64, 511, 512, 900] * 11, np.int64)[:N1]
    temps = np.array([0.0, 0.3, 0.9, 1.0, 2.5, 0.9], np.float32)
    one_t = np.array([temps[i % len(temps)] for i in range(N1)], np.float32)
    one_use = np.array([(i % 5) != 4 for i in range(N1)], np.int64)
    for i in range(N1):  # ties at the maximum and around the k-th value
        rows[i, (7 * i) % V1] = rows[i, (13 * i + 5) % V1] = rows[i].max() + 1.0
        rows[i, (3 * i + 1) % V1] = rows[i, (11 * i + 2) % V1]
    rows[5, :] = 0.0                      # all equal
    rows[6, 10:] = -np.inf                # mostly -inf
    rows[7, 1::2] = -0.0                  # +0 / -0 ties
    sampler = ref.sampler(9001)
    one_tok, one_draws = [], []
    for i in range(N1):
        one_tok.append(sampler.sample(rows[i], int(ks[i]), float(one_t[i]), bool(one_use[i])))
        one_draws.append(sampler.draw_count)
    fx.update(one_rows=rows.astype(np.float16), one_k=ks, one_t=one_t, one_use=one_use,
              one_seed=np.array([9001], np.int64), one_tokens=np.array(one_tok, np.int64),
              one_draws=np.array(one_draws, np.int64))

    # ---- Sampler::sample_streams, generation loop ------------------------------------
    P, S, V = 20, 3, 1025                 # V - 1 is the EOS id, excluded from the penalty
    cond = f16_grid(rng, (P, S, V), 3.0)
    uncond = f16_grid(rng, (P, S, V), 3.0)
    ignore = np.array([3, 9, 1023, -4, 5000], np.int64)
    window, penalty = 8, 1.1
    for seed, temp, use in ((77, 0.9, 1), (78, 0.4, 1), (79, 0.9, 0)):
        s = ref.sampler(seed)
        history = [[] for _ in range(S)]
        toks, draws = [], []
        for p in range(P):
            adjusted = ref.apply_cfg(cond[p].astype(np.float32), uncond[p].astype(np.float32), 1.5)
            width = min(window, len(history[0]))
            recent = np.full((S, max(width, 1)), -1, np.int64)
            for q in range(S):
                if width:
                    recent[q, :width] = history[q][-width:]
            got = s.sample_streams(adjusted, use_sampling=bool(use), temperature=temp, top_k_mixed=50,
                                   top_k_detail=1, repetition_window=window, repetition_penalty=penalty,
                                   recent=recent if width else None, ignore=ignore)
            for q in range(S):
                history[q].append(int(got[q]))
            toks.append(got)
            draws.append(s.draw_count)
        fx[f"streams_tokens_{seed}"] = np.array(toks, np.int64)
        fx[f"streams_draws_{seed}"] = np.array(draws, np.int64)
        fx[f"streams_params_{seed}"] = np.array([temp, use], np.float32)
    fx.update(streams_cond=cond, streams_uncond=uncond, streams_ignore=ignore,
              streams_window=np.array([window], np.int64), streams_penalty=np.array([penalty], np.float32))

    # ---- Euler time grid ------------------------------------------------------------------
    for steps in (1, 2, 3, 7, 50):
        times, dt = ref.euler_schedule(steps)
        fx[f"euler_times_{steps}"] = times
        fx[f"euler_dt_{steps}"] = np.array([dt], np.float32)

    # ---- repetition penalty ----------------------------------------------------------
    logits = (rng.standard_normal(300) * 3).astype(np.float32)
    recent = np.concatenate([rng.integers(0, 300, 40), [299, 299, -1, 300, 5, 5]]).astype(np.int64)
    fx["pen_logits"], fx["pen_recent"] = logits, recent
    fx["pen_out_full"] = ref.repetition_penalty(logits, recent, 1.1, 0)
    fx["pen_out_limit"] = ref.repetition_penalty(logits, recent, 2.0, 299)

    np.savez_compressed(OUT, **fx)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(fx)} arrays)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
