"""levo_hip_sample_step_static (the decode step on the library's own scratch,
no allocation) against levo_hip_sample_step with a caller workspace: two
calls in a row, the second smaller, every output identical; calls beyond the
scratch size are refused."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import from_dev
from test_gpu_sample_step import Case, workspace
from test_gpu_sampling import _f16_logits, peek_bits

pytestmark = pytest.mark.gpu


def _outputs_equal(a, b):
    for k in a:
        x, y = np.asarray(a[k]), np.asarray(b[k])
        assert np.array_equal(x.view(np.uint8), y.view(np.uint8)), k


def test_static_scratch_matches_workspace_entry(hip, binding, dev, oracle):
    calls = [(3, 16385, [50, 1, 1], True), (2, 4097, [7, 1], False)]  # second call smaller
    for rows, V, top_k, penalty in calls:
        cond = _f16_logits(oracle, rows, V, 3000 + V)
        uncond = _f16_logits(oracle, rows, V, 3100 + V)
        recent = None
        if penalty:
            recent = np.random.default_rng(V).integers(-1, V, (rows, 50)).astype(np.int64)
        c = Case(binding, dev, cond, uncond, top_k=top_k, n_streams=len(top_k), recent=recent, penalty_limit=V - 1,
                 ignore=(3, 9) if penalty else None)
        bits = peek_bits(oracle, 60 + rows, 0, rows)
        want = c.step(hip, ws=workspace(hip, dev, rows, V), bits=bits)
        a, o = c.outputs()
        hip.sample_step_static(a, c.draw_args(o, bits, 0.9, True))
        got = {k: from_dev(v) for k, v in o.items()}
        _outputs_equal(got, want)
        assert got["count"].min() >= 1 and np.all(got["draws"] == np.arange(1, rows + 1))


def test_static_scratch_refuses_oversized_calls(hip, binding, dev, oracle):
    V = 16385
    fits = max(r for r in range(1, 400) if hip.sample_step_workspace_bytes(r, V) <= 2 << 20)
    assert fits >= 200  # the documented capacity at this vocabulary
    rows = fits + 1
    c = Case(binding, dev, np.zeros((rows, V), np.float32), None, top_k=[5], n_streams=1)
    a, o = c.outputs()
    with pytest.raises(binding.LevoHipError, match="bytes of scratch"):
        hip.sample_step_static(a, None)
    a.rows = fits  # the largest call that fits at this vocabulary
    hip.sample_step_static(a, None)
    assert np.all(from_dev(o["count"])[:fits] == 16385)  # all-zero rows: every id ties at top-5
