"""Runs the C++17 drop-in tests (tests/cpp/test-*.cpp) on the GPU.

Each binary restates one of the reference's own C++ tests against the
levo::hip wrappers (tests/test-sampling.cpp, tests/test-flow-renderer.cpp,
tests/test-audio-ops.cpp, tests/test-quantization.cpp) and adds seeded parity
with the oracle; it exits non-zero on the first failed check.
"""
from __future__ import annotations

import glob
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin")
NAMES = ["test-hip-sampling", "test-hip-flow-renderer", "test-hip-ops", "test-hip-vae-decoder"]


@pytest.mark.parametrize("name", NAMES)
def test_cpp_dropin(name):
    path = os.path.join(BIN, name)
    if not os.path.exists(path):
        pytest.fail(f"{path} is not built; run __graft_entry__.build()")
    sys.stderr.write(f"[cpp-test] {name}\n")
    sys.stderr.flush()
    r = subprocess.run([path], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0, f"{name} rc={r.returncode}\nstdout:\n{r.stdout}\nstderr:\n{r.stderr}"
    assert r.stdout.strip().endswith("ok"), r.stdout


def test_every_cpp_test_is_listed():
    built = sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(HERE, "cpp", "test-*.cpp")))
    assert built == sorted(NAMES)
