"""Shared fixtures: the CPU oracle (checker), the compiled reference sources,
and the HIP library loaded through its C ABI."""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_levo_hip():
    """Import levo2.cpp_amd/levo_hip.py (the directory name is not a Python identifier)."""
    name = "levo_hip_binding"
    if name in sys.modules:
        return sys.modules[name]
    path = os.path.join(ROOT, "levo2.cpp_amd", "levo_hip.py")
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def oracle():
    from oracle.levo_oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.levo_oracle import Reference, have_reference
    if not have_reference():
        pytest.skip("oracle/_ref is not built (reference checkout absent when building)")
    return Reference()


@pytest.fixture(scope="session")
def binding():
    return load_levo_hip()


@pytest.fixture(scope="session")
def hip(binding):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return binding.LevoHip()


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


# ---- helpers shared by the GPU parity tests ----------------------------------------

def to_dev(a: np.ndarray, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def from_dev(t) -> np.ndarray:
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def f32_err(actual: np.ndarray, expected: np.ndarray) -> float:
    """max_i |a - b| / max(|b|, 1): relative above 1, absolute below."""
    a = actual.astype(np.float64).ravel()
    b = expected.astype(np.float64).ravel()
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1.0)))


def f16_ulp(actual_bits: np.ndarray, expected_bits: np.ndarray) -> int:
    """Max distance in F16 units in the last place (ordered-integer metric)."""
    def ordered(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, 0x8000 - (h & 0x7FFF), 0x8000 + (h & 0x7FFF))
    if actual_bits.size == 0:
        return 0
    return int(np.max(np.abs(ordered(actual_bits.ravel()) - ordered(expected_bits.ravel()))))


@pytest.fixture(autouse=True)
def _announce_gpu_case(request):
    """Name each GPU case on the real stderr before it touches the device."""
    if request.node.get_closest_marker("gpu") is not None:
        sys.__stderr__.write(f"\n[gpu-case] {request.node.nodeid}\n")
        sys.__stderr__.flush()
    yield
