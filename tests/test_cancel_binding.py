"""Cancellation binding of the C++17 drop-in layer (CPU only: compiles, runs
no GPU code).

Built inside the reference tree with -DLEVO_HIP_WITH_LEVO_H, the wrappers
throw the reference's own levo::operation_cancelled (include/levo.h:21-24),
so the reference's `catch (const levo::operation_cancelled &)` sites
(src/levo-flow-renderer.cpp:249, 325; src/cantor-abi.cpp:909) catch what the
drop-in throws. Checked three ways: the alias names the very same type, a
throw through the alias is caught by the reference's catch clause, and the
compiled drop-in objects reference the typeinfo of levo::operation_cancelled
(not a class of their own). Built standalone, the library keeps its own
class. Skipped where the reference checkout is absent.
"""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "levo2.cpp_amd", "host")
REFERENCE_INCLUDE = "/root/reference/include"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
FLAGS = ["-std=c++17", "-O1", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
         "-I", os.path.join(ROOT, "include"), "-I", HOST]
THROWING_SOURCES = ["levo-hip-flow-renderer.cpp", "levo-hip-vae-decoder.cpp"]

needs_reference = pytest.mark.skipif(not os.path.isfile(os.path.join(REFERENCE_INCLUDE, "levo.h")),
                                     reason="reference checkout (include/levo.h) not present")

PROGRAM = r"""
#include "levo.h"
#include "levo-hip-flow-renderer.h"
#include "levo-hip-vae-decoder.h"

#include <cstring>
#include <type_traits>

static_assert(std::is_same_v<levo::hip::operation_cancelled, levo::operation_cancelled>,
              "the drop-in must throw the reference's cancellation type");
static_assert(std::is_same_v<levo::hip::cancellation_callback, levo::cancellation_callback>,
              "the drop-in must take the reference's callback type");

int main() {
    // What the wrappers execute when the callback reports a cancel ...
    levo::hip::cancellation_callback cancelled = [] { return true; };
    try {
        if (cancelled()) throw levo::hip::operation_cancelled();
        return 3;
    } catch (const levo::operation_cancelled & e) {   // ... as the reference's catch sites see it
        return std::strcmp(e.what(), "LeVo operation cancelled") == 0 ? 0 : 2;
    } catch (...) {
        return 1;
    }
}
"""


def _nm(obj):
    return subprocess.run(["nm", "-C", obj], capture_output=True, text=True, check=True).stdout


@needs_reference
def test_reference_catch_clause_catches_the_dropin_throw(tmp_path):
    src = tmp_path / "binding.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "binding"
    subprocess.run(["g++", *FLAGS, "-DLEVO_HIP_WITH_LEVO_H", "-I", REFERENCE_INCLUDE, str(src), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    assert subprocess.run([str(exe)]).returncode == 0


@needs_reference
@pytest.mark.parametrize("name", THROWING_SOURCES)
def test_dropin_objects_throw_the_reference_type(tmp_path, name):
    obj = tmp_path / (name + ".o")
    subprocess.run(["g++", *FLAGS, "-fPIC", "-DLEVO_HIP_WITH_LEVO_H", "-I", REFERENCE_INCLUDE, "-c",
                    os.path.join(HOST, name), "-o", str(obj)], check=True, capture_output=True, text=True)
    syms = _nm(str(obj))
    assert "typeinfo for levo::operation_cancelled" in syms
    assert "levo::hip::operation_cancelled" not in syms


@pytest.mark.parametrize("name", THROWING_SOURCES)
def test_standalone_build_keeps_its_own_type(tmp_path, name):
    obj = tmp_path / (name + ".o")
    subprocess.run(["g++", *FLAGS, "-fPIC", "-c", os.path.join(HOST, name), "-o", str(obj)],
                   check=True, capture_output=True, text=True)
    assert "typeinfo for levo::hip::operation_cancelled" in _nm(str(obj))
