"""The C-ABI library loads and exports every entry point include/levo_hip.h
declares; argument validation fails with the reference's messages. These
calls return before any device work, so they run without a GPU."""
from __future__ import annotations

import ctypes
import os
import subprocess

import pytest


def test_library_exports_every_declared_symbol(binding):
    lib = binding.LevoHip()
    declared = binding.declared_symbols()
    assert len(declared) >= 14
    out = subprocess.run(["nm", "-D", "--defined-only", binding.KERNEL_LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        assert hasattr(lib.lib, s)
    assert lib.lib.levo_hip_abi_version() == binding.header_abi_version()


def test_host_library_links_kernel_library(binding):
    assert os.path.exists(binding.HOST_LIB), "run __graft_entry__.build()"
    out = subprocess.run(["ldd", binding.HOST_LIB], capture_output=True, text=True, check=True).stdout
    assert "liblevo_hip.so" in out


# The C++17 drop-in surface: each entry mirrors a reference declaration
# (src/levo-sampling.h:13-64, src/levo-flow-renderer.h:44-51,
# src/levo-audio-ops.h:30-33, tools/levo-quantize.cpp:386-388).
HOST_API = [
    "levo::hip::apply_cfg(std::vector<float, std::allocator<float> > const&, std::vector<float, std::allocator<float> > const&, float)",
    "levo::hip::apply_unique_token_repetition_penalty(std::vector<float, std::allocator<float> >&, std::vector<long, std::allocator<long> > const&, float, unsigned long)",
    "levo::hip::Sampler::sample(std::vector<float, std::allocator<float> > const&, unsigned long, float, bool)",
    "levo::hip::Sampler::sample_streams(",
    "levo::hip::Sampler::sample_device(",
    "levo::hip::Sampler::restore(unsigned long, unsigned long)",
    "levo::hip::Sampler::uniform_bits()",
    "levo::hip::Sampler::uniform01()",
    "levo::hip::sample_top_k(",
    "levo::hip::flow::solve_flow_euler(",
    "levo::hip::flow::solve_flow_euler_device(",
    "levo::hip::detail::snake_beta(",
    "levo::hip::residual_rms_norm(",
    "levo::hip::residual_layer_norm(",
    "levo::hip::quantize_chunk(",
    "levo::hip::quantize_rows(",
    "levo::hip::padded_input_columns(",
    "levo::hip::row_size(",
    "levo::hip::dequantize_row(",
    "levo::hip::fp32_to_fp16_row(",
    "levo::hip::fp16_to_fp32_row(",
]


def test_host_library_exports_the_dropin_api(binding):
    out = subprocess.run(["nm", "-DC", "--defined-only", binding.HOST_LIB], capture_output=True, text=True,
                         check=True).stdout
    missing = [name for name in HOST_API if name not in out]
    assert not missing, missing


def test_validation_errors(binding):
    lib = binding.LevoHip()
    L = lib.lib
    st = L.levo_hip_snake_beta(None, 4, None, None, 0, None, 4, 2, 4, None)
    assert st == -1 and "SnakeBeta input is null" in lib.last_error()
    st = L.levo_hip_snake_beta(16, 4, 16, 16, 3, 16, 4, 2, 4, None)
    assert st == -1 and "must be F32 or F16" in lib.last_error()
    st = L.levo_hip_snake_beta(16, 2, 16, 16, 0, 16, 4, 2, 4, None)
    assert st == -1 and "stride" in lib.last_error()
    assert L.levo_hip_snake_beta(None, 0, None, None, 0, None, 0, 0, 0, None) == 0  # empty: no-op
    assert L.levo_hip_row_size(8, 1536) == 48 * 34
    assert L.levo_hip_row_size(2, 2208) == 69 * 18
    assert L.levo_hip_row_size(8, 100) == -1 and "multiple of 32" in lib.last_error()
    assert L.levo_hip_quantize_chunk(2, 16, 16, 0, 1, 32, 16, None) == -1
    assert "importance matrix" in lib.last_error()
    assert L.levo_hip_quantize_chunk(8, 16, 16, 5, 1, 32, None, None) == -1
    assert "row boundary" in lib.last_error()
    assert L.levo_hip_quantize_rows(8, 16, 1, 40, 40, 16, 1, 32, None) == -1
    assert "smaller than the source width" in lib.last_error()
    assert L.levo_hip_residual_rms_norm(1, 16, None, 16, 0, None, 16, 1, 2048, ctypes.c_float(1e-6), None) == -1
    assert "F16 weight" in lib.last_error()
    assert L.levo_hip_residual_layer_norm(0, 16, None, 16, None, 0, None, 16, 1, 9000, ctypes.c_float(1e-6),
                                          None) == -1
    assert "8192" in lib.last_error()
    assert L.levo_hip_flow_cfg_euler(None, None, None, 10, ctypes.c_float(1.5), ctypes.c_float(0.02), None) == -1
    assert "LeVo Flow renderer" in lib.last_error()


def test_sample_args_validation(binding):
    lib = binding.LevoHip()
    a = binding.SampleArgs()
    a.rows, a.vocab, a.row_pitch, a.n_streams, a.capacity = 1, 0, 0, 1, 4
    a.cond = 16
    assert lib.lib.levo_hip_cfg_sample(ctypes.byref(a), None) == -1
    assert "empty vocabulary" in lib.last_error()
    a.vocab, a.row_pitch = 8, 8
    a.best = a.count = a.cand_ids = 16
    a.recent, a.n_recent, a.repetition_penalty = 16, 3, 0.0
    assert lib.lib.levo_hip_cfg_sample(ctypes.byref(a), None) == -1
    assert "repetition penalty must be finite and positive" in lib.last_error()
    a.recent, a.n_recent = None, 0
    a.cand_probs, a.temperature = 16, float("inf")
    assert lib.lib.levo_hip_cfg_sample(ctypes.byref(a), None) == -1
    assert "temperature" in lib.last_error()
