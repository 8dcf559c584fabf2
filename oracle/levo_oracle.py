"""ctypes binding of oracle/liblevo_oracle.so and oracle/_ref/libref_levo.so.

TEST INFRASTRUCTURE ONLY: the checker the HIP kernels are compared against.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
Each wrapper names the reference function its C restatement follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liblevo_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref_levo.so")

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F = ctypes.c_float

TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q8_0 = 0, 1, 2, 8
TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_K = 12, 13, 14, 15
KQUANT_BLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210, TYPE_Q8_K: 292}
BLOCK_BYTES = {TYPE_Q8_0: 34, TYPE_Q4_0: 18}


def build(reference: str | None = None) -> None:
    """Compile the oracle (and the reference shim when the checkout exists)."""
    cmd = ["make", "-s", "-C", HERE]
    if reference:
        cmd.append(f"REF={reference}")
    subprocess.run(cmd, check=True)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(_P)


class MT19937_64(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64 * 312), ("index", ctypes.c_int)]


class BatchVector(ctypes.Structure):
    """lo_batch_vector: entry b is dynamic[b * stride + c] + learned[c]."""
    _fields_ = [("dynamic", _P), ("stride", _I64), ("learned", _P)]


class Oracle:
    """The C restatement (oracle/levo_oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        self.lib = lib
        sig = {
            "lo_fp32_to_fp16_row": (None, [_P, _P, _I64]),
            "lo_fp16_to_fp32_row": (None, [_P, _P, _I64]),
            "lo_snake_beta_f32": (None, [_P, _P, _P, _P, _I64, _I64, ctypes.c_int]),
            "lo_residual_rms_norm_f16": (None, [_P, _P, _P, _P, _P, _I64, _I64, _F, ctypes.c_int]),
            "lo_residual_rms_norm_f32": (None, [_P, _P, _P, _P, _P, _I64, _I64, _F, ctypes.c_int]),
            "lo_residual_layer_norm_f16": (None, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, ctypes.c_int]),
            "lo_residual_layer_norm_f32": (None, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F, ctypes.c_int]),
            "lo_residual_layer_norm_modulated_f32": (None, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                                             _I64, _F]),
            "lo_apply_cfg": (None, [_P, _P, _P, _I64, _F]),
            "lo_mt_seed": (None, [_P, ctypes.c_uint64]),
            "lo_mt_next": (ctypes.c_uint64, [_P]),
            "lo_mt_discard": (None, [_P, ctypes.c_uint64]),
            "lo_repetition_penalty": (ctypes.c_int, [_P, _I64, _P, _I64, _F, _I64]),
            "lo_top_k_candidates": (_I64, [_P, _I64, _I64, _P, _P, _I64]),
            "lo_sample_top_k": (ctypes.c_int, [_P, _I64, _I64, _F, ctypes.c_int, _P, _P, _P]),
            "lo_sample_streams": (ctypes.c_int, [_P, _I64, _I64, ctypes.c_int, _F, _I64, _I64, _F,
                                                 _P, _I64, _P, _I64, _P, _P, _P]),
            "lo_flow_incontext": (None, [_P, _P, _P, _I64, _F, _F]),
            "lo_flow_cfg_euler": (None, [_P, _P, _P, _I64, _F, _F]),
            "lo_quantize_chunk": (ctypes.c_size_t, [ctypes.c_int, _P, _P, _I64, _I64, _I64]),
            "lo_quantize_f16_rows_padded": (ctypes.c_size_t, [ctypes.c_int, _P, _I64, _I64, _I64, _P]),
            "lo_dequantize_row_q8_0": (None, [_P, _P, _I64]),
            "lo_mul_mat_q8_0": (None, [_P, _P, _P, _I64, _I64, _I64]),
            "lo_conv1d_f32": (None, [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, ctypes.c_int]),
            "lo_conv_transpose1d_f32": (None, [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _P]),
            "lo_dequantize_row_q4_0": (None, [_P, _P, _I64]),
            "lo_gaussian_noise": (None, [_P, _I64, ctypes.c_uint64]),
            "lo_quantize_row_q8_K": (None, [_P, _P, _I64]),
            "lo_dequantize_row_kquant": (None, [ctypes.c_int, _P, _P, _I64]),
            "lo_vec_dot_kquant_q8_K": (_F, [ctypes.c_int, _P, _P, _I64]),
            "lo_mul_mat_kquant": (None, [ctypes.c_int, _P, _P, _P, _I64, _I64, _I64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args

    # -- conversions (ggml_fp32_to_fp16_row / ggml_fp16_to_fp32_row) --------
    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(x.shape, dtype=np.uint16)
        self.lib.lo_fp32_to_fp16_row(_ptr(x), _ptr(y), x.size)
        return y

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        y = np.empty(h.shape, dtype=np.float32)
        self.lib.lo_fp16_to_fp32_row(_ptr(h), _ptr(y), h.size)
        return y

    # -- seeded inputs (src/levo-render.cpp:87-112) ---------------------------
    def gaussian(self, count: int, seed: int) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self.lib.lo_gaussian_noise(_ptr(out), count, seed)
        return out

    # -- SnakeBeta (src/levo-audio-ops.cpp:125-152) ---------------------------
    def snake_beta(self, x: np.ndarray, alpha_log: np.ndarray, beta_log: np.ndarray,
                   threads: int = 1) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        C, T = x.shape
        a = np.ascontiguousarray(alpha_log, dtype=np.float32).reshape(C)
        b = np.ascontiguousarray(beta_log, dtype=np.float32).reshape(C)
        y = np.empty_like(x)
        self.lib.lo_snake_beta_f32(_ptr(x), _ptr(a), _ptr(b), _ptr(y), C, T, threads)
        return y

    # -- norms (src/levo-kv.cpp:153-160, src/levo-lm.cpp:131-137,
    #           src/levo-flow-estimator.cpp:106-109) --------------------------
    def rms_norm(self, x, delta, weight, eps, threads=1):
        dt = x.dtype
        rows, dim = x.shape
        h = np.empty_like(x)
        y = np.empty_like(x)
        fn = self.lib.lo_residual_rms_norm_f16 if dt == np.uint16 else self.lib.lo_residual_rms_norm_f32
        fn(_ptr(x), _ptr(delta), _ptr(weight), _ptr(h), _ptr(y), rows, dim, eps, threads)
        return h, y

    def layer_norm(self, x, delta, gamma, beta, eps, threads=1):
        dt = x.dtype
        rows, dim = x.shape
        h = np.empty_like(x)
        y = np.empty_like(x)
        fn = self.lib.lo_residual_layer_norm_f16 if dt == np.uint16 else self.lib.lo_residual_layer_norm_f32
        fn(_ptr(x), _ptr(delta), _ptr(gamma), _ptr(beta), _ptr(h), _ptr(y), rows, dim, eps, threads)
        return h, y

    def layer_norm_modulated(self, x, delta, gate, gamma, beta, scale, shift, rows_per_batch, eps):
        """lo_residual_layer_norm_modulated_f32 (src/levo-flow-estimator.cpp:
        89-109, 221-261). gate / scale / shift: None or (dynamic, learned)
        with dynamic [batches][stride >= dim] and learned [dim] or None."""
        x = np.ascontiguousarray(x, np.float32)
        rows, dim = x.shape
        keep = []

        def vec(v):
            if v is None:
                return None
            dyn, learned = v
            dyn = np.ascontiguousarray(dyn, np.float32)
            learned = None if learned is None else np.ascontiguousarray(learned, np.float32)
            keep.extend([dyn, learned])
            return ctypes.byref(BatchVector(dyn.ctypes.data, dyn.shape[-1], _ptr(learned)))

        delta = None if delta is None else np.ascontiguousarray(delta, np.float32)
        gamma = np.ascontiguousarray(gamma, np.float32)
        beta = np.ascontiguousarray(beta, np.float32)
        h = np.empty_like(x)
        y = np.empty_like(x)
        self.lib.lo_residual_layer_norm_modulated_f32(_ptr(x), _ptr(delta), vec(gate), _ptr(gamma), _ptr(beta),
                                                      vec(scale), vec(shift), _ptr(h), _ptr(y), rows,
                                                      rows_per_batch, dim, eps)
        return h, y

    # -- CFG / sampling (src/levo-sampling.cpp) ------------------------------
    def apply_cfg(self, cond, uncond, scale):
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        uncond = np.ascontiguousarray(uncond, dtype=np.float32)
        out = np.empty_like(cond)
        self.lib.lo_apply_cfg(_ptr(cond), _ptr(uncond), _ptr(out), cond.size, scale)
        return out

    def mt(self, seed: int) -> MT19937_64:
        rng = MT19937_64()
        self.lib.lo_mt_seed(ctypes.byref(rng), seed)
        return rng

    def mt_next(self, rng: MT19937_64) -> int:
        return int(self.lib.lo_mt_next(ctypes.byref(rng)))

    def repetition_penalty(self, logits, recent, penalty, limit=0):
        logits = np.array(logits, dtype=np.float32)
        recent = np.ascontiguousarray(recent, dtype=np.int64)
        st = self.lib.lo_repetition_penalty(_ptr(logits), logits.size, _ptr(recent), recent.size, penalty, limit)
        if st != 0:
            raise ValueError("repetition penalty must be finite and positive")
        return logits

    def top_k_candidates(self, logits, top_k):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        cand = np.empty(max(logits.size, 1), dtype=np.int64)
        best = ctypes.c_int64(-1)
        n = self.lib.lo_top_k_candidates(_ptr(logits), logits.size, top_k, ctypes.byref(best), _ptr(cand), cand.size)
        if n < 0:
            raise ValueError("logits contain NaN" if n == -3 else "cannot sample an empty vocabulary")
        return int(best.value), cand[:n].copy()

    def sample_top_k(self, logits, top_k, temperature, use_sampling, rng, draws=None):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        tok = ctypes.c_int64(-1)
        d = ctypes.c_uint64(0 if draws is None else draws)
        st = self.lib.lo_sample_top_k(_ptr(logits), logits.size, top_k, temperature, int(use_sampling),
                                      ctypes.byref(rng), ctypes.byref(d), ctypes.byref(tok))
        if st != 0:
            raise ValueError(f"sample_top_k failed with status {st}")
        return int(tok.value), int(d.value)

    def sample_streams(self, logits, *, use_sampling, temperature, top_k_mixed, top_k_detail,
                       repetition_penalty=1.1, recent=None, ignore=(), rng, draws=0):
        logits = np.ascontiguousarray(logits, dtype=np.float32)
        n_streams, vocab = logits.shape
        rec = None if recent is None else np.ascontiguousarray(recent, dtype=np.int64)
        ign = np.ascontiguousarray(np.asarray(ignore, dtype=np.int64))
        toks = np.empty(n_streams, dtype=np.int64)
        d = ctypes.c_uint64(draws)
        st = self.lib.lo_sample_streams(_ptr(logits), n_streams, vocab, int(use_sampling), temperature,
                                        top_k_mixed, top_k_detail, repetition_penalty,
                                        _ptr(rec), 0 if rec is None else rec.shape[1],
                                        _ptr(ign) if ign.size else None, ign.size,
                                        ctypes.byref(rng), ctypes.byref(d), _ptr(toks))
        if st != 0:
            raise ValueError(f"sample_streams failed with status {st}")
        return toks, int(d.value)

    # -- Flow Euler (src/levo-flow-renderer.cpp:91-117) -------------------------
    def flow_incontext(self, state, noise, context, n_prefix, time, sigma_min):
        self.lib.lo_flow_incontext(_ptr(state), _ptr(noise), _ptr(context), n_prefix, time, sigma_min)

    def flow_cfg_euler(self, state, v_uncond, v_cond, guidance, dt):
        self.lib.lo_flow_cfg_euler(_ptr(state), _ptr(v_uncond), _ptr(v_cond), state.size, guidance, dt)

    # -- quantization (ggml_quantize_chunk at tools/levo-quantize.cpp:386) --------
    @staticmethod
    def row_bytes(qtype, cols):
        """ggml_row_size for the block formats."""
        if qtype in KQUANT_BLOCK_BYTES:
            return (cols // 256) * KQUANT_BLOCK_BYTES[qtype]
        return (cols // 32) * BLOCK_BYTES[qtype]

    def quantize(self, qtype, x_f32: np.ndarray) -> np.ndarray:
        """ggml_quantize_chunk(type, x, ..., NULL): Q8_0, Q4_0 and the Q4_K /
        Q5_K / Q6_K reference quantizers."""
        x = np.ascontiguousarray(x_f32, dtype=np.float32)
        rows, cols = x.shape
        out = np.empty(rows * self.row_bytes(qtype, cols), dtype=np.uint8)
        n = self.lib.lo_quantize_chunk(qtype, _ptr(x), _ptr(out), 0, rows, cols)
        assert n == out.size
        return out

    def quantize_f16_padded(self, qtype, x_f16: np.ndarray, dst_cols: int) -> np.ndarray:
        x = np.ascontiguousarray(x_f16, dtype=np.uint16)
        rows, cols = x.shape
        out = np.empty(rows * self.row_bytes(qtype, dst_cols), dtype=np.uint8)
        n = self.lib.lo_quantize_f16_rows_padded(qtype, _ptr(x), rows, cols, dst_cols, _ptr(out))
        assert n == out.size
        return out

    def conv1d(self, x, w, bias, padding, dilation, threads=1):
        """conv_1d_f32 (stride 1): x [c_in][t_in], w [c_out][c_in][kernel] -> [c_out][t_out]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        c_in, t_in = x.shape
        c_out, _, kernel = w.shape
        t_out = t_in + 2 * padding - dilation * (kernel - 1)
        y = np.empty((c_out, t_out), dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self.lib.lo_conv1d_f32(_ptr(x), c_in, t_in, _ptr(w), c_out, kernel, _ptr(b), padding, dilation, _ptr(y),
                               threads)
        return y

    def conv_transpose1d(self, x, w, bias, stride, padding):
        """conv_transpose_1d_f32: x [c_in][t_in], w [c_in][c_out][kernel] -> [c_out][t_out]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        c_in, t_in = x.shape
        _, c_out, kernel = w.shape
        t_out = (t_in - 1) * stride + kernel - 2 * padding
        y = np.empty((c_out, t_out), dtype=np.float32)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self.lib.lo_conv_transpose1d_f32(_ptr(x), c_in, t_in, _ptr(w), c_out, kernel, stride, padding, _ptr(b),
                                         _ptr(y))
        return y

    def mul_mat_q8_0(self, w_blocks: np.ndarray, x: np.ndarray, rows: int, k: int) -> np.ndarray:
        """ggml CPU mul_mat of Q8_0 rows [rows][k/32] by x [n_vec][k] -> [n_vec][rows]."""
        w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
        y = np.empty((x.shape[0], rows), dtype=np.float32)
        self.lib.lo_mul_mat_q8_0(_ptr(w_blocks), _ptr(x), _ptr(y), rows, k, x.shape[0])
        return y

    def quantize_q8_K(self, x: np.ndarray) -> np.ndarray:
        """quantize_row_q8_K_ref over x (a multiple of 256 values) -> 292-byte blocks."""
        x = np.ascontiguousarray(x, dtype=np.float32).ravel()
        out = np.empty(x.size // 256 * 292, dtype=np.uint8)
        self.lib.lo_quantize_row_q8_K(_ptr(x), _ptr(out), x.size)
        return out

    def dequantize_kquant(self, qtype, blocks: np.ndarray, count: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        y = np.empty(count, dtype=np.float32)
        self.lib.lo_dequantize_row_kquant(qtype, _ptr(blocks), _ptr(y), count)
        return y

    def vec_dot_kquant(self, qtype, w_blocks: np.ndarray, x_blocks: np.ndarray, k: int) -> float:
        w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
        x_blocks = np.ascontiguousarray(x_blocks, dtype=np.uint8)
        return float(self.lib.lo_vec_dot_kquant_q8_K(qtype, _ptr(w_blocks), _ptr(x_blocks), k))

    def mul_mat_kquant(self, qtype, w_blocks: np.ndarray, x: np.ndarray, rows: int, k: int) -> np.ndarray:
        """ggml CPU mul_mat of K-quant rows [rows][k/256] by x [n_vec][k] -> [n_vec][rows]."""
        w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
        y = np.empty((x.shape[0], rows), dtype=np.float32)
        self.lib.lo_mul_mat_kquant(qtype, _ptr(w_blocks), _ptr(x), _ptr(y), rows, k, x.shape[0])
        return y

    def dequantize(self, qtype, blocks: np.ndarray, count: int) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
        y = np.empty(count, dtype=np.float32)
        fn = self.lib.lo_dequantize_row_q8_0 if qtype == TYPE_Q8_0 else self.lib.lo_dequantize_row_q4_0
        fn(_ptr(blocks), _ptr(y), count)
        return y


class Reference:
    """The reference's own sampling/renderer-pattern sources (oracle/_ref)."""

    def __init__(self, path: str = REF_SO):
        lib = ctypes.CDLL(path)
        self.lib = lib
        sig = {
            "ref_last_error": (ctypes.c_char_p, []),
            "ref_apply_cfg": (ctypes.c_int, [_P, _P, _I64, _F, _P]),
            "ref_combine_renderer_cfg": (ctypes.c_int, [_P, _P, _I64, _F, _P]),
            "ref_euler_schedule": (ctypes.c_int, [_I64, _P, _P]),
            "ref_repetition_penalty": (ctypes.c_int, [_P, _I64, _P, _I64, _F, _I64]),
            "ref_mt19937_64_after": (ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_uint64]),
            "ref_sampler_new": (_P, [ctypes.c_uint64]),
            "ref_sampler_free": (None, [_P]),
            "ref_sampler_draw_count": (ctypes.c_uint64, [_P]),
            "ref_sampler_restore": (None, [_P, ctypes.c_uint64, ctypes.c_uint64]),
            "ref_sampler_sample": (ctypes.c_int, [_P, _P, _I64, _I64, _F, ctypes.c_int, _P]),
            "ref_sampler_sample_streams": (ctypes.c_int, [_P, _P, _I64, _I64, ctypes.c_int, _F, _I64, _I64,
                                                          _I64, _F, _P, _I64, _P, _I64, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args

    def _check(self, st):
        if st != 0:
            raise ValueError(self.lib.ref_last_error().decode())

    def apply_cfg(self, cond, uncond, scale):
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        uncond = np.ascontiguousarray(uncond, dtype=np.float32)
        out = np.empty_like(cond)
        self._check(self.lib.ref_apply_cfg(_ptr(cond), _ptr(uncond), cond.size, scale, _ptr(out)))
        return out

    def combine_renderer_cfg(self, uncond, cond, g):
        uncond = np.ascontiguousarray(uncond, dtype=np.float32)
        cond = np.ascontiguousarray(cond, dtype=np.float32)
        out = np.empty_like(cond)
        self._check(self.lib.ref_combine_renderer_cfg(_ptr(uncond), _ptr(cond), cond.size, g, _ptr(out)))
        return out

    def euler_schedule(self, steps):
        times = np.empty(steps + 1, dtype=np.float32)
        dt = ctypes.c_float()
        self._check(self.lib.ref_euler_schedule(steps, _ptr(times), ctypes.byref(dt)))
        return times, dt.value

    def repetition_penalty(self, logits, recent, penalty, limit=0):
        logits = np.array(logits, dtype=np.float32)
        recent = np.ascontiguousarray(recent, dtype=np.int64)
        self._check(self.lib.ref_repetition_penalty(_ptr(logits), logits.size, _ptr(recent), recent.size,
                                                     penalty, limit))
        return logits

    def mt_after(self, seed, discard):
        return int(self.lib.ref_mt19937_64_after(seed, discard))

    class Sampler:
        def __init__(self, ref: "Reference", seed: int):
            self.ref = ref
            self.h = ref.lib.ref_sampler_new(seed)

        def __del__(self):
            if getattr(self, "h", None):
                self.ref.lib.ref_sampler_free(self.h)
                self.h = None

        @property
        def draw_count(self):
            return int(self.ref.lib.ref_sampler_draw_count(self.h))

        def restore(self, seed, draws):
            self.ref.lib.ref_sampler_restore(self.h, seed, draws)

        def sample(self, logits, top_k, temperature, use_sampling):
            logits = np.ascontiguousarray(logits, dtype=np.float32)
            tok = ctypes.c_int64()
            self.ref._check(self.ref.lib.ref_sampler_sample(self.h, _ptr(logits), logits.size, top_k,
                                                            temperature, int(use_sampling), ctypes.byref(tok)))
            return int(tok.value)

        def sample_streams(self, logits, *, use_sampling, temperature, top_k_mixed, top_k_detail,
                           repetition_window=50, repetition_penalty=1.1, recent=None, ignore=()):
            logits = np.ascontiguousarray(logits, dtype=np.float32)
            n_streams, vocab = logits.shape
            rec = None if recent is None else np.ascontiguousarray(recent, dtype=np.int64)
            ign = np.ascontiguousarray(np.asarray(ignore, dtype=np.int64))
            toks = np.empty(n_streams, dtype=np.int64)
            self.ref._check(self.ref.lib.ref_sampler_sample_streams(
                self.h, _ptr(logits), n_streams, vocab, int(use_sampling), temperature, top_k_mixed,
                top_k_detail, repetition_window, repetition_penalty, _ptr(rec),
                0 if rec is None else rec.shape[1], _ptr(ign) if ign.size else None, ign.size, _ptr(toks)))
            return toks

    def sampler(self, seed: int) -> "Reference.Sampler":
        return Reference.Sampler(self, seed)


def have_reference() -> bool:
    return os.path.exists(REF_SO)
