"""ctypes binding of levo2.cpp_amd/liblevo_hip.so (the C ABI in include/levo_hip.h).

Plumbing for tests and bench.py: arguments are torch device tensors (or raw
device addresses) and a HIP stream; every call goes straight to the gfx950
kernels. There is no CPU fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
KERNEL_LIB = os.path.join(PKG, "liblevo_hip.so")
HOST_LIB = os.path.join(PKG, "liblevo_hip_host.so")
HEADER = os.path.join(ROOT, "include", "levo_hip.h")

F32, F16, Q4_0, Q8_0 = 0, 1, 2, 8
MAX_STREAMS = 8
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_F = ctypes.c_float


class LevoHipError(RuntimeError):
    pass


class SampleArgs(ctypes.Structure):
    """levo_hip_sample_args (include/levo_hip.h)."""

    _fields_ = [
        ("cond", _P), ("uncond", _P), ("rows", _I64), ("vocab", _I64), ("row_pitch", _I64),
        ("cfg_scale", _F), ("temperature", _F), ("n_streams", _I32), ("top_k", _I32 * MAX_STREAMS),
        ("recent", _P), ("n_recent", _I32), ("repetition_penalty", _F), ("penalty_limit", _I64),
        ("ignore", _P), ("n_ignore", _I32),
        ("best", _P), ("count", _P), ("cand_ids", _P), ("cand_logits", _P), ("cand_probs", _P),
        ("row_max", _P), ("row_lse", _P), ("capacity", _I32),
    ]


class DrawArgs(ctypes.Structure):
    """levo_hip_draw_args (include/levo_hip.h)."""

    _fields_ = [
        ("best", _P), ("count", _P), ("cand_ids", _P), ("cand_logits", _P), ("row_max", _P),
        ("rows", _I64), ("capacity", _I32), ("temperature", _F), ("use_sampling", _I32),
        ("bits", _P), ("tokens", _P), ("draws", _P),
    ]


TOKEN_NAN, TOKEN_OVERFLOW, TOKEN_RECHECK = -1, -2, -3


class MatQ8_0(ctypes.Structure):
    """levo_hip_mat_q8_0 (include/levo_hip.h)."""

    _fields_ = [("weight", _P), ("y", _P), ("y_pitch", _I64), ("rows", _I64)]


class MatKquant(ctypes.Structure):
    """levo_hip_mat_kquant (include/levo_hip.h)."""

    _fields_ = [("type", ctypes.c_int), ("weight", _P), ("y", _P), ("y_pitch", _I64), ("rows", _I64)]


class FlowInputArgs(ctypes.Structure):
    """levo_hip_flow_input_args (include/levo_hip.h)."""

    _fields_ = [
        ("model_input", _P), ("batch", _I32), ("frames", _I64), ("mask_embedding", _P), ("mask_dim", _I64),
        ("context", _P), ("latent", _I64), ("conditioning", _P), ("condition_width", _I64),
        ("state", _P), ("noise", _P), ("prefix_frames", _I64), ("step", _I64), ("steps", _I64),
        ("sigma_min", _F),
    ]


class FlowStepArgs(ctypes.Structure):
    """levo_hip_flow_step_args (include/levo_hip.h)."""

    _fields_ = [
        ("state", _P), ("output", _P), ("out_pitch", _I64), ("vel_col", _I64), ("batch", _I32),
        ("guidance", _F), ("frames", _I64), ("latent", _I64), ("step", _I64), ("steps", _I64),
        ("noise", _P), ("context", _P), ("prefix_frames", _I64), ("sigma_min", _F),
        ("next_input", _P), ("in_pitch", _I64), ("state_col", _I64),
        ("mean", _P), ("stddev", _P), ("denormalized", _P), ("nonfinite", _P),
    ]


class BatchVector(ctypes.Structure):
    """levo_hip_batch_vector (include/levo_hip.h)."""

    _fields_ = [("dynamic", _P), ("stride", _I64), ("learned", _P)]


class ModulatedNormArgs(ctypes.Structure):
    """levo_hip_modulated_norm_args (include/levo_hip.h)."""

    _fields_ = [
        ("x", _P), ("delta", _P), ("gate", BatchVector), ("gamma", _P), ("beta", _P), ("param_type", ctypes.c_int),
        ("scale", BatchVector), ("shift", BatchVector), ("h_out", _P), ("y", _P), ("rows", _I64),
        ("rows_per_batch", _I64), ("dim", _I64), ("eps", _F),
    ]


class SnakeJob(ctypes.Structure):
    """levo_hip_snake_job (include/levo_hip.h)."""

    _fields_ = [("x", _P), ("x_stride", _I64), ("alpha_log", _P), ("beta_log", _P), ("param_type", ctypes.c_int),
                ("y", _P), ("y_stride", _I64), ("channels", _I64), ("time", _I64)]


class VaeSnake(ctypes.Structure):
    _fields_ = [("alpha_log", _P), ("beta_log", _P)]


class VaeConv(ctypes.Structure):
    _fields_ = [("weight", _P), ("bias", _P)]


class VaeResidual(ctypes.Structure):
    _fields_ = [("pre", VaeSnake), ("conv_0", VaeConv), ("post", VaeSnake), ("conv_1", VaeConv)]


class VaeStage(ctypes.Structure):
    _fields_ = [("activation", VaeSnake), ("upsample", VaeConv), ("residual", VaeResidual * 3)]


class VaeDecoderWeights(ctypes.Structure):
    """levo_hip_vae_decoder_weights (include/levo_hip.h)."""

    _fields_ = [("input", VaeConv), ("stage", VaeStage * 5), ("output_activation", VaeSnake),
                ("output_weight", _P), ("param_type", ctypes.c_int)]


VAE_STRIDES = (10, 6, 4, 4, 2)
VAE_IN_WIDTH = (2048, 1024, 512, 256, 128)
VAE_OUT_WIDTH = (1024, 512, 256, 128, 128)
VAE_DILATIONS = (1, 3, 9)


def header_abi_version(header: str = HEADER) -> int:
    """LEVO_HIP_ABI_VERSION as declared in include/levo_hip.h."""
    m = re.search(r"#define\s+LEVO_HIP_ABI_VERSION\s+(\d+)", open(header).read())
    return int(m.group(1))


def declared_symbols(header: str = HEADER) -> list[str]:
    """Every function name declared in include/levo_hip.h."""
    text = open(header).read()
    return sorted(set(re.findall(r"\b(levo_hip_[a-z0-9_]+)\s*\(", text)))


def _addr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class LevoHip:
    """The C ABI with status checking."""

    def __init__(self, path: str = KERNEL_LIB):
        if not os.path.exists(path):
            raise LevoHipError(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(path)
        self.lib = lib
        sig = {
            "levo_hip_last_error": (ctypes.c_char_p, []),
            "levo_hip_abi_version": (ctypes.c_int, []),
            "levo_hip_snake_beta": (ctypes.c_int, [_P, _I64, _P, _P, ctypes.c_int, _P, _I64, _I64, _I64, _P]),
            "levo_hip_snake_beta_batch": (ctypes.c_int, [ctypes.POINTER(SnakeJob), ctypes.c_int, _P]),
            "levo_hip_snake_conv1d": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P, _I64, _I64, _P,
                                                     _I64, _I64, _P, _I64, _P, _I64, _P]),
            "levo_hip_snake_conv1d_split_workspace_floats": (_I64, [_I64, _I64]),
            "levo_hip_snake_conv1d_split": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P, _I64, _I64,
                                                           _P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P]),
            "levo_hip_conv_transpose1d_pack_weights": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _P]),
            "levo_hip_snake_conv_transpose1d": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P, _I64,
                                                               _I64, _P, _I64, _P, _I64, _P]),
            "levo_hip_snake_conv_transpose1d_split_workspace_floats": (_I64, [_I64, _I64, _I64]),
            "levo_hip_snake_conv_transpose1d_split": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _P, ctypes.c_int, _P,
                                                                     _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P]),
            "levo_hip_vae_decode_workspace_bytes": (_I64, [_I64]),
            "levo_hip_vae_validate_weights": (ctypes.c_int, [ctypes.POINTER(VaeDecoderWeights)]),
            "levo_hip_vae_decode": (ctypes.c_int, [ctypes.POINTER(VaeDecoderWeights), _P, _I64, _P, _P, _P, _I64,
                                                    _P]),
            "levo_hip_vae_residual_unit": (ctypes.c_int, [_P, _I64, _I64, ctypes.POINTER(VaeResidual), _I64,
                                                          ctypes.c_int, _P, _P, _P]),
            "levo_hip_residual_rms_norm": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, ctypes.c_int, _P, _P,
                                                          _I64, _I64, _F, _P]),
            "levo_hip_residual_layer_norm": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _P, ctypes.c_int, _P, _P,
                                                            _I64, _I64, _F, _P]),
            "levo_hip_residual_layer_norm_modulated": (ctypes.c_int, [ctypes.POINTER(ModulatedNormArgs), _P]),
            "levo_hip_cfg_combine": (ctypes.c_int, [_P, _P, _P, _I64, _F, _P]),
            "levo_hip_cfg_sample": (ctypes.c_int, [ctypes.POINTER(SampleArgs), _P]),
            "levo_hip_sample_draw": (ctypes.c_int, [ctypes.POINTER(DrawArgs), _P]),
            "levo_hip_sample_step_workspace_bytes": (_I64, [_I64, _I64]),
            "levo_hip_sample_step": (ctypes.c_int, [ctypes.POINTER(SampleArgs), ctypes.POINTER(DrawArgs), _P, _I64,
                                                    _P]),
            "levo_hip_sample_step_static": (ctypes.c_int, [ctypes.POINTER(SampleArgs), ctypes.POINTER(DrawArgs), _P]),
            "levo_hip_flow_cfg_euler": (ctypes.c_int, [_P, _P, _P, _I64, _F, _F, _P]),
            "levo_hip_flow_cfg_euler_checked": (ctypes.c_int, [_P, _P, _P, _I64, _F, _F, _P, _P]),
            "levo_hip_check_finite": (ctypes.c_int, [_P, _I64, _P, ctypes.c_int32, _P]),
            "levo_hip_repetition_penalty": (ctypes.c_int, [_P, _I64, _P, ctypes.c_int32, _F, _I64, _P]),
            "levo_hip_flow_incontext": (ctypes.c_int, [_P, _P, _P, _I64, _F, _F, _P]),
            "levo_hip_flow_assemble_input": (ctypes.c_int, [ctypes.POINTER(FlowInputArgs), _P]),
            "levo_hip_flow_step": (ctypes.c_int, [ctypes.POINTER(FlowStepArgs), _P]),
            "levo_hip_flow_normalize": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _P, _P]),
            "levo_hip_flow_denormalize": (ctypes.c_int, [_P, _P, _P, _P, _I64, _I64, _P, _P]),
            "levo_hip_mul_mat_q8_0": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
            "levo_hip_mul_mat_q8_0_multi": (ctypes.c_int, [_P, _I32, _P, _P, _I64, _I64, _I64, _P]),
            "levo_hip_repack_q8_0": (ctypes.c_int, [_P, _P, _I64, _I64, _P]),
            "levo_hip_quantize_q8_0_columns": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _P]),
            "levo_hip_mul_mat_q8_0_packed": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _I64, _P]),
            "levo_hip_mul_mat_q8_0_packed_multi": (ctypes.c_int, [_P, _I32, _P, _P, _I64, _I64, _I64, _P]),
            "levo_hip_quantize_q8_K": (ctypes.c_int, [_P, _P, _I64, _P]),
            "levo_hip_mul_mat_kquant": (ctypes.c_int, [ctypes.c_int, _P, _P, _P, _I64, _I64, _I64, _I64, _P]),
            "levo_hip_mul_mat_kquant_multi": (ctypes.c_int, [_P, _I32, _P, _P, _I64, _I64, _I64, _P]),
            "levo_hip_row_size": (_I64, [ctypes.c_int, _I64]),
            "levo_hip_quantize_chunk": (_I64, [ctypes.c_int, _P, _P, _I64, _I64, _I64, _P, _P]),
            "levo_hip_quantize_rows": (_I64, [ctypes.c_int, _P, ctypes.c_int, _I64, _I64, _P, _I64, _I64, _P]),
            "levo_hip_dequantize": (ctypes.c_int, [ctypes.c_int, _P, _P, ctypes.c_int, _I64, _P]),
            "levo_hip_fp32_to_fp16_row": (ctypes.c_int, [_P, _P, _I64, _P]),
            "levo_hip_fp16_to_fp32_row": (ctypes.c_int, [_P, _P, _I64, _P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args

    def last_error(self) -> str:
        return self.lib.levo_hip_last_error().decode()

    def _check(self, status: int) -> int:
        if status < 0:
            raise LevoHipError(f"status {status}: {self.last_error()}")
        return status

    # ---- ops ---------------------------------------------------------------------
    def snake_beta(self, x, alpha_log, beta_log, y, *, param_type=F32, channels=None, time=None,
                   x_stride=None, y_stride=None, stream=None):
        C = channels if channels is not None else x.shape[0]
        T = time if time is not None else x.shape[1]
        xs = x_stride if x_stride is not None else (x.stride(0) if hasattr(x, "stride") else T)
        ys = y_stride if y_stride is not None else (y.stride(0) if hasattr(y, "stride") else T)
        return self._check(self.lib.levo_hip_snake_beta(_addr(x), xs, _addr(alpha_log), _addr(beta_log), param_type,
                                                        _addr(y), ys, C, T, _stream(stream)))

    def snake_beta_batch(self, jobs, stream=None):
        """jobs: (x, alpha_log, beta_log, y) tuples of [C][T] tensors, or (.., param_type)."""
        arr = (SnakeJob * max(len(jobs), 1))()
        for i, job in enumerate(jobs):
            x, a, b, y = job[:4]
            pt = job[4] if len(job) > 4 else F32
            arr[i] = SnakeJob(_addr(x), x.stride(0), _addr(a), _addr(b), pt, _addr(y), y.stride(0), x.shape[0],
                              x.shape[1])
        return self._check(self.lib.levo_hip_snake_beta_batch(arr, len(jobs), _stream(stream)))

    def snake_conv1d(self, x, c_in, t_in, weight, c_out, kernel, *, alpha_log=None, beta_log=None, param_type=F32,
                     bias=None, padding=0, dilation=1, residual=None, y=None, x_stride=None, residual_stride=None,
                     y_stride=None, stream=None):
        t_out = t_in + 2 * padding - dilation * (kernel - 1)
        return self._check(self.lib.levo_hip_snake_conv1d(
            _addr(x), x_stride or t_in, c_in, t_in, _addr(alpha_log), _addr(beta_log), param_type,
            _addr(weight), c_out, kernel, _addr(bias), padding, dilation, _addr(residual),
            residual_stride or t_out, _addr(y), y_stride or t_out, _stream(stream)))

    def snake_conv1d_split_workspace_floats(self, c_out, t_out) -> int:
        return int(self.lib.levo_hip_snake_conv1d_split_workspace_floats(c_out, t_out))

    def snake_conv1d_split(self, x, c_in, t_in, weight, c_out, kernel, *, workspace, workspace_floats,
                           alpha_log=None, beta_log=None, param_type=F32, bias=None, padding=0, dilation=1,
                           residual=None, y=None, x_stride=None, residual_stride=None, y_stride=None, stream=None):
        """snake_conv1d with a workspace: split K over several workgroups per tile when the grid is small."""
        t_out = t_in + 2 * padding - dilation * (kernel - 1)
        return self._check(self.lib.levo_hip_snake_conv1d_split(
            _addr(x), x_stride or t_in, c_in, t_in, _addr(alpha_log), _addr(beta_log), param_type,
            _addr(weight), c_out, kernel, _addr(bias), padding, dilation, _addr(residual),
            residual_stride or t_out, _addr(y), y_stride or t_out, _addr(workspace), workspace_floats,
            _stream(stream)))

    def conv_transpose1d_pack_weights(self, weight, packed, c_in, c_out, stride, stream=None):
        return self._check(self.lib.levo_hip_conv_transpose1d_pack_weights(_addr(weight), _addr(packed), c_in, c_out,
                                                                           stride, _stream(stream)))

    def snake_conv_transpose1d(self, x, c_in, t_in, packed_weight, c_out, stride, *, alpha_log=None, beta_log=None,
                               param_type=F32, bias=None, padding=0, y=None, x_stride=None, y_stride=None,
                               stream=None):
        t_out = (t_in + 1) * stride - 2 * padding
        return self._check(self.lib.levo_hip_snake_conv_transpose1d(
            _addr(x), x_stride or t_in, c_in, t_in, _addr(alpha_log), _addr(beta_log), param_type,
            _addr(packed_weight), c_out, stride, _addr(bias), padding, _addr(y), y_stride or t_out,
            _stream(stream)))

    def snake_conv_transpose1d_split_workspace_floats(self, c_out, t_in, stride) -> int:
        return int(self.lib.levo_hip_snake_conv_transpose1d_split_workspace_floats(c_out, t_in, stride))

    def snake_conv_transpose1d_split(self, x, c_in, t_in, packed_weight, c_out, stride, *, workspace,
                                     workspace_floats, alpha_log=None, beta_log=None, param_type=F32, bias=None,
                                     padding=0, y=None, x_stride=None, y_stride=None, stream=None):
        """snake_conv_transpose1d with a workspace: split K when the grid is small."""
        t_out = (t_in + 1) * stride - 2 * padding
        return self._check(self.lib.levo_hip_snake_conv_transpose1d_split(
            _addr(x), x_stride or t_in, c_in, t_in, _addr(alpha_log), _addr(beta_log), param_type,
            _addr(packed_weight), c_out, stride, _addr(bias), padding, _addr(y), y_stride or t_out,
            _addr(workspace), workspace_floats, _stream(stream)))

    def vae_validate_weights(self, weights: VaeDecoderWeights):
        return self._check(self.lib.levo_hip_vae_validate_weights(ctypes.byref(weights)))

    def vae_decode_workspace_bytes(self, frames):
        return int(self.lib.levo_hip_vae_decode_workspace_bytes(frames))

    def vae_decode(self, weights: VaeDecoderWeights, latent, frames, audio, workspace, workspace_bytes, *,
                   stage_outputs=None, stream=None):
        """stage_outputs: None or 5 device tensors (or None) receiving each stage's output."""
        stages = None
        if stage_outputs is not None:
            if len(stage_outputs) != 5:
                raise ValueError("stage_outputs holds one tensor (or None) per stage")
            stages = (ctypes.c_void_p * 5)(*[_addr(t) for t in stage_outputs])
        return self._check(self.lib.levo_hip_vae_decode(ctypes.byref(weights), _addr(latent), frames, _addr(audio),
                                                        stages, _addr(workspace), workspace_bytes, _stream(stream)))

    def vae_residual_unit(self, x, channels, time, unit: VaeResidual, dilation, y, h, *, param_type=F32,
                          stream=None):
        """One residual unit (run_residual): y = x + conv_1(snake(conv_0(snake(x)))); h: conv_0's output
        unless the unit runs as one launch."""
        return self._check(self.lib.levo_hip_vae_residual_unit(_addr(x), channels, time, ctypes.byref(unit), dilation,
                                                               param_type, _addr(y), _addr(h), _stream(stream)))

    def rms_norm(self, act_type, x, delta, weight, weight_type, h_out, y, rows, dim, eps, stream=None):
        return self._check(self.lib.levo_hip_residual_rms_norm(act_type, _addr(x), _addr(delta), _addr(weight),
                                                               weight_type, _addr(h_out), _addr(y), rows, dim,
                                                               eps, _stream(stream)))

    def layer_norm(self, act_type, x, delta, gamma, beta, param_type, h_out, y, rows, dim, eps, stream=None):
        return self._check(self.lib.levo_hip_residual_layer_norm(act_type, _addr(x), _addr(delta), _addr(gamma),
                                                                 _addr(beta), param_type, _addr(h_out), _addr(y),
                                                                 rows, dim, eps, _stream(stream)))

    def layer_norm_modulated(self, args: ModulatedNormArgs, stream=None):
        return self._check(self.lib.levo_hip_residual_layer_norm_modulated(ctypes.byref(args), _stream(stream)))

    def cfg_combine(self, out, uncond, cond, n, scale, stream=None):
        return self._check(self.lib.levo_hip_cfg_combine(_addr(out), _addr(uncond), _addr(cond), n, scale,
                                                         _stream(stream)))

    def cfg_sample(self, args: SampleArgs, stream=None):
        return self._check(self.lib.levo_hip_cfg_sample(ctypes.byref(args), _stream(stream)))

    def sample_draw(self, args: DrawArgs, stream=None):
        return self._check(self.lib.levo_hip_sample_draw(ctypes.byref(args), _stream(stream)))

    def sample_step_workspace_bytes(self, rows: int, vocab: int) -> int:
        return self._check(self.lib.levo_hip_sample_step_workspace_bytes(rows, vocab))

    def sample_step_static(self, args: SampleArgs, draw: DrawArgs | None, stream=None):
        d = ctypes.byref(draw) if draw is not None else None
        return self._check(self.lib.levo_hip_sample_step_static(ctypes.byref(args), d, _stream(stream)))

    def sample_step(self, args: SampleArgs, draw: DrawArgs | None, workspace, workspace_bytes: int, stream=None):
        d = ctypes.byref(draw) if draw is not None else None
        return self._check(self.lib.levo_hip_sample_step(ctypes.byref(args), d, _addr(workspace), workspace_bytes,
                                                         _stream(stream)))

    def flow_cfg_euler(self, state, v_uncond, v_cond, n, guidance, dt, stream=None):
        return self._check(self.lib.levo_hip_flow_cfg_euler(_addr(state), _addr(v_uncond), _addr(v_cond), n,
                                                            guidance, dt, _stream(stream)))

    def flow_cfg_euler_checked(self, state, v_uncond, v_cond, n, guidance, dt, flags, stream=None):
        return self._check(self.lib.levo_hip_flow_cfg_euler_checked(_addr(state), _addr(v_uncond), _addr(v_cond),
                                                                    n, guidance, dt, _addr(flags), _stream(stream)))

    def check_finite(self, x, n, flags, bit, stream=None):
        return self._check(self.lib.levo_hip_check_finite(_addr(x), n, _addr(flags), bit, _stream(stream)))

    def repetition_penalty(self, logits, vocab, recent, n_recent, penalty, limit=0, stream=None):
        return self._check(self.lib.levo_hip_repetition_penalty(_addr(logits), vocab, _addr(recent), n_recent,
                                                                penalty, limit, _stream(stream)))

    def flow_incontext(self, state, noise, context, n_prefix, time, sigma_min, stream=None):
        return self._check(self.lib.levo_hip_flow_incontext(_addr(state), _addr(noise), _addr(context), n_prefix,
                                                            time, sigma_min, _stream(stream)))

    def flow_assemble_input(self, args: FlowInputArgs, stream=None):
        return self._check(self.lib.levo_hip_flow_assemble_input(ctypes.byref(args), _stream(stream)))

    def flow_step(self, args: FlowStepArgs, stream=None):
        return self._check(self.lib.levo_hip_flow_step(ctypes.byref(args), _stream(stream)))

    def flow_normalize(self, raw, mean, stddev, out, frames, latent, flags=None, stream=None):
        return self._check(self.lib.levo_hip_flow_normalize(_addr(raw), _addr(mean), _addr(stddev), _addr(out),
                                                             frames, latent, _addr(flags), _stream(stream)))

    def flow_denormalize(self, x, mean, stddev, out, frames, latent, flags=None, stream=None):
        return self._check(self.lib.levo_hip_flow_denormalize(_addr(x), _addr(mean), _addr(stddev), _addr(out),
                                                               frames, latent, _addr(flags), _stream(stream)))

    def mul_mat_q8_0(self, weight, x_blocks, y, y_pitch, rows, k, n_vec, stream=None):
        return self._check(self.lib.levo_hip_mul_mat_q8_0(_addr(weight), _addr(x_blocks), _addr(y), y_pitch,
                                                          rows, k, n_vec, _stream(stream)))

    def mul_mat_q8_0_multi(self, mats, k, n_vec, x_blocks=None, x=None, x_pitch=0, stream=None, packed=False):
        """mats: (weight, y, y_pitch, rows) tuples sharing the activations,
        given as Q8_0 blocks (x_blocks) or as F32 rows (x, x_pitch); packed:
        the weights come from repack_q8_0 and x_blocks holds columns
        (quantize_q8_0_columns)."""
        arr = (MatQ8_0 * max(len(mats), 1))()
        for i, (w, y, y_pitch, rows) in enumerate(mats):
            arr[i] = MatQ8_0(_addr(w), _addr(y), y_pitch, rows)
        fn = self.lib.levo_hip_mul_mat_q8_0_packed_multi if packed else self.lib.levo_hip_mul_mat_q8_0_multi
        return self._check(fn(arr, len(mats), _addr(x_blocks), _addr(x), x_pitch, k, n_vec, _stream(stream)))

    def repack_q8_0(self, blocks, packed, rows, k, stream=None):
        return self._check(self.lib.levo_hip_repack_q8_0(_addr(blocks), _addr(packed), rows, k, _stream(stream)))

    def quantize_q8_0_columns(self, x, x_pitch, columns, n_vec, k, stream=None):
        return self._check(self.lib.levo_hip_quantize_q8_0_columns(_addr(x), x_pitch, _addr(columns), n_vec, k,
                                                                   _stream(stream)))

    def mul_mat_q8_0_packed(self, packed, x_columns, y, y_pitch, rows, k, n_vec, stream=None):
        return self._check(self.lib.levo_hip_mul_mat_q8_0_packed(_addr(packed), _addr(x_columns), _addr(y), y_pitch,
                                                                 rows, k, n_vec, _stream(stream)))

    def quantize_q8_K(self, x, y, k, stream=None):
        return self._check(self.lib.levo_hip_quantize_q8_K(_addr(x), _addr(y), k, _stream(stream)))

    def mul_mat_kquant(self, qtype, weight, x_blocks, y, y_pitch, rows, k, n_vec, stream=None):
        return self._check(self.lib.levo_hip_mul_mat_kquant(qtype, _addr(weight), _addr(x_blocks), _addr(y), y_pitch,
                                                            rows, k, n_vec, _stream(stream)))

    def mul_mat_kquant_multi(self, mats, k, n_vec, x_blocks=None, x=None, x_pitch=0, stream=None):
        """mats: (type, weight, y, y_pitch, rows) tuples sharing the activations,
        given as Q8_K blocks (x_blocks) or as F32 rows (x, x_pitch)."""
        arr = (MatKquant * max(len(mats), 1))()
        for i, (t, w, y, y_pitch, rows) in enumerate(mats):
            arr[i] = MatKquant(t, _addr(w), _addr(y), y_pitch, rows)
        return self._check(self.lib.levo_hip_mul_mat_kquant_multi(arr, len(mats), _addr(x_blocks), _addr(x),
                                                                  x_pitch, k, n_vec, _stream(stream)))

    def row_size(self, qtype, n):
        return self._check(self.lib.levo_hip_row_size(qtype, n))

    def quantize_chunk(self, qtype, src, dst, start, nrows, n_per_row, imatrix=None, stream=None):
        return self._check(self.lib.levo_hip_quantize_chunk(qtype, _addr(src), _addr(dst), start, nrows, n_per_row,
                                                            _addr(imatrix), _stream(stream)))

    def quantize_rows(self, qtype, src, src_type, src_cols, src_stride, dst, nrows, dst_cols, stream=None):
        return self._check(self.lib.levo_hip_quantize_rows(qtype, _addr(src), src_type, src_cols, src_stride,
                                                           _addr(dst), nrows, dst_cols, _stream(stream)))

    def dequantize(self, qtype, src, dst, dst_type, k, stream=None):
        return self._check(self.lib.levo_hip_dequantize(qtype, _addr(src), _addr(dst), dst_type, k,
                                                        _stream(stream)))

    def fp32_to_fp16_row(self, x, y, n, stream=None):
        return self._check(self.lib.levo_hip_fp32_to_fp16_row(_addr(x), _addr(y), n, _stream(stream)))

    def fp16_to_fp32_row(self, x, y, n, stream=None):
        return self._check(self.lib.levo_hip_fp16_to_fp32_row(_addr(x), _addr(y), n, _stream(stream)))


_LIB: LevoHip | None = None


def lib() -> LevoHip:
    global _LIB
    if _LIB is None:
        _LIB = LevoHip()
    return _LIB
