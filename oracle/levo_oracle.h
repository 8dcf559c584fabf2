/*
 * levo_oracle.h — CPU restatement of the reference's hot-path arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it. The product path (levo2.cpp_amd/) never links or calls it.
 *
 * Every function restates one reference function or ggml-cpu op chain with the
 * same rounding points (F32 intermediates, no FMA contraction: the library is
 * built with -ffp-contract=off) and cites the reference file:line it follows.
 * ggml itself is an un-vendored submodule of the reference (pinned at
 * 8846b79e66747bb9f68597420e95114c177315ce), so the ggml-internal pieces
 * (rms_norm/norm row reductions, quantize_row_q8_0_ref/q4_0_ref, fp16
 * conversion) are restated from ggml's published scalar algorithms.
 *
 * Pinning status per function (what checks it: tests/test_oracle.py):
 *   lo_fp32_to_fp16 / lo_fp16_to_fp32 .... numpy float16 (IEEE RNE), exhaustive
 *   lo_snake_beta_f32 .................... reference KAT (tests/test-audio-ops.cpp:163-215),
 *                                          float64 closed form, special cases
 *   lo_residual_rms_norm_* /
 *   lo_residual_layer_norm_* ............. float64 closed forms (constant rows, +-1 rows),
 *                                          float64 brute force, numpy float16 pipeline
 *   lo_residual_layer_norm_modulated_f32 . float64 brute force of the ggml op chain,
 *                                          reductions to lo_residual_layer_norm_f32 (no gate,
 *                                          no modulation; gate 1, scale 0, shift 0)
 *   lo_apply_cfg ......................... reference KATs (tests/test-sampling.cpp:8,
 *                                          tests/test-renderer-pattern.cpp:88-90) and the
 *                                          compiled reference (oracle/_ref) bit-for-bit
 *   lo_mt19937_64 ........................ C++ standard [rand.predef] 10000th value,
 *                                          compiled reference engine
 *   lo_sample_top_k / lo_sample_streams .. reference KATs (tests/test-sampling.cpp) and the
 *                                          compiled reference (oracle/_ref) token-for-token
 *   lo_flow_* ............................ reference KAT (tests/test-flow-renderer.cpp:33-65),
 *                                          closed form for constant velocity
 *   lo_quantize_row_q8_0 / q4_0 .......... reference KAT (tests/test-quantization.cpp:32-81),
 *                                          block invariants, numpy restatement of ggml's
 *                                          published reference quantizer
 *   lo_conv1d_f32 ........................ float64 direct convolution within the sequential-sum
 *                                          error bound; identity / shift kernels exactly
 *   lo_conv_transpose1d_f32 .............. float64 scatter form within the error bound; delta
 *                                          kernels upsample exactly
 *   lo_mul_mat_q8_0 ...................... float64 sum of the same block terms within the
 *                                          sequential-sum error bound; integer-valued
 *                                          blocks (d = 1) equal the exact integer product
 *   lo_quantize_row_q8_K ................. invariants (code range, bsums, extreme -> -127),
 *                                          exact recovery of representable rows, zero block
 *   lo_dequantize_row_kquant ............. blocks packed from the published layout by an
 *                                          independent packer: every value exact
 *   lo_vec_dot_kquant_q8_K /
 *   lo_mul_mat_kquant .................... integer-valued blocks exactly; float64 dot of
 *                                          the dequantized operands within the bound
 */
#ifndef LEVO_ORACLE_H
#define LEVO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes mirror the reference's thrown exceptions. */
enum {
    LO_OK = 0,
    LO_ERR_EMPTY = -1,        /* "cannot sample an empty vocabulary" */
    LO_ERR_TEMPERATURE = -2,  /* "temperature must be finite and non-negative" */
    LO_ERR_NAN = -3,          /* "logits contain NaN" */
    LO_ERR_PENALTY = -4,      /* "repetition penalty must be finite and positive" */
    LO_ERR_ARGUMENT = -5,
};

/* ggml_type numbering for the block formats (ggml.h public enum). */
enum { LO_TYPE_F32 = 0, LO_TYPE_F16 = 1, LO_TYPE_Q4_0 = 2, LO_TYPE_Q8_0 = 8,
       LO_TYPE_Q4_K = 12, LO_TYPE_Q5_K = 13, LO_TYPE_Q6_K = 14, LO_TYPE_Q8_K = 15 };

/* ---- F16 <-> F32 (ggml_fp32_to_fp16_row / ggml_fp16_to_fp32_row,
 *      tools/levo-quantize.cpp:358,369; IEEE binary16, round-to-nearest-even) */
uint16_t lo_fp32_to_fp16(float f);
float lo_fp16_to_fp32(uint16_t h);
void lo_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n);
void lo_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n);

/* ---- SnakeBeta: the ggml-cpu chain built by levo::detail::snake_beta
 *      (src/levo-audio-ops.cpp:146-151): alpha = exp(a), beta = exp(b)*1 + 1e-9,
 *      then five full passes mul -> sin -> sqr -> div -> add over x[C][T]. */
void lo_snake_beta_f32(const float * x, const float * alpha_log, const float * beta_log,
                       float * y, int64_t channels, int64_t time, int n_threads);

/* ---- Residual add + RMSNorm, F16 activations (src/levo-kv.cpp:153-160 with
 *      emulate_fp16_activations, residual adds :462,507): h = f16(x + d);
 *      n = f16(rms_norm_f32(h)); y = f16(n * w).  delta may be NULL (no add),
 *      h_out may be NULL. */
void lo_residual_rms_norm_f16(const uint16_t * x, const uint16_t * delta, const uint16_t * weight,
                              uint16_t * h_out, uint16_t * y, int64_t rows, int64_t dim,
                              float eps, int n_threads);
/* F32 tower (src/levo-lm.cpp:131-137): h = x + d; y = rms_norm(h) * w. */
void lo_residual_rms_norm_f32(const float * x, const float * delta, const float * weight,
                              float * h_out, float * y, int64_t rows, int64_t dim,
                              float eps, int n_threads);
/* Residual add + LayerNorm (src/levo-flow-estimator.cpp:106-109):
 * y = norm(h) * gamma + beta.  F32 and F16-activation variants. */
void lo_residual_layer_norm_f32(const float * x, const float * delta, const float * gamma,
                                const float * beta, float * h_out, float * y, int64_t rows,
                                int64_t dim, float eps, int n_threads);
void lo_residual_layer_norm_f16(const uint16_t * x, const uint16_t * delta, const uint16_t * gamma,
                                const uint16_t * beta, uint16_t * h_out, uint16_t * y,
                                int64_t rows, int64_t dim, float eps, int n_threads);

/* Per-batch modulation vector of the Flow estimator's blocks: entry b is
 * dynamic[b * stride + c] + learned[c] (learned may be NULL). */
typedef struct lo_batch_vector {
    const float * dynamic;
    int64_t stride;
    const float * learned;
} lo_batch_vector;
/* Gated residual + LayerNorm + AdaLN modulation (src/levo-flow-estimator.cpp:
 * 89-109, 221-233, 243-261): current = (delta * gate) + x;
 * y = ((norm(current) * gamma + beta) * (scale + 1)) + shift. gate NULL:
 * current = x + delta; delta NULL: current = x; scale NULL: no modulation
 * (shift is then ignored). Single-threaded. */
void lo_residual_layer_norm_modulated_f32(const float * x, const float * delta, const lo_batch_vector * gate,
                                          const float * gamma, const float * beta,
                                          const lo_batch_vector * scale, const lo_batch_vector * shift,
                                          float * h_out, float * y, int64_t rows, int64_t rows_per_batch,
                                          int64_t dim, float eps);

/* ---- CFG (src/levo-sampling.cpp:22-28; src/levo-renderer-pattern.cpp:123-135):
 *      out = u + s * (c - u), two F32 roundings, no FMA. */
void lo_apply_cfg(const float * cond, const float * uncond, float * out, int64_t n, float scale);

/* ---- std::mt19937_64 (C++ [rand.predef]) and the sampler's uniform draw
 *      (src/levo-sampling.cpp:12-18). */
typedef struct lo_mt19937_64 {
    uint64_t state[312];
    int index;
} lo_mt19937_64;
void lo_mt_seed(lo_mt19937_64 * rng, uint64_t seed);
uint64_t lo_mt_next(lo_mt19937_64 * rng);
void lo_mt_discard(lo_mt19937_64 * rng, uint64_t count);
double lo_manual_uniform(lo_mt19937_64 * rng, uint64_t * draws);

/* Unique-token repetition penalty (src/levo-sampling.cpp:39-47). */
int lo_repetition_penalty(float * logits, int64_t vocab, const int64_t * recent, int64_t n_recent,
                          float penalty, int64_t vocabulary_limit);

/* Top-k candidate set of sample_top_k_counted (src/levo-sampling.cpp:84-96):
 * candidates are every index whose value is >= the k-th largest value, in
 * ascending index order; best is the first maximum among them.  Returns the
 * candidate count (>= 0) or a negative LO_ERR_*; writes at most cap ids. */
int64_t lo_top_k_candidates(const float * logits, int64_t vocab, int64_t top_k,
                            int64_t * best, int64_t * candidates, int64_t cap);

/* Full sample_top_k_counted (src/levo-sampling.cpp:75-116). Returns LO_OK and
 * writes *token, or a negative LO_ERR_*. *draws counts consumed RNG values. */
int lo_sample_top_k(const float * logits, int64_t vocab, int64_t top_k, float temperature,
                    int use_sampling, lo_mt19937_64 * rng, uint64_t * draws, int64_t * token);

/* Sampler::sample_streams (src/levo-sampling.cpp:129-152) for one position:
 * streams[q] = logits + q*vocab.  recent is [n_streams][n_recent] (entries < 0
 * are padding and ignored; pass NULL for no history).  The repetition window
 * is applied by the caller (pass the trailing window). */
int lo_sample_streams(const float * logits, int64_t n_streams, int64_t vocab,
                      int use_sampling, float temperature, int64_t top_k_mixed,
                      int64_t top_k_detail, float repetition_penalty,
                      const int64_t * recent, int64_t n_recent,
                      const int64_t * ignore_tokens, int64_t n_ignore,
                      lo_mt19937_64 * rng, uint64_t * draws, int64_t * tokens);

/* ---- Flow Euler/CFG (src/levo-flow-renderer.cpp:91-117, :283-310) */
/* state[e] = noise_scale*noise[e] + time*context[e] for e < n_prefix, with
 * noise_scale = 1 - (1 - sigma_min) * time (src/levo-flow-renderer.cpp:94-101). */
void lo_flow_incontext(float * state, const float * noise, const float * context,
                       int64_t n_prefix, float time, float sigma_min);
/* v = u + g*(c - u) (or v = u when cond is NULL); state += dt * v
 * (src/levo-flow-renderer.cpp:105, :307). */
void lo_flow_cfg_euler(float * state, const float * v_uncond, const float * v_cond, int64_t n,
                       float guidance, float dt);

/* ---- Q8_0 / Q4_0 (ggml quantize_row_q8_0_ref / quantize_row_q4_0_ref,
 *      dequantize_row_q8_0 / q4_0; called via ggml_quantize_chunk at
 *      tools/levo-quantize.cpp:386-388). k must be a multiple of 32. */
void lo_quantize_row_q8_0(const float * x, void * y, int64_t k);
void lo_quantize_row_q4_0(const float * x, void * y, int64_t k);
void lo_dequantize_row_q8_0(const void * x, float * y, int64_t k);
void lo_dequantize_row_q4_0(const void * x, float * y, int64_t k);
/* conv_1d_f32 (src/levo-audio-ops.cpp:56-87), stride 1: ggml_im2col (input
 * index t + k * dilation - padding, zero outside [0, t_in)), ggml_mul_mat of
 * the columns with the [c_out][c_in * kernel] weight (the dot over
 * ci * kernel + k in that order, F32, generic loop), then the bias add
 * (add_channel_bias, :42-54) as its own rounding. x [c_in][t_in],
 * w [c_out][c_in][kernel] (ggml ne = [kernel, c_in, c_out]), bias [c_out] or
 * NULL, y [c_out][t_out], t_out = t_in + 2 * padding - dilation * (kernel - 1). */
void lo_conv1d_f32(const float * x, int64_t c_in, int64_t t_in, const float * w, int64_t c_out, int64_t kernel,
                   const float * bias, int64_t padding, int64_t dilation, float * y, int threads);

/* conv_transpose_1d_f32 (src/levo-audio-ops.cpp:89-123): ggml_conv_transpose_1d
 * (stride, no padding, dilation 1), then the crop of `padding` samples on
 * both sides and the bias add. ggml-cpu's loop: for every output channel,
 * input position i and tap k, v = dot over ci of w[ci][co][k] * x[ci][i]
 * (F32, generic order), then full[co][i * stride + k] += v in order of i.
 * x [c_in][t_in], w [c_in][c_out][kernel] (ggml ne = [kernel, c_out, c_in]),
 * y [c_out][t_out], t_out = (t_in - 1) * stride + kernel - 2 * padding. */
void lo_conv_transpose1d_f32(const float * x, int64_t c_in, int64_t t_in, const float * w, int64_t c_out,
                             int64_t kernel, int64_t stride, int64_t padding, const float * bias, float * y);

/* ggml_mul_mat(W, x) on ggml's CPU backend for a Q8_0 weight (the quantized
 * LeLM / Flow matrices, src/levo-quantization.h:96-118): W is [rows][k/32]
 * Q8_0 blocks, x [n_vec][k] F32, y [n_vec][rows]. Each activation column is
 * quantized with lo_quantize_row_q8_0 (Q8_0's vec_dot_type is Q8_0), then
 * every row takes ggml_vec_dot_q8_0_q8_0's generic loop: per block the exact
 * int32 dot sumi of the quants, sumf += sumi * (d_w * d_x) in block order,
 * F32. (ggml's SIMD variants sum the same terms in another order.) */
void lo_mul_mat_q8_0(const void * w, const float * x, float * y, int64_t rows, int64_t k, int64_t n_vec);

/* ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, NULL).
 * Returns bytes written or 0 for an unsupported type. */
/* ---- K-quants (ggml quantize_row_q8_K_ref, dequantize_row_q{4,5,6}_K,
 *      ggml_vec_dot_q{4,5,6}_K_q8_K generic loops; the Q6_K / Q5_K_M / Q4_K_M
 *      profiles' matrices, src/levo-quantization.h:47-55, 96-118). k is a
 *      multiple of 256. The Q4_K / Q5_K dequantizers round d1 * q - m1 once
 *      (fmaf), as ggml's backends are compiled; Q8_K blocks of zeros get zero
 *      bsums. */
int64_t lo_kquant_block_bytes(int type);
void lo_quantize_row_q8_K(const float * x, void * y, int64_t k);
void lo_dequantize_row_kquant(int type, const void * x, float * y, int64_t k);
float lo_vec_dot_kquant_q8_K(int type, const void * w, const void * xq, int64_t k);
/* ggml CPU mul_mat of K-quant rows [rows][k / 256] by x [n_vec][k] (each
 * vector quantized to Q8_K first) -> y [n_vec][rows]. */
void lo_mul_mat_kquant(int type, const void * w, const float * x, float * y, int64_t rows, int64_t k,
                       int64_t n_vec);

/* ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row, NULL) for
 * Q8_0, Q4_0 and the K-quant reference quantizers (quantize_row_q{4,5,6}_K_ref,
 * n_per_row a multiple of 256). */
void lo_quantize_row_q4_K(const float * x, void * y, int64_t k);
void lo_quantize_row_q5_K(const float * x, void * y, int64_t k);
void lo_quantize_row_q6_K(const float * x, void * y, int64_t k);
size_t lo_quantize_chunk(int type, const float * src, void * dst, int64_t start, int64_t nrows,
                         int64_t n_per_row);
/* write_tensor's per-chunk path (tools/levo-quantize.cpp:355-388): widen F16
 * rows exactly, zero-pad each row from src_cols to dst_cols, quantize. */
size_t lo_quantize_f16_rows_padded(int type, const uint16_t * src, int64_t nrows, int64_t src_cols,
                                   int64_t dst_cols, void * dst);

/* ---- Seeded synthetic inputs: SplitMix64 + Box-Muller as in
 *      src/levo-render.cpp:87-112 (native_gaussian_noise). */
void lo_gaussian_noise(float * out, int64_t count, uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif /* LEVO_ORACLE_H */
