/*
 * levo_hip.h — C ABI of the MI355X (gfx950) kernels behind LeVo2.cpp's
 * elementwise / reduction / broadcast hot path.
 *
 * Conventions (all entry points):
 *   - Every data pointer is a device pointer owned by the caller; no entry
 *     point allocates device memory.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and
 *     runs asynchronously; entry points are reentrant across streams.
 *   - Return LEVO_HIP_OK (0) or a negative levo_hip_status. The message of the
 *     last failure on the calling thread is levo_hip_last_error(), the same
 *     pattern as the reference's C ABI (include/cantor_engine.h:50-60,
 *     src/cantor-abi.cpp:58-82).
 *   - Arithmetic follows the reference's F32 rounding points (no FMA
 *     contraction where the reference computes a*b+c in two roundings).
 *
 * Each declaration names the reference function or ggml op chain it replaces.
 */
#ifndef LEVO_HIP_H
#define LEVO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LEVO_HIP_ABI_VERSION 4

/* Same tag as HIP's hipStream_t, so a hipStream_t converts without a cast. */
typedef struct ihipStream_t * levo_hip_stream_t;

typedef enum levo_hip_status {
    LEVO_HIP_OK = 0,
    LEVO_HIP_ERR_INVALID = -1,     /* bad argument (null pointer, shape, value) */
    LEVO_HIP_ERR_UNSUPPORTED = -2, /* type / shape combination not implemented */
    LEVO_HIP_ERR_RUNTIME = -3      /* HIP runtime reported an error */
} levo_hip_status;

/* Element / block types, numbered as ggml's public ggml_type enum so that a
 * ggml caller passes its tensor->type unchanged. */
typedef enum levo_hip_type {
    LEVO_HIP_TYPE_F32 = 0,
    LEVO_HIP_TYPE_F16 = 1,
    LEVO_HIP_TYPE_Q4_0 = 2,
    LEVO_HIP_TYPE_Q8_0 = 8,
    LEVO_HIP_TYPE_Q4_K = 12,
    LEVO_HIP_TYPE_Q5_K = 13,
    LEVO_HIP_TYPE_Q6_K = 14,
    LEVO_HIP_TYPE_Q8_K = 15
} levo_hip_type;

/* Message of the last failing call on this thread ("" if none). */
const char * levo_hip_last_error(void);
int levo_hip_abi_version(void);

/* ------------------------------------------------------------------------ */
/* SnakeBeta                                                                 */
/* ------------------------------------------------------------------------ */

/* Replaces levo::detail::snake_beta (src/levo-audio-ops.cpp:125-152; decl
 * src/levo-audio-ops.h:30-33), which builds the ggml chain
 *   y = x + sin(x * exp(alpha_log))^2 / (exp(beta_log) * 1 + 1e-9)
 * over x of ggml shape [time, channels, 1] (each channel row contiguous).
 * x, y: F32 [channels][time] with row strides x_stride, y_stride (elements,
 * >= time); y may equal x. alpha_log, beta_log: [channels] of param_type
 * (F32, or F16 promoted exactly to F32 as src/levo-audio-ops.cpp:143-144). */
int levo_hip_snake_beta(const float * x, int64_t x_stride,
                        const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                        float * y, int64_t y_stride,
                        int64_t channels, int64_t time, levo_hip_stream_t stream);

/* One job of levo_hip_snake_beta_batch: the arguments of levo_hip_snake_beta. */
typedef struct levo_hip_snake_job {
    const float * x;
    int64_t x_stride;
    const void * alpha_log;
    const void * beta_log;
    levo_hip_type param_type;
    float * y;
    int64_t y_stride;
    int64_t channels;
    int64_t time;
} levo_hip_snake_job;

/* Up to 16 independent levo_hip_snake_beta jobs in one launch (the SnakeBeta
 * instances of a decoder window, src/levo-vae.cpp:80-88, 94-97, 218-233):
 * their tiles share one grid, so the small jobs run beside the large ones
 * instead of each paying a launch and a ramp of its own. Each job computes
 * exactly what levo_hip_snake_beta computes for it; jobs must not overlap
 * (y may equal x within a job). Jobs the vector path cannot take (time or a
 * stride not a multiple of 4, unaligned rows) run as separate launches. */
int levo_hip_snake_beta_batch(const levo_hip_snake_job * jobs, int n_jobs, levo_hip_stream_t stream);

/* SnakeBeta + Conv1d (stride 1) + bias + residual in one pass: the Oobleck
 * decoder's conv_1d_f32 calls (ggml_im2col + ggml_mul_mat + bias,
 * src/levo-audio-ops.cpp:56-87) with the SnakeBeta that feeds them
 * (run_residual src/levo-vae.cpp:91-100; decode :219-221, :260-262):
 *   y[co][t] = (sum_{ci,k} weight[co][ci][k] * s(x)[ci][t + k*dilation - padding])
 *              + bias[co] (+ residual[co][t])
 * x: F32 [c_in][x_stride], t_in samples, zero outside [0, t_in). s: SnakeBeta
 * with alpha_log / beta_log [c_in] of param_type (F32 or F16), as
 * levo_hip_snake_beta computes it; both NULL: s is the identity. weight: F32
 * [c_out][c_in][kernel] (ggml ne = [kernel, c_in, c_out]), kernel 1, 3, 5 or
 * 7. bias [c_out] or NULL. residual [c_out][residual_stride] or NULL.
 * y: F32 [c_out][y_stride], t_out = t_in + 2*padding - dilation*(kernel-1).
 * y may be the residual, never x. Accumulation on the F32 matrix cores, so
 * y agrees with the reference to F32 rounding. */
int levo_hip_snake_conv1d(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                          const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                          const float * weight, int64_t c_out, int64_t kernel, const float * bias,
                          int64_t padding, int64_t dilation, const float * residual, int64_t residual_stride,
                          float * y, int64_t y_stride, levo_hip_stream_t stream);

/* Floats of workspace levo_hip_snake_conv1d_split uses at most for an output
 * of c_out x t_out: four partial sums of the output, rows padded to a
 * multiple of 4 floats; < 0 if invalid. */
int64_t levo_hip_snake_conv1d_split_workspace_floats(int64_t c_out, int64_t t_out);

/* levo_hip_snake_conv1d (the same arguments, results and errors) with a
 * device workspace of workspace_floats floats (16-byte aligned, overlapping
 * none of the tensors). When the output has fewer 128 x 128 tiles than the
 * GPU has compute units, the input channels are split over up to four
 * workgroups per tile (as many partial sums as the workspace holds), each
 * writing its partial sum to the workspace, and a second launch adds the
 * partials in split order, then the bias and the residual. The result is
 * deterministic; it differs from levo_hip_snake_conv1d's by the F32 rounding
 * of the other summation order. A grid that already fills the GPU, c_out <= 4
 * or too small a workspace run levo_hip_snake_conv1d's path unchanged. Same
 * reference call sites as levo_hip_snake_conv1d. */
int levo_hip_snake_conv1d_split(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                                const float * weight, int64_t c_out, int64_t kernel, const float * bias,
                                int64_t padding, int64_t dilation, const float * residual, int64_t residual_stride,
                                float * y, int64_t y_stride, float * workspace, int64_t workspace_floats,
                                levo_hip_stream_t stream);

/* Weights of a ConvTranspose1d with kernel 2 * stride (the decoder's
 * upsamplers) rearranged for levo_hip_snake_conv_transpose1d: weight is
 * ggml's [c_in][c_out][2 * stride] (ne = [kernel, c_out, c_in]); packed
 * (stride * c_out * c_in * 2 floats) holds, for every phase r < stride,
 * [c_out][c_in][2] = (weight[..][..][r + stride], weight[..][..][r]). Done once
 * per model; packed must be 16-byte aligned for the fast weight loads. */
int levo_hip_conv_transpose1d_pack_weights(const float * weight, float * packed, int64_t c_in, int64_t c_out,
                                           int64_t stride, levo_hip_stream_t stream);

/* SnakeBeta + ConvTranspose1d (kernel 2 * stride) + crop + bias: the
 * decoder's upsample step, run_snake then conv_transpose_1d_f32
 * (src/levo-vae.cpp:223-228; src/levo-audio-ops.cpp:89-123:
 * ggml_conv_transpose_1d, the crop of `padding` samples on both sides, the
 * bias). Output sample t = q * stride + r - padding of phase r is
 * sum_ci (w[ci][co][r] * s(x)[ci][q] + w[ci][co][r + stride] * s(x)[ci][q - 1]),
 * so each phase is a 2-tap convolution on the matrix cores (one launch, the
 * phase on the grid's z axis). x: F32 [c_in][x_stride] with t_in samples;
 * SnakeBeta parameters as in levo_hip_snake_conv1d (NULL: none);
 * packed_weight from levo_hip_conv_transpose1d_pack_weights; bias [c_out] or
 * NULL; y: F32 [c_out][y_stride] with (t_in + 1) * stride - 2 * padding
 * samples. The sum is accumulated on the F32 matrix cores in another order
 * than ggml's, so y agrees with the reference to F32 rounding. */
int levo_hip_snake_conv_transpose1d(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                    const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                                    const float * packed_weight, int64_t c_out, int64_t stride, const float * bias,
                                    int64_t padding, float * y, int64_t y_stride, levo_hip_stream_t stream);

/* Floats of workspace levo_hip_snake_conv_transpose1d_split uses at most:
 * four partial sums of every phase's t_in + 1 output columns, rows padded to
 * a multiple of 4 floats; < 0 if invalid. */
int64_t levo_hip_snake_conv_transpose1d_split_workspace_floats(int64_t c_out, int64_t t_in, int64_t stride);

/* levo_hip_snake_conv_transpose1d (the same arguments, results and errors)
 * with a device workspace (16-byte aligned, overlapping none of the
 * tensors): when the launch has fewer workgroups (128 x 128 tiles times
 * stride phases) than the GPU has compute units, the input channels are
 * split over up to four workgroups per tile and phase, as
 * levo_hip_snake_conv1d_split does, and a second launch adds each output
 * sample's partial sums in split order, then the bias. Deterministic; it
 * differs from levo_hip_snake_conv_transpose1d by the F32 rounding of the
 * other summation order. Same reference call sites. */
int levo_hip_snake_conv_transpose1d_split(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                          const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                                          const float * packed_weight, int64_t c_out, int64_t stride,
                                          const float * bias, int64_t padding, float * y, int64_t y_stride,
                                          float * workspace, int64_t workspace_floats, levo_hip_stream_t stream);

/* The VAE decoder's weights in device memory, the fields of
 * vae_decoder_weights (src/levo-vae-model.h:39-66). Convolution weights are
 * F32 in ggml order ([k][c_in][c_out] ne = W[c_out][c_in][k] in memory);
 * each upsample weight is the packed form of
 * levo_hip_conv_transpose1d_pack_weights. The reference promotes F16
 * artifacts' convolution weights to F32 before every operator; widen them
 * once at load with levo_hip_fp16_to_fp32_row (exact). SnakeBeta parameters
 * are of param_type (F32 or F16). */
typedef struct levo_hip_vae_snake {
    const void * alpha_log;
    const void * beta_log;
} levo_hip_vae_snake;
typedef struct levo_hip_vae_conv {
    const float * weight;
    const float * bias;
} levo_hip_vae_conv;
typedef struct levo_hip_vae_residual {
    levo_hip_vae_snake pre;
    levo_hip_vae_conv conv_0;     /* k 7, dilation 1 / 3 / 9 */
    levo_hip_vae_snake post;
    levo_hip_vae_conv conv_1;     /* k 1 */
} levo_hip_vae_residual;
typedef struct levo_hip_vae_stage {
    levo_hip_vae_snake activation;
    levo_hip_vae_conv upsample;   /* packed ConvTranspose1d weight */
    levo_hip_vae_residual residual[3];
} levo_hip_vae_stage;
typedef struct levo_hip_vae_decoder_weights {
    levo_hip_vae_conv input;      /* [2048][64][7] */
    levo_hip_vae_stage stage[5];  /* decode order: strides 10, 6, 4, 4, 2 */
    levo_hip_vae_snake output_activation;
    const float * output_weight;  /* [2][128][7], no bias */
    levo_hip_type param_type;
} levo_hip_vae_decoder_weights;

/* validate_weights (src/levo-vae.cpp:56-78): LEVO_HIP_OK when every weight
 * levo_hip_vae_decode reads is non-null and param_type is F32 or F16, else
 * LEVO_HIP_ERR_INVALID naming the first missing one in the reference's order. */
int levo_hip_vae_validate_weights(const levo_hip_vae_decoder_weights * weights);

/* One residual unit of the decoder, run_residual (src/levo-vae.cpp:91-100):
 * y = x + conv_1(snake_post(conv_0(snake_pre(x)))), conv_0 kernel 7 at
 * `dilation` with padding 3 * dilation, conv_1 kernel 1, each with its bias
 * (either may be null). x, y, h: [channels][time] F32, rows contiguous. y must
 * not overlap x: every output sample reads its neighbours' inputs. h receives
 * conv_0's output unless the unit runs as one launch (128 channels, both
 * SnakeBeta parameter sets, 16-byte aligned weights), where the intermediate
 * never leaves the device's caches and h is not touched. */
int levo_hip_vae_residual_unit(const float * x, int64_t channels, int64_t time,
                               const levo_hip_vae_residual * unit, int64_t dilation,
                               levo_hip_type param_type, float * y, float * h,
                               levo_hip_stream_t stream);

/* Workspace bytes levo_hip_vae_decode needs for `frames` latent frames
 * (three activation buffers of 128 x 1920 x frames floats); < 0 if invalid. */
int64_t levo_hip_vae_decode_workspace_bytes(int64_t frames);

/* vae_decoder::decode (src/levo-vae.cpp:172-276) on the device: latent
 * [64][frames] F32 to audio [2][frames * 1920] F32, with the reference's
 * hyper-parameters (latent 64, widths 2048 -> 1024 -> 512 -> 256 -> 128 ->
 * 128, strides 10, 6, 4, 4, 2, dilations 1, 3, 9). 37 fused SnakeBeta +
 * convolution steps (input conv, 7 per stage, output conv) in 31 launches:
 * the 128-channel residual units (stages 4 and 5) are one launch each, as
 * levo_hip_vae_residual_unit runs them; a convolution whose grid would
 * leave compute units idle runs split-K (levo_hip_snake_conv1d_split) with
 * one more combine launch, its partial sums in the free tail of a workspace
 * buffer. None of the activations leaves the device, the caller's
 * workspace (16-byte aligned, levo_hip_vae_decode_workspace_bytes) holds
 * them. Every weight the
 * reference's validate_weights requires (src/levo-vae.cpp:56-78) must be
 * non-null. stage_outputs, when non-null, holds 5 device pointers (each may
 * be null): stage s's output [width_s][frames * prod(strides[0..s])] is
 * copied there, the reference's capture_stages tensors. Every convolution
 * agrees with the reference to F32 rounding; so does the composition. The
 * reference's host-side latent checks (shape, finite values) belong to the
 * caller, which holds the latent on the host. */
int levo_hip_vae_decode(const levo_hip_vae_decoder_weights * weights, const float * latent, int64_t frames,
                        float * audio, float * const * stage_outputs, void * workspace, int64_t workspace_bytes,
                        levo_hip_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Residual add + RMSNorm / LayerNorm (rows of `dim` contiguous elements)    */
/* ------------------------------------------------------------------------ */

/* h = x + delta (delta may be NULL: h = x), written to h_out when non-NULL;
 * y = rms_norm(h, eps) * weight.
 * act_type F16: the LeLM F16-activation chain of rms_norm_weighted
 *   (src/levo-kv.cpp:153-160) after the F16 residual add (:462, :507):
 *   h = f16(x + d); y = f16(f16(h * 1/sqrtf(mean(h^2) + eps)) * w); weight F16.
 * act_type F32: src/levo-lm.cpp:131-137 (weight F32, or F16 promoted to F32).
 * The row reduction accumulates in double, like ggml-cpu's ggml_float sum. */
int levo_hip_residual_rms_norm(levo_hip_type act_type, const void * x, const void * delta,
                               const void * weight, levo_hip_type weight_type,
                               void * h_out, void * y, int64_t rows, int64_t dim, float eps,
                               levo_hip_stream_t stream);

/* h = x + delta as above; y = norm(h, eps) * gamma + beta — the Flow
 * estimator's layer_norm = ggml_norm -> ggml_mul -> ggml_add
 * (src/levo-flow-estimator.cpp:106-109) fused with its residual add
 * (:221-227, :243-247). act_type F32 (reference) or F16 (F16 storage with the
 * same F32 chain, output rounded once to F16). gamma/beta of param_type. */
int levo_hip_residual_layer_norm(levo_hip_type act_type, const void * x, const void * delta,
                                 const void * gamma, const void * beta, levo_hip_type param_type,
                                 void * h_out, void * y, int64_t rows, int64_t dim, float eps,
                                 levo_hip_stream_t stream);

/* One per-batch vector of the Flow estimator's modulation
 * (modulation_chunk, src/levo-flow-estimator.cpp:95-104): entry b, channel c
 * is dynamic[b * stride + c] + learned[c] (ggml_add(dynamic, learned)), or
 * dynamic[b * stride + c] when learned is NULL. dynamic NULL: no vector. */
typedef struct levo_hip_batch_vector {
    const float * dynamic;  /* [batches] entries of dim floats, `stride` floats apart */
    int64_t stride;
    const float * learned;  /* [dim], or NULL */
} levo_hip_batch_vector;

typedef struct levo_hip_modulated_norm_args {
    const float * x;              /* [rows][dim] F32 residual stream */
    const float * delta;          /* [rows][dim] branch output, or NULL (h = x) */
    levo_hip_batch_vector gate;   /* h = (delta * gate) + x; no gate: h = x + delta */
    const void * gamma;           /* [dim] */
    const void * beta;            /* [dim] */
    levo_hip_type param_type;     /* F32 or F16 gamma / beta */
    levo_hip_batch_vector scale;  /* y = (t * (scale + 1)) + shift; no scale: y = t */
    levo_hip_batch_vector shift;  /* given exactly when scale is */
    float * h_out;                /* [rows][dim], or NULL */
    float * y;                    /* [rows][dim] */
    int64_t rows;                 /* a multiple of rows_per_batch */
    int64_t rows_per_batch;       /* row r uses batch entry r / rows_per_batch */
    int64_t dim;                  /* a multiple of 4, at most 4096 */
    float eps;
} levo_hip_modulated_norm_args;

/* A Flow estimator block boundary in one pass, one rounding per ggml op as the
 * graph computes it: the gated residual current = (out * gate) + residual
 * (src/levo-flow-estimator.cpp:221-227, 243-246), layer_norm
 * t = (norm(current, eps) * gamma) + beta (:106-109) and add_scale_shift
 * y = (t * (scale + 1)) + shift (:89-93, at :214, :233, :260). h_out receives
 * current (the next residual). x, delta, h_out, y, gamma, beta and each
 * vector's rows are 16-byte aligned (8-byte for F16 gamma / beta); x may be
 * h_out (in place). */
int levo_hip_residual_layer_norm_modulated(const levo_hip_modulated_norm_args * args,
                                           levo_hip_stream_t stream);

/* ------------------------------------------------------------------------ */
/* CFG combine + temperature softmax + argmax / top-k (LeLM sampling)        */
/* ------------------------------------------------------------------------ */

/* Elementwise out = uncond + scale * (cond - uncond): levo::apply_cfg
 * (src/levo-sampling.cpp:22-28) and combine_renderer_cfg
 * (src/levo-renderer-pattern.cpp:123-135). */
int levo_hip_cfg_combine(float * out, const float * uncond, const float * cond, int64_t n,
                         float scale, levo_hip_stream_t stream);

#define LEVO_HIP_MAX_STREAMS 8

/* Arguments of levo_hip_cfg_sample. Rows are ordered [position][stream]
 * (stream = row % n_streams) and start row_pitch elements apart. */
typedef struct levo_hip_sample_args {
    const float * cond;   /* [rows][row_pitch] conditional logits */
    const float * uncond; /* [rows][row_pitch]; NULL: logits = cond (no CFG) */
    int64_t rows;
    int64_t vocab;        /* logits per row (V), 1 <= V <= 32768 */
    int64_t row_pitch;    /* >= vocab */
    float cfg_scale;      /* l = u + cfg_scale * (c - u) */
    float temperature;    /* softmax temperature for cand_probs / row_lse (> 0) */
    int32_t n_streams;    /* 1 .. LEVO_HIP_MAX_STREAMS */
    int32_t top_k[LEVO_HIP_MAX_STREAMS]; /* per stream; 0 or >= V keeps every id */
    /* Optional unique-token repetition penalty (src/levo-sampling.cpp:39-47,
     * :137-143): recent is [rows][n_recent] ids (< 0 = padding); each distinct
     * id in [0, penalty_limit) is divided once by repetition_penalty. */
    const int64_t * recent;
    int32_t n_recent;
    float repetition_penalty;
    int64_t penalty_limit; /* 0 = V */
    /* Optional ids forced to -inf on stream-0 rows after the penalty
     * (src/levo-sampling.cpp:146-147). */
    const int64_t * ignore;
    int32_t n_ignore;
    /* Outputs. */
    int32_t * best;       /* [rows] first maximum (std::max_element, :94-96); -1 on NaN */
    int32_t * count;      /* [rows] candidate count (may exceed capacity); -1 on NaN */
    int32_t * cand_ids;   /* [rows][capacity] candidates in ascending id order (:84-93) */
    float * cand_logits;  /* [rows][capacity] their adjusted logits, or NULL */
    float * cand_probs;   /* [rows][capacity] exp((l-max)/T) normalised over the
                           * candidates (:98-107), or NULL */
    float * row_max;      /* [rows] max adjusted logit, or NULL */
    float * row_lse;      /* [rows] log sum_v exp(l_v / T) over all V ids, or NULL */
    int32_t capacity;     /* candidate slots per row (>= 1) */
} levo_hip_sample_args;

/* levo::apply_unique_token_repetition_penalty (src/levo-sampling.cpp:39-47)
 * on one device row of `vocab` logits, in place: each distinct id of
 * recent[0, n_recent) inside [0, limit) is divided once by `penalty`
 * (limit 0 or > vocab means vocab). Fails with "repetition penalty must be
 * finite and positive" like the reference. */
int levo_hip_repetition_penalty(float * logits, int64_t vocab, const int64_t * recent,
                                int32_t n_recent, float penalty, int64_t limit,
                                levo_hip_stream_t stream);

/* One launch per batch of rows: CFG, penalty/ignore, NaN check, row max and
 * argmax, the top-k candidate set of sample_top_k_counted
 * (src/levo-sampling.cpp:75-116; ties with the k-th value are kept) and the
 * temperature softmax over it. The single uniform draw of a sampled token
 * stays on the host so the mt19937_64 cursor is unchanged. */
int levo_hip_cfg_sample(const levo_hip_sample_args * args, levo_hip_stream_t stream);

/* Token codes of levo_hip_sample_draw besides ids >= 0. */
#define LEVO_HIP_TOKEN_NAN (-1)      /* the row holds a NaN: the reference throws "logits contain NaN" */
#define LEVO_HIP_TOKEN_OVERFLOW (-2) /* more candidates than `capacity`: run levo_hip_cfg_sample again
                                      * with a larger capacity and draw again with the same bits */
#define LEVO_HIP_TOKEN_RECHECK (-3)  /* the target lies within the double-rounding bound of a cumulative
                                      * boundary: draw this row on the host from its candidates with
                                      * the raw value bits[draws[r] - 1] */

/* Arguments of levo_hip_sample_draw. The candidate inputs are the outputs of
 * levo_hip_cfg_sample for the same rows (cand_logits and row_max required). */
typedef struct levo_hip_draw_args {
    const int32_t * best;        /* [rows] */
    const int32_t * count;       /* [rows] */
    const int32_t * cand_ids;    /* [rows][capacity] */
    const float * cand_logits;   /* [rows][capacity] */
    const float * row_max;       /* [rows] */
    int64_t rows;
    int32_t capacity;
    float temperature;           /* finite, >= 0; 0 = greedy */
    int32_t use_sampling;        /* 0 = greedy: tokens = best, no draws */
    const uint64_t * bits;       /* [rows] the next raw outputs of the caller's mt19937_64 */
    int64_t * tokens;            /* [rows] out: sampled id or LEVO_HIP_TOKEN_* */
    int32_t * draws;             /* [rows] out: raw values consumed by rows 0..r */
} levo_hip_draw_args;

/* The sampled branch of sample_top_k_counted (src/levo-sampling.cpp:97-115;
 * Sampler::sample_streams :129-152 for consecutive rows) on the device: the
 * double weights exp((double)((v - max) / T)) of the candidates in id order,
 * their sequential sum, the uniform (bits >> 11 + 0.5) / 2^53 and the
 * cumulative search. Row r draws, taking the next unused entry of `bits`,
 * exactly when the reference's row would consume one mt19937_64 value
 * (sampling, T != 0, no NaN, finite maximum); greedy rows return `best`.
 * The caller advances its engine by draws[rows - 1]. One small launch; only
 * `tokens` and `draws` need to reach the host. */
int levo_hip_sample_draw(const levo_hip_draw_args * args, levo_hip_stream_t stream);

/* Workspace bytes levo_hip_sample_step needs for `rows` rows of `vocab`
 * logits; < 0 if invalid. */
int64_t levo_hip_sample_step_workspace_bytes(int64_t rows, int64_t vocab);

/* One decode step of Sampler::sample_streams (src/levo-sampling.cpp:129-152):
 * levo_hip_cfg_sample's outputs for every row (CFG, penalty, ignore list,
 * first maximum, top-k candidates of sample_top_k_counted :75-116), then,
 * when `draw` is not NULL, the tokens and draw counts of levo_hip_sample_draw
 * (:97-115). The results equal those two calls'. Each row is split over
 * one-wave parts of 512 ids that hand the ids above a bound to `workspace`;
 * a second launch checks that they hold the row's top k, selects it and, with
 * at most 8 rows, draws (more rows take a third launch for the draw; a row
 * the hand-over does not cover is selected again from its logits). It is
 * made for the few rows of a decode step
 * (rows <= 4095). workspace: 16-byte aligned device memory of
 * levo_hip_sample_step_workspace_bytes(rows, vocab) bytes, whose contents
 * need no initialization; one workspace serves calls of any shape. Calls
 * that share a workspace must not overlap. `draw`
 * reads the rows' own outputs: its best, count, cand_ids, cand_logits,
 * row_max, rows and capacity must be those of `args`. */
int levo_hip_sample_step(const levo_hip_sample_args * args, const levo_hip_draw_args * draw,
                         void * workspace, int64_t workspace_bytes, levo_hip_stream_t stream);

/* levo_hip_sample_step without a workspace argument and without any
 * allocation: the workspace is a 2 MiB array the library holds on every GPU
 * it runs on, until the process ends (enough for 230 rows of 16385 logits;
 * larger calls fail with LEVO_HIP_ERR_INVALID, naming the sizes). Same
 * results as levo_hip_sample_step. Calls that overlap on one GPU share that
 * array and race: serialize them. The first call on each GPU looks the
 * array's address up (hipGetSymbolAddress, which may load the code object):
 * make that first call outside stream capture, e.g. one eager call before
 * capturing; later calls only launch kernels. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (HIP graph
 * capture, serving loops that forbid hipMalloc). */
int levo_hip_sample_step_static(const levo_hip_sample_args * args, const levo_hip_draw_args * draw,
                                levo_hip_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Flow Euler / CFG latent update                                            */
/* ------------------------------------------------------------------------ */

/* state[e] += dt * (v_uncond[e] + guidance * (v_cond[e] - v_uncond[e]))
 * (src/levo-flow-renderer.cpp:105 with the CFG lambda :307); v_cond NULL:
 * state += dt * v_uncond. Two roundings per product/sum, as the reference. */
int levo_hip_flow_cfg_euler(float * state, const float * v_uncond, const float * v_cond,
                            int64_t n, float guidance, float dt, levo_hip_stream_t stream);

/* Bits of the non-finite flag word written by the checked entry points. */
#define LEVO_HIP_NONFINITE_VELOCITY 1 /* a combined velocity was NaN or infinite */
#define LEVO_HIP_NONFINITE_STATE 2    /* an updated state value was NaN or infinite */

/* levo_hip_flow_cfg_euler plus the reference's per-step finiteness checks
 * (require_finite on the velocity and on the updated state,
 * src/levo-flow-renderer.cpp:104, :106): ORs LEVO_HIP_NONFINITE_VELOCITY /
 * LEVO_HIP_NONFINITE_STATE into *nonfinite (a device int32 the caller clears)
 * when any combined velocity / updated state element is not finite. The
 * update itself is identical to the unchecked entry point. */
int levo_hip_flow_cfg_euler_checked(float * state, const float * v_uncond, const float * v_cond,
                                    int64_t n, float guidance, float dt, int32_t * nonfinite,
                                    levo_hip_stream_t stream);

/* *flags |= bit when any x[e], e < n, is NaN or infinite (device int32 flag
 * word): the entry checks of solve_flow_euler on the noise, the in-context
 * latent and a resume state (src/levo-flow-renderer.cpp:24-28, 70-71, 80). */
int levo_hip_check_finite(const float * x, int64_t n, int32_t * flags, int32_t bit,
                          levo_hip_stream_t stream);

/* In-context prefix of one Euler step (src/levo-flow-renderer.cpp:94-101):
 * state[e] = (1 - (1 - sigma_min) * time) * noise[e] + time * context[e]
 * for e < n_prefix. */
int levo_hip_flow_incontext(float * state, const float * noise, const float * context,
                            int64_t n_prefix, float time, float sigma_min,
                            levo_hip_stream_t stream);

/* ---- Device-resident Flow step (estimator tensors left in HBM) ---------- */

/* Arguments of levo_hip_flow_assemble_input: the estimator input rows
 * [batch][frames][mask_dim + latent + condition_width + latent] that
 * append_model_row builds on the host for every step
 * (src/levo-flow-renderer.cpp:35-53, :287-295). */
typedef struct levo_hip_flow_input_args {
    float * model_input;           /* out: [batch][frames][hidden] */
    int32_t batch;                 /* 1, or 2 with row 0 unconditional (conditioning zeroed) */
    int64_t frames;
    const float * mask_embedding;  /* [frames][mask_dim] */
    int64_t mask_dim;
    const float * context;         /* normalized in-context latent [frames][latent] */
    int64_t latent;
    const float * conditioning;    /* [frames][condition_width] (2 * condition_dim) */
    int64_t condition_width;
    const float * state;           /* Euler state [frames][latent] before step `step` */
    const float * noise;           /* initial noise [frames][latent] (prefix rows) */
    int64_t prefix_frames;         /* in-context frames */
    int64_t step, steps;           /* the state columns carry step `step`'s prefix interpolation */
    float sigma_min;
} levo_hip_flow_input_args;

/* Writes every estimator input row: mask embedding | in-context latent |
 * conditioning (zeros for the unconditional row) | state, the state's
 * prefix rows interpolated as at the start of step `step` (:93-101). One
 * launch per window; levo_hip_flow_step keeps the state columns current. */
int levo_hip_flow_assemble_input(const levo_hip_flow_input_args * args, levo_hip_stream_t stream);

/* Arguments of levo_hip_flow_step. */
typedef struct levo_hip_flow_step_args {
    float * state;                 /* [frames][latent] the reference's Euler `state`, in place */
    const float * output;          /* estimator output [batch][frames][out_pitch] */
    int64_t out_pitch;             /* floats per output row (hidden) */
    int64_t vel_col;               /* first velocity column (hidden - latent) */
    int32_t batch;                 /* 1: v = output; 2: row 0 unconditional, row 1 conditional */
    float guidance;                /* v = u + guidance * (c - u) when batch == 2 */
    int64_t frames, latent;
    int64_t step, steps;           /* performs step `step` of `steps` (dt = 1 / steps) */
    const float * noise;           /* [frames][latent] */
    const float * context;         /* [frames][latent] normalized in-context latent */
    int64_t prefix_frames;
    float sigma_min;
    float * next_input;            /* estimator input [batch][frames][in_pitch] or NULL */
    int64_t in_pitch, state_col;   /* where the state columns of next_input start */
    const float * mean, * stddev;  /* [latent], used with denormalized */
    float * denormalized;          /* [frames][latent] after the last step, or NULL */
    int32_t * nonfinite;           /* device flag word: LEVO_HIP_NONFINITE_* ORed in, or NULL */
} levo_hip_flow_step_args;

/* One Euler step of solve_flow_euler (src/levo-flow-renderer.cpp:89-117) fed
 * straight from the estimator output: the velocity slice of
 * estimator::velocity (src/levo-flow-estimator.cpp:390-399), the CFG lambda
 * (src/levo-flow-renderer.cpp:301-309), the step's prefix interpolation
 * (:93-101) and update (:105) with its finiteness checks (:104, :106). The
 * next step's state columns (prefix interpolated for step + 1) go into
 * next_input; after the last step the prefix is restored (:112-113) and
 * denormalize_latents (src/levo-flow-conditioning.cpp:124-133) writes
 * state * stddev + mean. Replaces the 17.6 MB host-to-device and 17.6 MB
 * device-to-host copies per step at LeVo's window (2 x 1000 x 2200 F32,
 * src/levo-flow-estimator.cpp:368, :382). */
int levo_hip_flow_step(const levo_hip_flow_step_args * args, levo_hip_stream_t stream);

/* conditioning::normalize_latents (src/levo-flow-conditioning.cpp:113-121):
 * normalized[f][c] = (raw[f][c] - mean[c]) / stddev[c]; and
 * denormalize_latents (:124-133): raw = normalized * stddev + mean. Two F32
 * roundings each. ORs LEVO_HIP_NONFINITE_STATE into *nonfinite (device
 * int32, or NULL) when an input value is not finite (the reference's
 * require_finite on the input, :116, :128). */
int levo_hip_flow_normalize(const float * raw, const float * mean, const float * stddev, float * normalized,
                            int64_t frames, int64_t latent, int32_t * nonfinite, levo_hip_stream_t stream);
int levo_hip_flow_denormalize(const float * normalized, const float * mean, const float * stddev, float * raw,
                              int64_t frames, int64_t latent, int32_t * nonfinite, levo_hip_stream_t stream);

/* ------------------------------------------------------------------------ */
/* Q8_0 / Q4_0 block quantization (ggml block layouts, little-endian)        */
/*   block_q8_0 = { f16 d; int8 qs[32]; }  34 bytes                          */
/*   block_q4_0 = { f16 d; uint8 qs[16]; } 18 bytes                          */
/* ------------------------------------------------------------------------ */

/* ggml_row_size(type, n_per_row) for Q8_0 / Q4_0 (n_per_row a multiple of 32)
 * and the K-quants Q4_K / Q5_K / Q6_K / Q8_K (a multiple of 256); < 0 on error. */
int64_t levo_hip_row_size(levo_hip_type type, int64_t n_per_row);

/* Replaces ggml_quantize_chunk(type, src, dst, start, nrows, n_per_row,
 * imatrix) as called at tools/levo-quantize.cpp:386-388 (ggml's
 * quantize_row_q8_0_ref / quantize_row_q4_0_ref, and for the Q4_K_M / Q5_K_M
 * / Q6_K profiles quantize_row_q4_K_ref / q5_K_ref / q6_K_ref with n_per_row
 * a multiple of 256: block_q4_K 144 B, block_q5_K 176 B, block_q6_K 210 B).
 * Returns the bytes written (nrows * row size) or a negative levo_hip_status.
 * Q8_0 ignores imatrix as ggml does; the other types require imatrix ==
 * NULL (the tool passes NULL). Q8_0 / Q4_0 dst needs 2-byte alignment
 * (16-byte aligned destinations take the dwordx4 store path); K-quant dst
 * any alignment. The source values must be finite, as the tool checks. */
int64_t levo_hip_quantize_chunk(levo_hip_type type, const float * src, void * dst,
                                int64_t start, int64_t nrows, int64_t n_per_row,
                                const float * imatrix, levo_hip_stream_t stream);

/* write_tensor's chunk path fused into one pass (tools/levo-quantize.cpp:
 * 355-388): rows of src_cols values (src_type F32 or F16, widened exactly),
 * row stride src_row_stride elements, zero-padded to dst_cols (a multiple of
 * 32 for Q8_0 / Q4_0, of 256 for Q4_K / Q5_K / Q6_K, >= src_cols) and
 * quantized. Returns bytes written or < 0. */
int64_t levo_hip_quantize_rows(levo_hip_type type, const void * src, levo_hip_type src_type,
                               int64_t src_cols, int64_t src_row_stride, void * dst,
                               int64_t nrows, int64_t dst_cols, levo_hip_stream_t stream);

/* dequantize_row_q8_0 / dequantize_row_q4_0 (ggml to_float): k values
 * (multiple of 32) to dst_type F32, or F16 (exact products rounded RNE).
 * Also dequantize_row_q4_K / q5_K / q6_K (k a multiple of 256, src 16-byte
 * aligned): Q4_K / Q5_K y = d1 * q - m1 with d1 = d * sc and m1 = dmin * m
 * each rounded and the last step in one rounding (as ggml's backends are
 * compiled, contraction on); Q6_K y = (d * sc) * (q - 32), two roundings. */
int levo_hip_dequantize(levo_hip_type type, const void * src, void * dst, levo_hip_type dst_type,
                        int64_t k, levo_hip_stream_t stream);

/* Decode mat-vec with Q8_0 weights and Q8_0 activations: the
 * ggml_vec_dot_q8_0_q8_0 rows of ggml_mul_mat(W, x) on ggml's CPU backend
 * for the quantized LeLM / Flow matrices (src/levo-quantization.h:96-118).
 * weight: [rows][k/32] block_q8_0; x_blocks: [n_vec][k/32] block_q8_0, the
 * activation columns quantized once with levo_hip_quantize_chunk (ggml's
 * vec_dot_type for Q8_0 is Q8_0), shared by every matrix with that input;
 * both 16-byte aligned. y: [n_vec][y_pitch] F32, y[v][r] = sum over blocks of
 * (float)sumi * (d_w * d_x), sumi the exact int32 dot of the quants. The F32
 * terms are summed in a tree, so y agrees with ggml's sequential loop to F32
 * rounding. k a multiple of 32 (pad rows as padded_input_columns does,
 * :120-130), k <= 32768; 1 <= n_vec <= 8, n_vec * k <= 26000 or so (the
 * activations live in the workgroup's LDS; k = 11008 at n_vec = 2 fits). */
int levo_hip_mul_mat_q8_0(const void * weight, const void * x_blocks, float * y, int64_t y_pitch,
                          int64_t rows, int64_t k, int64_t n_vec, levo_hip_stream_t stream);

/* One matrix of levo_hip_mul_mat_q8_0_multi. */
typedef struct levo_hip_mat_q8_0 {
    const void * weight;  /* [rows][k/32] block_q8_0, 16-byte aligned */
    float * y;            /* [n_vec][y_pitch] F32 */
    int64_t y_pitch;      /* >= rows */
    int64_t rows;
} levo_hip_mat_q8_0;

/* levo_hip_mul_mat_q8_0 for 1 to 4 matrices that read the same activation
 * columns (a decode layer's q / k / v, or gate / up: ggml_mul_mat calls that
 * share src1, each quantizing it to its vec_dot_type first) in one launch.
 * The activations come either as Q8_0 blocks (x_blocks, as for
 * levo_hip_mul_mat_q8_0) or as F32 x [n_vec][x_pitch] (16-byte aligned,
 * x_pitch >= k and a multiple of 4), which the launch quantizes itself with
 * levo_hip_quantize_chunk's block function, for n_vec * k / 32 <= 256
 * blocks; pass exactly one of the two. Every y equals what
 * levo_hip_quantize_chunk + levo_hip_mul_mat_q8_0 give for that matrix, bit
 * for bit. Matrices of zero rows are skipped. */
int levo_hip_mul_mat_q8_0_multi(const levo_hip_mat_q8_0 * mats, int32_t n_mats, const void * x_blocks,
                                const float * x, int64_t x_pitch, int64_t k, int64_t n_vec,
                                levo_hip_stream_t stream);

/* A Q8_0 matrix rearranged once, when the model is loaded, for the decode
 * mat-vec: the same bytes (rows * k/32 * 34) in aligned pieces. Row r takes
 * bytes [32 k/32 r, 32 k/32 (r + 1)): the first 16 quants of each of its
 * blocks in block order, then the last 16 of each; the F16 scales follow all
 * rows, [rows][k/32], at byte 32 k/32 rows. No counterpart in the reference
 * (ggml keeps block_q8_0 in its buffers; its CPU backend has repacked
 * buffer types for some formats): the layout lets every lane load whole
 * blocks with aligned 16-byte loads. blocks and packed are device memory,
 * 16-byte aligned, not overlapping; k a multiple of 32, k <= 32768. */
int levo_hip_repack_q8_0(const void * blocks, void * packed, int64_t rows, int64_t k, levo_hip_stream_t stream);

/* Activation columns for the packed mat-vec: x [n_vec][x_pitch] F32 (16-byte
 * aligned, x_pitch >= k and a multiple of 4) quantized to Q8_0 by
 * levo_hip_quantize_chunk's block function, stored as the quants of every
 * column in value order ([n_vec][k] int8) followed by the block scales
 * widened to F32 ([n_vec][k/32]): n_vec * k / 32 * 36 bytes, 16-byte
 * aligned. The same numbers as levo_hip_quantize_chunk's blocks, in the form
 * the mat-vec keeps in LDS. 1 <= n_vec <= 8, k a multiple of 32. */
int levo_hip_quantize_q8_0_columns(const float * x, int64_t x_pitch, void * columns, int64_t n_vec, int64_t k,
                                   levo_hip_stream_t stream);

/* levo_hip_mul_mat_q8_0 and levo_hip_mul_mat_q8_0_multi on matrices repacked
 * by levo_hip_repack_q8_0 (levo_hip_mat_q8_0.weight points at the packed
 * matrix), with the activations as columns (levo_hip_quantize_q8_0_columns)
 * where the block-layout entry points take Q8_0 blocks; the multi form also
 * takes F32 x as levo_hip_mul_mat_q8_0_multi does. Same limits, and y equal
 * bit for bit to what the block-layout entry points give on the original
 * blocks and the same activations. */
int levo_hip_mul_mat_q8_0_packed(const void * packed, const void * x_columns, float * y, int64_t y_pitch,
                                 int64_t rows, int64_t k, int64_t n_vec, levo_hip_stream_t stream);
int levo_hip_mul_mat_q8_0_packed_multi(const levo_hip_mat_q8_0 * mats, int32_t n_mats, const void * x_columns,
                                       const float * x, int64_t x_pitch, int64_t k, int64_t n_vec,
                                       levo_hip_stream_t stream);

/* ------------------------------------------------------------------------ */
/* K-quants on the decode path (ggml block layouts, QK_K = 256):              */
/*   block_q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}            144 B */
/*   block_q5_K {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} 176 B */
/*   block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}           210 B */
/*   block_q8_K {f32 d; i8 qs[256]; i16 bsums[16]}                      292 B */
/* the matrices of the Q6_K / Q5_K_M / Q4_K_M profiles                       */
/* (src/levo-quantization.h:47-55, 96-118).                                   */
/* ------------------------------------------------------------------------ */

/* quantize_row_q8_K_ref, ggml's vec_dot_type for Q4_K / Q5_K / Q6_K (the
 * activation side of ggml_mul_mat on the CPU backend): k values (a multiple
 * of 256; x 16-byte aligned) to k / 256 blocks of 292 bytes (y 4-byte
 * aligned). Per block d = 1 / (-127 / max) with max the first value of
 * largest magnitude, q = min(127, nearest_int(-127 / max * x)), bsums the
 * sums of 16 quants. A block of zeros gets zero bsums (ggml leaves them as
 * they were). */
int levo_hip_quantize_q8_K(const float * x, void * y, int64_t k, levo_hip_stream_t stream);

/* Decode mat-vec with K-quant weights: the ggml_vec_dot_q4_K_q8_K /
 * q5_K_q8_K / q6_K_q8_K rows of ggml_mul_mat(W, x). weight: [rows][k / 256]
 * blocks of `type` (16-byte aligned); x_blocks: [n_vec][k / 256] block_q8_K
 * from levo_hip_quantize_q8_K (4-byte aligned), shared by every matrix with
 * that input. y: [n_vec][y_pitch] F32, y[v][r] = sum over blocks of
 * (d_w * d_x) * sumi - (dmin_w * d_x) * summ (Q6_K: no min term), sumi and
 * summ the exact integer sums of the reference's loop; the F32 terms are
 * summed in a tree, so y agrees with ggml's loop to F32 rounding. k a
 * multiple of 256 (pad rows as padded_input_columns does,
 * src/levo-quantization.h:120-125); 1 <= n_vec <= 8, n_vec * k * 1.14 bytes
 * of activations in LDS (<= 160 KB). */
int levo_hip_mul_mat_kquant(levo_hip_type type, const void * weight, const void * x_blocks, float * y,
                            int64_t y_pitch, int64_t rows, int64_t k, int64_t n_vec, levo_hip_stream_t stream);

/* One matrix of levo_hip_mul_mat_kquant_multi. */
typedef struct levo_hip_mat_kquant {
    levo_hip_type type;   /* Q4_K, Q5_K or Q6_K */
    const void * weight;  /* [rows][k / 256] blocks, 16-byte aligned */
    float * y;            /* [n_vec][y_pitch] F32 */
    int64_t y_pitch;      /* >= rows */
    int64_t rows;
} levo_hip_mat_kquant;

/* levo_hip_mul_mat_kquant for 1 to 4 matrices, of any of the three types,
 * that read the same activation columns (a decode layer's q / k / v, or
 * gate / up: ggml_mul_mat calls that share src1 and quantize it to Q8_K
 * first; the Q4_K_M / Q5_K_M profiles mix Q4_K or Q5_K with Q6_K in such a
 * group, src/levo-quantization.h:75-95) in one launch. The activations come
 * either as block_q8_K (x_blocks, as for levo_hip_mul_mat_kquant) or as F32
 * x [n_vec][x_pitch] (16-byte aligned, x_pitch >= k and a multiple of 4),
 * which the launch quantizes itself exactly as levo_hip_quantize_q8_K does,
 * for n_vec * k <= 4096; pass exactly one of the two. Each y equals what
 * levo_hip_quantize_q8_K + levo_hip_mul_mat_kquant give for that matrix bit
 * for bit when the matrices have equal row counts (the launch shares one lane
 * geometry, chosen for the largest matrix; with unequal row counts the sums
 * may associate differently, within F32 rounding). Matrices of zero rows are
 * skipped. */
int levo_hip_mul_mat_kquant_multi(const levo_hip_mat_kquant * mats, int32_t n_mats, const void * x_blocks,
                                  const float * x, int64_t x_pitch, int64_t k, int64_t n_vec,
                                  levo_hip_stream_t stream);

/* ggml_fp32_to_fp16_row / ggml_fp16_to_fp32_row (tools/levo-quantize.cpp:
 * 358, 369): IEEE round-to-nearest-even narrowing, exact widening. */
int levo_hip_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n, levo_hip_stream_t stream);
int levo_hip_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n, levo_hip_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LEVO_HIP_H */
