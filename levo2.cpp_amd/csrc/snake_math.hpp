// SnakeBeta arithmetic shared by the standalone kernel and the convolution
// that applies it to its input tile: y = x + sin^2(x * alpha_c) / beta_c with
// alpha_c = exp(alpha_log_c), beta_c = exp(beta_log_c) * 1 + 1e-9, the
// ggml chain of levo::detail::snake_beta (src/levo-audio-ops.cpp:125-152).
#pragma once

#include "common.hpp"

namespace levo_hip {

template <typename P>
__device__ __forceinline__ float param_f32(const P * p, uint32_t i);
template <>
__device__ __forceinline__ float param_f32<float>(const float * p, uint32_t i) {
    return p[i];
}
template <>
__device__ __forceinline__ float param_f32<uint16_t>(const uint16_t * p, uint32_t i) {
    return h2f(p[i]);
}

struct snake_param {
    float alpha;  // exp(alpha_log)
    float beta;   // exp(beta_log) * 1 + 1e-9
    float rbeta;  // RN(1 / beta)
};

// Quotient p / beta from the correctly rounded reciprocal plus one FMA
// residual correction (Markstein): q0 = p*r, e = p - q0*beta (exact in an FMA),
// q = q0 + e*r.
__device__ __forceinline__ float div_by(float p, float beta, float rbeta) {
    const float q0 = p * rbeta;
    const float e = __builtin_fmaf(-q0, beta, p);
    return __builtin_fmaf(e, rbeta, q0);
}

// sin(m)^2 for |m| <= kSinSqFastMax. sin^2 has period pi, so one Cody-Waite
// reduction m = k*pi + r (pi split into three F32 parts, each product and
// subtraction one FMA) leaves |r| <= pi/2, where sin(r) = r + r^3 * P(r^2)
// with P of degree 4. The coefficients are a least-squares fit with Lawson
// reweighting towards the minimax absolute error on [0, pi/2] (1.9e-11 in
// double); after F32 rounding of coefficients and arithmetic the result is
// within 2.4e-7 of sin^2 over |m| <= 8192, the same size as the error of
// squaring a correctly rounded F32 sine.
constexpr float kSinSqFastMax = 8192.0f;

__device__ __forceinline__ float sin_sq_reduced(float m) {
    constexpr float kInvPi = 0x1.45f306p-2f;
    constexpr float kPi1 = 0x1.921fb6p+1f;   // pi rounded to F32
    constexpr float kPi2 = -0x1.777a5cp-24f; // pi - kPi1 rounded to F32
    constexpr float kPi3 = -0x1.ee59dap-49f; // pi - kPi1 - kPi2
    constexpr float c3 = -0x1.555556p-3f;
    constexpr float c5 = 0x1.11110ap-7f;
    constexpr float c7 = -0x1.a01770p-13f;
    constexpr float c9 = 0x1.7164e2p-19f;
    constexpr float c11 = -0x1.9982bcp-26f;
    const float k = __builtin_rintf(m * kInvPi);
    float r = __builtin_fmaf(-k, kPi1, m);
    r = __builtin_fmaf(-k, kPi2, r);
    r = __builtin_fmaf(-k, kPi3, r);
    const float r2 = r * r;
    float p = __builtin_fmaf(r2, c11, c9);
    p = __builtin_fmaf(r2, p, c7);
    p = __builtin_fmaf(r2, p, c5);
    p = __builtin_fmaf(r2, p, c3);
    const float s = __builtin_fmaf(r * r2, p, r);
    return s * s;
}

// ggml_sqr(ggml_sin(m)): the reduced form, or sinf for |m| beyond it and for
// NaN / infinity (the branch is skipped unless a lane needs it).
__device__ __forceinline__ float sin_sq(float m) {
    float p = sin_sq_reduced(m);
    if (!(__builtin_fabsf(m) <= kSinSqFastMax)) {
        const float s = sinf(m);
        p = s * s;
    }
    return p;
}

__device__ __forceinline__ float snake(float x, const snake_param & q) {
    const float m = x * q.alpha;    // ggml_mul(input, alpha)
    const float p = sin_sq(m);      // ggml_sin, ggml_sqr
    const float d = div_by(p, q.beta, q.rbeta);  // ggml_div(periodic, beta)
    return x + d;                   // ggml_add(input, .)
}

// The per-channel parameters from the log-domain values
// (src/levo-audio-ops.cpp:146-148: exp, then scale_bias(., 1, 1e-9)).
__device__ __forceinline__ snake_param make_snake_param(float alpha_log, float beta_log) {
    snake_param q;
    q.alpha = expf(alpha_log);
    const float e = expf(beta_log);
    q.beta = e * 1.0f + 1.0e-9f;  // ggml_scale_bias(exp(beta_log), 1, 1e-9)
    q.rbeta = 1.0f / q.beta;
    return q;
}

}  // namespace levo_hip
