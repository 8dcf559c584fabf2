// Fused residual add + RMSNorm / LayerNorm, one wave64 per row.
//
// Each row (dim contiguous elements) is owned by one wavefront: it is loaded
// once with dwordx4 accesses, kept in registers, reduced with cross-lane
// shuffles (no LDS, no barrier), normalised and written once. The reduction
// accumulates in double like ggml-cpu's ggml_float row sums, so the F32 mean /
// variance (and hence every rounding point after it) matches the CPU chain.
//
//   RMSNorm F16 (src/levo-kv.cpp:153-160, residual :462/:507):
//     h = f16(x + d); n = f16(h * 1/sqrtf(mean(h^2) + eps)); y = f16(n * w)
//   RMSNorm F32 (src/levo-lm.cpp:131-137): h = x + d; y = (h * scale) * w
//   LayerNorm  (src/levo-flow-estimator.cpp:106-109, residual :221-227):
//     h = x + d; v = h - mean; scale = 1/sqrtf(mean(v^2) + eps);
//     y = ((v * scale) * gamma) + beta   (F16 storage: h and y rounded to F16)
#include "common.hpp"

#include <type_traits>

namespace levo_hip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

// Loads n consecutive values starting at p (16-byte aligned when n*size >= 16).
template <int N>
__device__ __forceinline__ void load_f32(const float * p, float (&o)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
            const f32x4 v = reinterpret_cast<const f32x4 *>(p)[k];
            o[4 * k] = v.x;
            o[4 * k + 1] = v.y;
            o[4 * k + 2] = v.z;
            o[4 * k + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) o[k] = p[k];
    }
}

template <int N>
__device__ __forceinline__ void load_u16(const uint16_t * p, uint16_t (&o)[N]) {
    if constexpr (N == 8) {
        const u16x8 v = *reinterpret_cast<const u16x8 *>(p);
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = v[k];
    } else if constexpr (N == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        o[0] = v.x & 0xffffu;
        o[1] = v.x >> 16;
        o[2] = v.y & 0xffffu;
        o[3] = v.y >> 16;
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) o[k] = p[k];
    }
}

template <int N>
__device__ __forceinline__ void store_u16(uint16_t * p, const uint16_t (&v)[N]) {
    if constexpr (N == 8) {
        u16x8 w;
#pragma unroll
        for (int k = 0; k < 8; ++k) w[k] = v[k];
        *reinterpret_cast<u16x8 *>(p) = w;
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) p[k] = v[k];
    }
}

template <int N>
__device__ __forceinline__ void store_f32(float * p, const float (&v)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int k = 0; k < N / 4; ++k) {
            f32x4 w;
            w.x = v[4 * k];
            w.y = v[4 * k + 1];
            w.z = v[4 * k + 2];
            w.w = v[4 * k + 3];
            reinterpret_cast<f32x4 *>(p)[k] = w;
        }
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) p[k] = v[k];
    }
}

// Parameter vector (F32 or F16 storage, chosen at run time) widened to F32.
template <int N>
__device__ __forceinline__ void load_param(const void * p, bool f16, int64_t e, float (&o)[N]) {
    if (f16) {
        uint16_t t[N];
        load_u16<N>(static_cast<const uint16_t *>(p) + e, t);
#pragma unroll
        for (int k = 0; k < N; ++k) o[k] = h2f(t[k]);
    } else {
        load_f32<N>(static_cast<const float *>(p) + e, o);
    }
}

// T = uint16_t (F16 storage) or float. VEC elements per group, NV groups per lane.
template <typename T, bool kLayer, int VEC, int NV>
__global__ __launch_bounds__(kThreads) void norm_kernel(const T * __restrict__ x, const T * __restrict__ d,
                                                        const void * __restrict__ w,
                                                        const void * __restrict__ b, bool p_f16,
                                                        T * h_out, T * y, int64_t rows, int dim, float eps) {
    constexpr bool kF16 = std::is_same<T, uint16_t>::value;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole wavefront leaves; no block barrier follows
    const T * xr = x + row * dim;
    const T * dr = d ? d + row * dim : nullptr;
    T * hr = h_out ? h_out + row * dim : nullptr;
    T * yr = y + row * dim;

    float h[NV][VEC];
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = (lane + 64 * j) * VEC;
        if (e < dim) {
            if constexpr (kF16) {
                uint16_t xv[VEC], hv[VEC];
                load_u16<VEC>(xr + e, xv);
                if (dr) {
                    uint16_t dv[VEC];
                    load_u16<VEC>(dr + e, dv);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) hv[k] = f2h(h2f(xv[k]) + h2f(dv[k]));
                } else {
#pragma unroll
                    for (int k = 0; k < VEC; ++k) hv[k] = xv[k];
                }
                if (hr) store_u16<VEC>(hr + e, hv);
#pragma unroll
                for (int k = 0; k < VEC; ++k) h[j][k] = h2f(hv[k]);
            } else {
                load_f32<VEC>(xr + e, h[j]);
                if (dr) {
                    float dv[VEC];
                    load_f32<VEC>(dr + e, dv);
#pragma unroll
                    for (int k = 0; k < VEC; ++k) h[j][k] = h[j][k] + dv[k];
                }
                if (hr) store_f32<VEC>(hr + e, h[j]);
            }
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                if constexpr (kLayer)
                    acc += static_cast<double>(h[j][k]);
                else
                    acc += static_cast<double>(h[j][k] * h[j][k]);
            }
        }
    }
    acc = wave_sum_f64(acc);

    float scale;
    float mean = 0.0f;
    if constexpr (kLayer) {
        mean = static_cast<float>(acc / static_cast<double>(dim));
        double acc2 = 0.0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int e = (lane + 64 * j) * VEC;
            if (e < dim) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) {
                    const float v = h[j][k] - mean;
                    h[j][k] = v;
                    acc2 += static_cast<double>(v * v);
                }
            }
        }
        acc2 = wave_sum_f64(acc2);
        const float variance = static_cast<float>(acc2 / static_cast<double>(dim));
        scale = 1.0f / sqrtf(variance + eps);
    } else {
        const float ms = static_cast<float>(acc / static_cast<double>(dim));
        scale = 1.0f / sqrtf(ms + eps);
    }

#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = (lane + 64 * j) * VEC;
        if (e < dim) {
            float wv[VEC];
            load_param<VEC>(w, p_f16, e, wv);
            float o[VEC];
            if constexpr (kLayer) {
                float bv[VEC];
                load_param<VEC>(b, p_f16, e, bv);
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[k] = ((h[j][k] * scale) * wv[k]) + bv[k];
            } else if constexpr (kF16) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[k] = h2f(f2h(h[j][k] * scale)) * wv[k];
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) o[k] = (h[j][k] * scale) * wv[k];
            }
            if constexpr (kF16) {
                uint16_t ov[VEC];
#pragma unroll
                for (int k = 0; k < VEC; ++k) ov[k] = f2h(o[k]);
                store_u16<VEC>(yr + e, ov);
            } else {
                store_f32<VEC>(yr + e, o);
            }
        }
    }
}

template <typename T, bool kLayer, int VEC>
int launch_nv(const T * x, const T * d, const void * w, const void * b, bool p_f16, T * h, T * y,
              int64_t rows, int dim, float eps, hipStream_t stream) {
    const int groups = static_cast<int>(ceil_div(dim, 64 * VEC));
    const int64_t grid = ceil_div(rows, kWaves);
    constexpr int kMaxNV = 8192 / (64 * VEC);
#define LEVO_NORM_CASE(NVV)                                                                           \
    if constexpr (NVV <= kMaxNV) {                                                                    \
        if (groups <= NVV) {                                                                          \
            norm_kernel<T, kLayer, VEC, NVV><<<grid, kThreads, 0, stream>>>(x, d, w, b, p_f16, h, y,  \
                                                                            rows, dim, eps);          \
            return launch_status("levo_hip_residual_norm");                                           \
        }                                                                                             \
    }
    LEVO_NORM_CASE(1)
    LEVO_NORM_CASE(2)
    LEVO_NORM_CASE(4)
    LEVO_NORM_CASE(8)
    LEVO_NORM_CASE(16)
    LEVO_NORM_CASE(32)
    LEVO_NORM_CASE(64)
    LEVO_NORM_CASE(128)
#undef LEVO_NORM_CASE
    set_error("residual norm: row length %d exceeds the supported 8192", dim);
    return LEVO_HIP_ERR_UNSUPPORTED;
}

template <typename T, bool kLayer>
int launch_norm(const void * x, const void * d, const void * w, const void * b, bool p_f16, void * h,
                void * y, int64_t rows, int64_t dim, float eps, hipStream_t stream) {
    constexpr int kVec = std::is_same<T, uint16_t>::value ? 8 : 4;
    const bool vec = dim % 8 == 0 && aligned16(x) && (d == nullptr || aligned16(d)) && aligned16(w) &&
                     (b == nullptr || aligned16(b)) && (h == nullptr || aligned16(h)) && aligned16(y);
    const T * xt = static_cast<const T *>(x);
    const T * dt = static_cast<const T *>(d);
    T * ht = static_cast<T *>(h);
    T * yt = static_cast<T *>(y);
    if (vec) return launch_nv<T, kLayer, kVec>(xt, dt, w, b, p_f16, ht, yt, rows, static_cast<int>(dim), eps, stream);
    return launch_nv<T, kLayer, 1>(xt, dt, w, b, p_f16, ht, yt, rows, static_cast<int>(dim), eps, stream);
}

int check_norm_args(levo_hip_type act, const void * x, const void * w, levo_hip_type pt, const void * y,
                    int64_t rows, int64_t dim, float eps) {
    LEVO_REQUIRE(act == LEVO_HIP_TYPE_F32 || act == LEVO_HIP_TYPE_F16,
                 "residual norm: activations must be F32 or F16");
    LEVO_REQUIRE(pt == LEVO_HIP_TYPE_F32 || pt == LEVO_HIP_TYPE_F16,
                 "residual norm: parameters must be F32 or F16");
    LEVO_REQUIRE(rows >= 0 && dim >= 0, "residual norm: negative shape");
    LEVO_REQUIRE(rows == 0 || dim > 0, "residual norm: empty rows");
    LEVO_REQUIRE(dim <= 8192, "residual norm: row length exceeds the supported 8192");
    LEVO_REQUIRE(eps >= 0.0f, "residual norm: eps must be non-negative");
    LEVO_REQUIRE(rows == 0 || (x != nullptr && w != nullptr && y != nullptr),
                 "residual norm: null input, parameter or output");
    return LEVO_HIP_OK;
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_residual_rms_norm(levo_hip_type act_type, const void * x, const void * delta,
                                          const void * weight, levo_hip_type weight_type, void * h_out,
                                          void * y, int64_t rows, int64_t dim, float eps,
                                          levo_hip_stream_t stream) {
    const int st = check_norm_args(act_type, x, weight, weight_type, y, rows, dim, eps);
    if (st != LEVO_HIP_OK) return st;
    if (rows == 0) return LEVO_HIP_OK;
    const bool p_f16 = weight_type == LEVO_HIP_TYPE_F16;
    if (act_type == LEVO_HIP_TYPE_F16) {
        LEVO_REQUIRE(p_f16, "residual RMSNorm: F16 activations take the F16 weight (src/levo-kv.cpp:159)");
        return launch_norm<uint16_t, false>(x, delta, weight, nullptr, p_f16, h_out, y, rows, dim, eps,
                                            as_hip(stream));
    }
    return launch_norm<float, false>(x, delta, weight, nullptr, p_f16, h_out, y, rows, dim, eps, as_hip(stream));
}

extern "C" int levo_hip_residual_layer_norm(levo_hip_type act_type, const void * x, const void * delta,
                                            const void * gamma, const void * beta, levo_hip_type param_type,
                                            void * h_out, void * y, int64_t rows, int64_t dim, float eps,
                                            levo_hip_stream_t stream) {
    const int st = check_norm_args(act_type, x, gamma, param_type, y, rows, dim, eps);
    if (st != LEVO_HIP_OK) return st;
    if (rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(beta != nullptr, "residual LayerNorm: beta is null");
    const bool p_f16 = param_type == LEVO_HIP_TYPE_F16;
    if (act_type == LEVO_HIP_TYPE_F16)
        return launch_norm<uint16_t, true>(x, delta, gamma, beta, p_f16, h_out, y, rows, dim, eps,
                                           as_hip(stream));
    return launch_norm<float, true>(x, delta, gamma, beta, p_f16, h_out, y, rows, dim, eps, as_hip(stream));
}
