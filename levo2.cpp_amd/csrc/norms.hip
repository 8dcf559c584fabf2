// Fused residual add + RMSNorm / LayerNorm, one 4-wave workgroup per row.
//
// Every load of the row (x, delta, weight, bias) is issued up front with
// dwordx4 accesses, the row stays in registers, is reduced with DPP cross-lane
// steps and one LDS exchange between the four waves, normalised and
// written once. The reduction accumulates in double like ggml-cpu's ggml_float
// row sums, so the F32 mean / variance (and hence every rounding point after
// it) matches the CPU chain.
//
//   RMSNorm F16 (src/levo-kv.cpp:153-160, residual :462/:507):
//     h = f16(x + d); n = f16(h * 1/sqrtf(mean(h^2) + eps)); y = f16(n * w)
//   RMSNorm F32 (src/levo-lm.cpp:131-137): h = x + d; y = (h * scale) * w
//   LayerNorm  (src/levo-flow-estimator.cpp:106-109, residual :221-227):
//     h = x + d; v = h - mean; scale = 1/sqrtf(mean(v^2) + eps);
//     y = ((v * scale) * gamma) + beta   (F16 storage: h and y rounded to F16)
//
// Rows whose length is not a multiple of 8, longer than 8192, or unaligned
// buffers take a loop kernel (one wave per row) that reads the row from L2
// again per pass.
#include "common.hpp"

#include <type_traits>

namespace levo_hip {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kVec = 8;  // elements per lane per group (16 B of F16, 32 B of F32)
constexpr int kRowWaves = 4;  // waves sharing one row in the vector kernel

template <typename T>
__device__ __forceinline__ void load8(const T * p, float (&o)[kVec]);
template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t * p, float (&o)[kVec]) {
    const u16x8 v = *reinterpret_cast<const u16x8 *>(p);
#pragma unroll
    for (int k = 0; k < kVec; ++k) o[k] = h2f(v[k]);
}
template <>
__device__ __forceinline__ void load8<float>(const float * p, float (&o)[kVec]) {
    const f32x4 a = reinterpret_cast<const f32x4 *>(p)[0];
    const f32x4 b = reinterpret_cast<const f32x4 *>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}

// Raw F16 bits are kept for the residual (h = f16(x + d) is formed from them).
__device__ __forceinline__ void load8_raw(const uint16_t * p, uint16_t (&o)[kVec]) {
    const u16x8 v = *reinterpret_cast<const u16x8 *>(p);
#pragma unroll
    for (int k = 0; k < kVec; ++k) o[k] = v[k];
}

__device__ __forceinline__ void store8(uint16_t * p, const float (&v)[kVec]) {
    u16x8 w;
#pragma unroll
    for (int k = 0; k < kVec; ++k) w[k] = f2h(v[k]);
    *reinterpret_cast<u16x8 *>(p) = w;
}
__device__ __forceinline__ void store8_bits(uint16_t * p, const uint16_t (&v)[kVec]) {
    u16x8 w;
#pragma unroll
    for (int k = 0; k < kVec; ++k) w[k] = v[k];
    *reinterpret_cast<u16x8 *>(p) = w;
}
__device__ __forceinline__ void store8(float * p, const float (&v)[kVec]) {
    f32x4 a, b;
    a.x = v[0]; a.y = v[1]; a.z = v[2]; a.w = v[3];
    b.x = v[4]; b.y = v[5]; b.z = v[6]; b.w = v[7];
    reinterpret_cast<f32x4 *>(p)[0] = a;
    reinterpret_cast<f32x4 *>(p)[1] = b;
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) {
    if constexpr (std::is_same<T, uint16_t>::value) return h2f(v);
    else return v;
}

// Output rounding of the chains above, given the normalised value n.
template <typename T, bool kLayer>
__device__ __forceinline__ float norm_out(float n, float w, float b) {
    if constexpr (kLayer) return (n * w) + b;
    else if constexpr (std::is_same<T, uint16_t>::value) return h2f(f2h(n)) * w;  // cast_f16 then mul
    else return n * w;
}

// T: activation storage (uint16_t = F16, float); P: parameter storage.
// One row per workgroup of W waves; lane groups g = tid + 64*W*j, NV groups of
// 8 elements per lane (dim <= 512 * W * NV). The wave sums meet in LDS and are
// added in wave order.
// x / d may alias h_out or y (in-place residual): each element is loaded and
// stored by the same lane, loads first, so no __restrict__ on them.
template <typename T, typename P, bool kLayer, int NV, int W>
__global__ __launch_bounds__(64 * W) void norm_kernel_wg(const T * x, const T * d, const P * __restrict__ w,
                                                         const P * __restrict__ b, T * h_out, T * y,
                                                         int64_t rows, int dim, float eps) {
    constexpr bool kF16 = std::is_same<T, uint16_t>::value;
    __shared__ double part[2][W];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const T * xr = x + row * dim;
    const T * dr = d ? d + row * dim : nullptr;
    T * hr = h_out ? h_out + row * dim : nullptr;
    T * yr = y + row * dim;
    bool in[NV];
    int off[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int e = (tid + 64 * W * j) * kVec;
        in[j] = e < dim;
        off[j] = in[j] ? e : 0;
    }
    float h[NV][kVec];
    float wv[NV][kVec];
    float bv[NV][kVec];
    uint16_t xb[NV][kVec], db[NV][kVec];
    float df[NV][kVec];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) load8_raw(xr + off[j], xb[j]);
        else load8(xr + off[j], h[j]);
    }
    if (dr) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (kF16) load8_raw(dr + off[j], db[j]);
            else load8(dr + off[j], df[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        load8(w + off[j], wv[j]);
        if constexpr (kLayer) load8(b + off[j], bv[j]);
    }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) {
            uint16_t hb[kVec];
#pragma unroll
            for (int k = 0; k < kVec; ++k) hb[k] = dr ? f2h(h2f(xb[j][k]) + h2f(db[j][k])) : xb[j][k];
            if (hr && in[j]) store8_bits(hr + off[j], hb);
#pragma unroll
            for (int k = 0; k < kVec; ++k) h[j][k] = h2f(hb[k]);
        } else {
            if (dr) {
#pragma unroll
                for (int k = 0; k < kVec; ++k) h[j][k] = h[j][k] + df[j][k];
            }
            if (hr && in[j]) store8(hr + off[j], h[j]);
        }
        if (in[j]) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) {
                if constexpr (kLayer) acc += static_cast<double>(h[j][k]);
                else acc += static_cast<double>(h[j][k] * h[j][k]);
            }
        }
    }
    acc = wave_sum_f64(acc);
    if ((tid & 63) == 0) part[0][wave] = acc;
    __syncthreads();
    acc = part[0][0];
#pragma unroll
    for (int i = 1; i < W; ++i) acc += part[0][i];
    float scale;
    if constexpr (kLayer) {
        const float mean = static_cast<float>(acc / static_cast<double>(dim));
        double acc2 = 0.0;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) {
                const float v = h[j][k] - mean;
                h[j][k] = v;
                if (in[j]) acc2 += static_cast<double>(v * v);
            }
        }
        acc2 = wave_sum_f64(acc2);
        if ((tid & 63) == 0) part[1][wave] = acc2;
        __syncthreads();
        acc2 = part[1][0];
#pragma unroll
        for (int i = 1; i < W; ++i) acc2 += part[1][i];
        const float variance = static_cast<float>(acc2 / static_cast<double>(dim));
        scale = 1.0f / sqrtf(variance + eps);
    } else {
        const float ms = static_cast<float>(acc / static_cast<double>(dim));
        scale = 1.0f / sqrtf(ms + eps);
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (in[j]) {
            float o[kVec];
#pragma unroll
            for (int k = 0; k < kVec; ++k)
                o[k] = norm_out<T, kLayer>(h[j][k] * scale, wv[j][k], kLayer ? bv[j][k] : 0.0f);
            store8(yr + off[j], o);
        }
    }
}

// Any dim / alignment: the wave loops over its row, re-reading it per pass.
// Each element is read and written by the same lane, reads first, so the
// residual may be written in place.
template <typename T, typename P, bool kLayer>
__global__ __launch_bounds__(kThreads) void norm_kernel_loop(const T * x, const T * d, const P * __restrict__ w,
                                                             const P * __restrict__ b, T * h_out, T * y,
                                                             int64_t rows, int dim, float eps) {
    constexpr bool kF16 = std::is_same<T, uint16_t>::value;
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T * xr = x + row * dim;
    const T * dr = d ? d + row * dim : nullptr;
    T * hr = h_out ? h_out + row * dim : nullptr;
    T * yr = y + row * dim;
    auto residual = [&](int e) -> float {
        if constexpr (kF16) return dr ? h2f(f2h(h2f(xr[e]) + h2f(dr[e]))) : h2f(xr[e]);
        else return dr ? xr[e] + dr[e] : xr[e];
    };
    double acc = 0.0;
    for (int e = lane; e < dim; e += 64) {
        const float h = residual(e);
        if constexpr (kLayer) acc += static_cast<double>(h);
        else acc += static_cast<double>(h * h);
    }
    acc = wave_sum_f64(acc);
    float scale, mean = 0.0f;
    if constexpr (kLayer) {
        mean = static_cast<float>(acc / static_cast<double>(dim));
        double acc2 = 0.0;
        for (int e = lane; e < dim; e += 64) {
            const float v = residual(e) - mean;
            acc2 += static_cast<double>(v * v);
        }
        acc2 = wave_sum_f64(acc2);
        scale = 1.0f / sqrtf(static_cast<float>(acc2 / static_cast<double>(dim)) + eps);
    } else {
        scale = 1.0f / sqrtf(static_cast<float>(acc / static_cast<double>(dim)) + eps);
    }
    for (int e = lane; e < dim; e += 64) {
        const float h = residual(e);
        const float n = kLayer ? (h - mean) * scale : h * scale;
        const float o = norm_out<T, kLayer>(n, to_f32(w[e]), kLayer ? to_f32(b[e]) : 0.0f);
        if (hr) {
            if constexpr (kF16) hr[e] = f2h(h);
            else hr[e] = h;
        }
        if constexpr (kF16) yr[e] = f2h(o);
        else yr[e] = o;
    }
}

template <typename T, typename P, bool kLayer>
int launch_norm(const void * xv, const void * dv, const void * wv, const void * bv, void * hv, void * yv,
                int64_t rows, int64_t dim64, float eps, hipStream_t stream) {
    const T * x = static_cast<const T *>(xv);
    const T * d = static_cast<const T *>(dv);
    const P * w = static_cast<const P *>(wv);
    const P * b = static_cast<const P *>(bv);
    T * h = static_cast<T *>(hv);
    T * y = static_cast<T *>(yv);
    const int dim = static_cast<int>(dim64);
    const int64_t grid = ceil_div(rows, kWaves);
    const bool vec = dim % kVec == 0 && aligned16(x) && (d == nullptr || aligned16(d)) && aligned16(w) &&
                     (b == nullptr || aligned16(b)) && (h == nullptr || aligned16(h)) && aligned16(y) &&
                     dim <= 64 * kRowWaves * kVec * 4;
    if (vec) {
        // One row per 4-wave workgroup: 8 values per lane at dim 2048, so the
        // per-lane chain load -> reduce -> store is short and every CU gets rows.
        constexpr int W = kRowWaves;
        const int groups = static_cast<int>(ceil_div(dim, 64 * W * kVec));
        const hipStream_t s = stream;
        if (groups <= 1) norm_kernel_wg<T, P, kLayer, 1, W><<<rows, 64 * W, 0, s>>>(x, d, w, b, h, y, rows, dim, eps);
        else if (groups <= 2) norm_kernel_wg<T, P, kLayer, 2, W><<<rows, 64 * W, 0, s>>>(x, d, w, b, h, y, rows, dim, eps);
        else norm_kernel_wg<T, P, kLayer, 4, W><<<rows, 64 * W, 0, s>>>(x, d, w, b, h, y, rows, dim, eps);
        return launch_status("levo_hip_residual_norm");
    }
    norm_kernel_loop<T, P, kLayer><<<grid, kThreads, 0, stream>>>(x, d, w, b, h, y, rows, dim, eps);
    return launch_status("levo_hip_residual_norm");
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
    LEVO_REQUIRE(rows < (int64_t{1} << 31), "residual norm: too many rows");
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
    const hipStream_t s = as_hip(stream);
    if (act_type == LEVO_HIP_TYPE_F16) {
        LEVO_REQUIRE(weight_type == LEVO_HIP_TYPE_F16,
                     "residual RMSNorm: F16 activations take the F16 weight (src/levo-kv.cpp:159)");
        return launch_norm<uint16_t, uint16_t, false>(x, delta, weight, nullptr, h_out, y, rows, dim, eps, s);
    }
    if (weight_type == LEVO_HIP_TYPE_F16)
        return launch_norm<float, uint16_t, false>(x, delta, weight, nullptr, h_out, y, rows, dim, eps, s);
    return launch_norm<float, float, false>(x, delta, weight, nullptr, h_out, y, rows, dim, eps, s);
}

extern "C" int levo_hip_residual_layer_norm(levo_hip_type act_type, const void * x, const void * delta,
                                            const void * gamma, const void * beta, levo_hip_type param_type,
                                            void * h_out, void * y, int64_t rows, int64_t dim, float eps,
                                            levo_hip_stream_t stream) {
    const int st = check_norm_args(act_type, x, gamma, param_type, y, rows, dim, eps);
    if (st != LEVO_HIP_OK) return st;
    if (rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(beta != nullptr, "residual LayerNorm: beta is null");
    const hipStream_t s = as_hip(stream);
    const bool p16 = param_type == LEVO_HIP_TYPE_F16;
    if (act_type == LEVO_HIP_TYPE_F16)
        return p16 ? launch_norm<uint16_t, uint16_t, true>(x, delta, gamma, beta, h_out, y, rows, dim, eps, s)
                   : launch_norm<uint16_t, float, true>(x, delta, gamma, beta, h_out, y, rows, dim, eps, s);
    return p16 ? launch_norm<float, uint16_t, true>(x, delta, gamma, beta, h_out, y, rows, dim, eps, s)
               : launch_norm<float, float, true>(x, delta, gamma, beta, h_out, y, rows, dim, eps, s);
}
