// Fused residual add + RMSNorm / LayerNorm, one wave per row up to 2048
// elements (two or four waves for longer rows).
//
// Every load of the row (x, delta, weight, bias) is issued up front with
// dwordx4 accesses, the row stays in registers, is reduced with DPP cross-lane
// steps (plus one LDS exchange when several waves share the row), normalised
// and written once; row data is loaded and stored with streaming
// (nontemporal) accesses. The reduction accumulates in double like ggml-cpu's ggml_float
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
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

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

// Row loads and stores stream past the caches (each row is touched once);
// the parameters, shared by every row, are ordinary cached loads.
__device__ __forceinline__ void load8_row(const uint16_t * p, uint16_t (&o)[kVec]) {
    const u16x8 v = __builtin_nontemporal_load(reinterpret_cast<const u16x8 *>(p));
#pragma unroll
    for (int k = 0; k < kVec; ++k) o[k] = v[k];
}
__device__ __forceinline__ void store8_row(uint16_t * p, const uint16_t (&v)[kVec]) {
    u16x8 w;
#pragma unroll
    for (int k = 0; k < kVec; ++k) w[k] = v[k];
    __builtin_nontemporal_store(w, reinterpret_cast<u16x8 *>(p));
}

// F32 groups as two 4-value pieces (see norm_kernel_wg): parameters (cached),
// row values and their stores (streaming); a store of a piece past the row is
// left out.
__device__ __forceinline__ void load4x2(const float * p0, const float * p1, float (&o)[kVec]) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(p0);
    const f32x4 b = *reinterpret_cast<const f32x4 *>(p1);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void load4x2(const uint16_t * p0, const uint16_t * p1, float (&o)[kVec]) {
    const u16x4 a = *reinterpret_cast<const u16x4 *>(p0);
    const u16x4 b = *reinterpret_cast<const u16x4 *>(p1);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        o[k] = h2f(a[k]);
        o[k + 4] = h2f(b[k]);
    }
}
__device__ __forceinline__ void load4x2_row(const float * p0, const float * p1, float (&o)[kVec]) {
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p0));
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p1));
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void store4x2_row(float * p0, float * p1, const float (&v)[kVec], bool in0, bool in1) {
    if (in0) __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4 *>(p0));
    if (in1) __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f32x4 *>(p1));
}

// Sum in double of this lane's values (kSquare: of their F32 squares) over
// the groups in range, as a pairwise tree: the dependent chain is a few adds
// long instead of one per element. Any order differs from the CPU's
// sequential ggml_float sum; in double the difference stays near 2^-40 of the
// sum of magnitudes, far below the F32 rounding the result then takes.
template <int NV, bool kSquare>
__device__ __forceinline__ double lane_sum(const float (&h)[NV][kVec], const bool (&in)[NV]) {
    double g[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        double t[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) t[k] = static_cast<double>(kSquare ? h[j][k] * h[j][k] : h[j][k]);
#pragma unroll
        for (int w = kVec / 2; w >= 1; w /= 2) {
#pragma unroll
            for (int k = 0; k < w; ++k) t[k] = t[2 * k] + t[2 * k + 1];
        }
        g[j] = in[j] ? t[0] : 0.0;
    }
    double s = g[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) s += g[j];
    return s;
}

// Sum of v over the W waves of one row: DPP within the wave, then (W > 1)
// one LDS exchange, added in wave order.
template <int W>
__device__ __forceinline__ double row_sum(double v, double (*part)[4], int slot, int wave, int lane) {
    v = wave_sum_f64(v);
    if constexpr (W == 1) {
        return v;
    } else {
        if (lane == 0) part[slot][wave] = v;
        lds_barrier();
        double s = part[slot][0];
#pragma unroll
        for (int i = 1; i < W; ++i) s += part[slot][i];
        return s;
    }
}

// T: activation storage (uint16_t = F16, float); P: parameter storage.
// A 256-thread workgroup holds 4 / W rows, W waves per row; lane groups
// g = t + 64*W*j (t the thread's index within its row), NV groups of 8
// elements per lane (dim <= 512 * W * NV). A row of up to 2048 elements is one
// wave's: its sums need no LDS and no barrier.
// x / d may alias h_out or y (in-place residual): each element is loaded and
// stored by the same lane, loads first, so no __restrict__ on them.
template <typename T, typename P, bool kLayer, bool kDelta, int NV, int W>
__global__ __launch_bounds__(kThreads) void norm_kernel_wg(const T * x, const T * d, const P * __restrict__ w,
                                                           const P * __restrict__ b, T * h_out, T * y,
                                                           int64_t rows, int dim, float eps) {
    constexpr bool kF16 = std::is_same<T, uint16_t>::value;
    constexpr int kRows = 4 / W;
    __shared__ double part[2][kRows][4];
    const int t = threadIdx.x % (64 * W);
    const int slot = threadIdx.x / (64 * W);
    const int wave = t >> 6;
    const int lane = t & 63;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kRows + slot;
    // A slot past the last row computes on the last row and stores nothing, so
    // every wave reaches the barriers of its row.
    const bool valid = row0 < rows;
    const int64_t row = valid ? row0 : rows - 1;
    const T * xr = x + row * dim;
    const T * dr = kDelta ? d + row * dim : nullptr;
    T * hr = h_out ? h_out + row * dim : nullptr;
    T * yr = y + row * dim;
    // Group j of a lane: F16, 8 consecutive values (one 16-byte access per
    // lane, contiguous across the wave); F32, two pieces of 4 values 64 * W
    // pieces apart, so that each 16-byte access of the wave covers one
    // contiguous KiB (8 consecutive floats per lane would leave every access
    // at a 32-byte lane stride, two half-used cache lines per lane).
    bool in[NV], in2[NV];
    int off[NV], off2[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) {
            const int e = (t + 64 * W * j) * kVec;
            in[j] = e < dim;
            in2[j] = in[j];
            off[j] = in[j] ? e : 0;
            off2[j] = off[j] + 4;
        } else {
            const int e0 = (t + 64 * W * (2 * j)) * 4;
            const int e1 = (t + 64 * W * (2 * j + 1)) * 4;
            in[j] = e0 < dim;
            in2[j] = e1 < dim;
            off[j] = in[j] ? e0 : 0;
            off2[j] = in2[j] ? e1 : 0;
        }
    }
    float h[NV][kVec];
    float wv[NV][kVec];
    float bv[NV][kVec];
    T xb[NV][kVec], db[NV][kVec];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) {
            load8(w + off[j], wv[j]);
            if constexpr (kLayer) load8(b + off[j], bv[j]);
        } else {
            load4x2(w + off[j], w + off2[j], wv[j]);
            if constexpr (kLayer) load4x2(b + off[j], b + off2[j], bv[j]);
        }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) load8_row(xr + off[j], xb[j]);
        else load4x2_row(xr + off[j], xr + off2[j], xb[j]);
    }
    if constexpr (kDelta) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (kF16) load8_row(dr + off[j], db[j]);
            else load4x2_row(dr + off[j], dr + off2[j], db[j]);
        }
    }
    if constexpr (kDelta) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) {
                if constexpr (kF16) xb[j][k] = f2h(h2f(xb[j][k]) + h2f(db[j][k]));
                else xb[j][k] = xb[j][k] + db[j][k];
            }
        }
    }
    // a second piece past the row holds no value (F32; F16 groups are whole)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
        for (int k = 0; k < kVec; ++k) h[j][k] = k < 4 || in2[j] ? to_f32(xb[j][k]) : 0.0f;
    }
    double acc = lane_sum<NV, !kLayer>(h, in);
    // The residual is stored once every load has been consumed: stores share
    // the load counter on this GPU, so a later wait for a load would also wait
    // for these stores.
    if (hr && valid) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (kF16) {
                if (in[j]) store8_row(hr + off[j], xb[j]);
            } else {
                store4x2_row(hr + off[j], hr + off2[j], xb[j], in[j], in2[j]);
            }
        }
    }
    acc = row_sum<W>(acc, part[0], slot, wave, lane);
    float scale;
    if constexpr (kLayer) {
        const float mean = static_cast<float>(acc / static_cast<double>(dim));
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) h[j][k] = k < 4 || in2[j] ? h[j][k] - mean : 0.0f;
        }
        double acc2 = lane_sum<NV, true>(h, in);
        acc2 = row_sum<W>(acc2, part[1], slot, wave, lane);
        const float variance = static_cast<float>(acc2 / static_cast<double>(dim));
        scale = 1.0f / sqrtf(variance + eps);
    } else {
        const float ms = static_cast<float>(acc / static_cast<double>(dim));
        scale = 1.0f / sqrtf(ms + eps);
    }
    if (!valid) return;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float o[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k)
            o[k] = norm_out<T, kLayer>(h[j][k] * scale, wv[j][k], kLayer ? bv[j][k] : 0.0f);
        if constexpr (kF16) {
            if (in[j]) {
                uint16_t ob[kVec];
#pragma unroll
                for (int k = 0; k < kVec; ++k) ob[k] = f2h(o[k]);
                store8_row(yr + off[j], ob);
            }
        } else {
            store4x2_row(yr + off[j], yr + off2[j], o, in[j], in2[j]);
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
                     dim <= 64 * 4 * kVec * 4;
    if (vec) {
        // Many rows: one wave per row up to 1536 elements, four rows per
        // workgroup; a row of 1537-2048 elements over four waves (one group
        // of 8 per lane: at 756 x 2048 RMS 4.18 -> 3.85 us and LayerNorm
        // 4.77 -> 4.39 us against one wave per row; at 1536 elements four
        // waves leave a quarter of the lanes idle and gain nothing); two or
        // four waves for longer rows, except F32 rows of 2049-2560 elements
        // (the Flow estimator's 2200), one wave each (five groups per lane,
        // sums without LDS or barrier: 16.2 -> 15.8 us at 2000 x 2200). A
        // few rows (decode): four waves per row, so each lane's share and
        // chain stay short.
        const int groups = static_cast<int>(ceil_div(dim, 64 * kVec));
        constexpr bool kF32 = std::is_same<T, float>::value;
        const int wpr = rows < 512 ? 4 : groups <= 3 || (kF32 && groups == 5) ? 1 : groups == 4 ? 4 : groups <= 8 ? 2 : 4;
        const int nv = static_cast<int>(ceil_div(groups, wpr));
        const hipStream_t s = stream;
        const uint32_t grid_w = static_cast<uint32_t>(ceil_div(rows, 4 / wpr));
#define LEVO_NORM_LAUNCH(NV, W)                                                                            \
    do {                                                                                                   \
        if (d) norm_kernel_wg<T, P, kLayer, true, NV, W><<<grid_w, kThreads, 0, s>>>(x, d, w, b, h, y, rows, dim, eps); \
        else norm_kernel_wg<T, P, kLayer, false, NV, W><<<grid_w, kThreads, 0, s>>>(x, d, w, b, h, y, rows, dim, eps); \
    } while (0)
        if (wpr == 1) {
            if (nv == 1) LEVO_NORM_LAUNCH(1, 1);
            else if (nv == 2) LEVO_NORM_LAUNCH(2, 1);
            else if (nv == 3) LEVO_NORM_LAUNCH(3, 1);
            else if (nv == 5) LEVO_NORM_LAUNCH(5, 1);
            else LEVO_NORM_LAUNCH(4, 1);
        } else if (wpr == 2) {
            if (nv == 3) LEVO_NORM_LAUNCH(3, 2);  // 2049-3072 elements: no idle fourth group of registers
            else LEVO_NORM_LAUNCH(4, 2);
        } else {
            if (nv == 1) LEVO_NORM_LAUNCH(1, 4);
            else if (nv == 2) LEVO_NORM_LAUNCH(2, 4);
            else LEVO_NORM_LAUNCH(4, 4);
        }
#undef LEVO_NORM_LAUNCH
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
