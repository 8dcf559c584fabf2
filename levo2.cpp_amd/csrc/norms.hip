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

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Two F16 residual adds in one packed instruction. The reference rounds
// f32(x) + f32(d) to F32 and then to F16; an F16 add rounds the exact sum once.
// The two agree: F32 carries 24 >= 2 * 11 + 2 significand bits, and rounding
// first to such a format and then to the 11-bit one gives the correctly
// rounded sum (Figueroa, "When is double rounding innocuous?", 1995).
__device__ __forceinline__ uint32_t add_f16x2(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) + __builtin_bit_cast(f16x2, b));
}

// Row loads and stores stream past the caches (each row is touched once);
// the parameters, shared by every row, are ordinary cached loads.
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

// Sum in double of one group's 8 values (kSquare: of their F32 squares) as a
// pairwise tree, 0 for a group past the row.
template <bool kSquare>
__device__ __forceinline__ double group_sum8(const float (&h)[kVec], bool in) {
    double t[kVec];
#pragma unroll
    for (int k = 0; k < kVec; ++k) t[k] = static_cast<double>(kSquare ? h[k] * h[k] : h[k]);
#pragma unroll
    for (int w = kVec / 2; w >= 1; w /= 2) {
#pragma unroll
        for (int k = 0; k < w; ++k) t[k] = t[2 * k] + t[2 * k + 1];
    }
    return in ? t[0] : 0.0;
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

// lane_sum for F32 groups of two 4-value pieces, each masked as a whole.
template <int NV, bool kSquare>
__device__ __forceinline__ double lane_sum_pieces(const float (&h)[NV][kVec], const bool (&in)[NV],
                                                  const bool (&in2)[NV]) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        double t[kVec];
#pragma unroll
        for (int k = 0; k < kVec; ++k) t[k] = static_cast<double>(kSquare ? h[j][k] * h[j][k] : h[j][k]);
        const double p0 = (t[0] + t[1]) + (t[2] + t[3]);
        const double p1 = (t[4] + t[5]) + (t[6] + t[7]);
        s += (in[j] ? p0 : 0.0) + (in2[j] ? p1 : 0.0);
    }
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
template <typename T, typename P, bool kLayer, bool kDelta, int NV, int W, int R>
__global__ __launch_bounds__(64 * W * R) void norm_kernel_wg(const T * x, const T * d, const P * __restrict__ w,
                                                           const P * __restrict__ b, T * h_out, T * y,
                                                           int64_t rows, int dim, float eps) {
    constexpr bool kF16 = std::is_same<T, uint16_t>::value;
    constexpr int kRows = R;
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
    T xb[NV][kVec], db[NV][kVec];  // F32 rows
    u32x4 xw[NV], dw[NV];          // F16 rows: 8 halves as 4 packed dwords
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
    // F16 rows: x and delta of group j requested together, so that group j
    // is complete while later groups are still in flight (its residual,
    // widening and partial sum run then, below)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) {
            xw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(xr + off[j]));
            if constexpr (kDelta) dw[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(dr + off[j]));
        } else {
            load4x2_row(xr + off[j], xr + off2[j], xb[j]);
        }
    }
    if constexpr (kDelta && !kF16) {
#pragma unroll
        for (int j = 0; j < NV; ++j) load4x2_row(dr + off[j], dr + off2[j], db[j]);
    }
    // every load is issued before any loaded value is used (the scheduler
    // would otherwise start converting the first parameters, and wait for
    // them, before requesting the row)
    __builtin_amdgcn_sched_barrier(0);
    // The parameters (cached, first to arrive) are converted while the row is
    // in flight, and no load is waited for after the residual store below.
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        consume_now(wv[j]);
        if constexpr (kLayer) consume_now(bv[j]);
    }
    // Residual, widening and the first pass's per-group sums, group by group
    // in the order the loads were requested (F16: each group as soon as its
    // x and delta are in).
    double gsum[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if constexpr (kF16) {
            if constexpr (kDelta) {
#pragma unroll
                for (int i = 0; i < kVec / 2; ++i) xw[j][i] = add_f16x2(xw[j][i], dw[j][i]);
            }
#pragma unroll
            for (int k = 0; k < kVec; ++k) h[j][k] = h2f(static_cast<uint16_t>(xw[j][k / 2] >> (16 * (k & 1))));
            gsum[j] = group_sum8<!kLayer>(h[j], in[j]);
            // group j's work stays ahead of the wait for group j + 1: its sum
            // is pinned here (an empty asm with no memory clobber) and the
            // scheduler may not move group j + 1 above this point
            asm volatile("" : "+v"(gsum[j]));
            __builtin_amdgcn_sched_barrier(0);
        } else {
            if constexpr (kDelta) {
#pragma unroll
                for (int k = 0; k < kVec; ++k) xb[j][k] = xb[j][k] + db[j][k];
            }
        }
    }
    // The whole row is in registers before the residual store. A second F32
    // piece past the row holds no value; an F16 group past the row is left out
    // of the sums.
    if constexpr (kF16) {
        consume_now(xw);
    } else {
#pragma unroll
        for (int j = 0; j < NV; ++j) consume_now(xb[j]);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
#pragma unroll
            for (int k = 0; k < kVec; ++k) h[j][k] = k < 4 || in2[j] ? xb[j][k] : 0.0f;
            gsum[j] = group_sum8<!kLayer>(h[j], in[j]);
        }
    }
    double acc = gsum[0];
#pragma unroll
    for (int j = 1; j < NV; ++j) acc += gsum[j];
    // The residual is stored once every load has been consumed: stores share
    // the load counter on this GPU, so a later wait for a load would also wait
    // for these stores.
    if (hr && valid) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (kF16) {
                if (in[j]) __builtin_nontemporal_store(xw[j], reinterpret_cast<u32x4 *>(hr + off[j]));
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
            for (int k = 0; k < kVec; ++k) h[j][k] = kF16 || k < 4 || in2[j] ? h[j][k] - mean : 0.0f;
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
        // A row of one wave: fewer rows than four per CU (756 x 1536) take one
        // row per workgroup, so they reach all 256 CUs (four one-wave rows per
        // workgroup left 67 CUs idle: RMS 3.6-3.8 -> 3.56 us, LayerNorm 3.93 ->
        // 3.83 us); more rows keep four per workgroup (2000 x 2200 F32: 14.9
        // against 15.2-15.5 us for one per workgroup).
        const bool one_row_wg = wpr == 1 && rows < 4 * 256;
        const uint32_t grid_w = static_cast<uint32_t>(one_row_wg ? rows : ceil_div(rows, 4 / wpr));
#define LEVO_NORM_LAUNCH(NV, W, R)                                                                          \
    do {                                                                                                    \
        if (d) norm_kernel_wg<T, P, kLayer, true, NV, W, R><<<grid_w, 64 * W * R, 0, s>>>(x, d, w, b, h, y, rows, dim, eps); \
        else norm_kernel_wg<T, P, kLayer, false, NV, W, R><<<grid_w, 64 * W * R, 0, s>>>(x, d, w, b, h, y, rows, dim, eps); \
    } while (0)
        if (wpr == 1 && one_row_wg) {
            if (nv == 1) LEVO_NORM_LAUNCH(1, 1, 1);
            else if (nv == 2) LEVO_NORM_LAUNCH(2, 1, 1);
            else if (nv == 3) LEVO_NORM_LAUNCH(3, 1, 1);
            else if (nv == 5) LEVO_NORM_LAUNCH(5, 1, 1);
            else LEVO_NORM_LAUNCH(4, 1, 1);
        } else if (wpr == 1) {
            if (nv == 1) LEVO_NORM_LAUNCH(1, 1, 4);
            else if (nv == 2) LEVO_NORM_LAUNCH(2, 1, 4);
            else if (nv == 3) LEVO_NORM_LAUNCH(3, 1, 4);
            else if (nv == 5) LEVO_NORM_LAUNCH(5, 1, 4);
            else LEVO_NORM_LAUNCH(4, 1, 4);
        } else if (wpr == 2) {
            if (nv == 3) LEVO_NORM_LAUNCH(3, 2, 2);  // 2049-3072 elements: no idle fourth group of registers
            else LEVO_NORM_LAUNCH(4, 2, 2);
        } else {
            if (nv == 1) LEVO_NORM_LAUNCH(1, 4, 1);
            else if (nv == 2) LEVO_NORM_LAUNCH(2, 4, 1);
            else LEVO_NORM_LAUNCH(4, 4, 1);
        }
#undef LEVO_NORM_LAUNCH
        return launch_status("levo_hip_residual_norm");
    }
    norm_kernel_loop<T, P, kLayer><<<grid, kThreads, 0, stream>>>(x, d, w, b, h, y, rows, dim, eps);
    return launch_status("levo_hip_residual_norm");
}

// ---- gated residual + LayerNorm + AdaLN modulation (Flow estimator) --------
//
//   h = (delta * gate) + x;  t = (norm(h) * gamma) + beta;  y = (t * (scale + 1)) + shift
//
// with gate, scale and shift per batch entry (modulation_chunk: dynamic[b] +
// learned). A 256-thread workgroup takes four rows (one wave each) of one
// batch entry. Its threads stage that entry's vectors once in LDS: gate,
// gamma, beta, scale + 1 and shift, each its one rounding as the graph
// computes it. Every row then reads them from LDS where it uses them, so the
// row itself (x, delta and h) is all a wave holds in registers. The staging
// loads (cached) are issued before the row loads (streaming) and waited for
// on their own; every row load is consumed before the first store.

struct bvec {
    const float * dyn;
    int64_t stride;
    const float * learned;
};

struct mod_norm_params {
    const float * x;
    const float * d;
    bvec gate, scale, shift;
    const void * gamma;
    const void * beta;
    float * h_out;
    float * y;
    int64_t rows_per_batch;
    int wg_per_batch;
    int dim;
    float eps;
};

template <typename P>
__device__ __forceinline__ f32x4 load_param4(const void * base, int q) {
    if constexpr (std::is_same<P, float>::value) {
        return reinterpret_cast<const f32x4 *>(base)[q];
    } else {
        const u16x4 v = reinterpret_cast<const u16x4 *>(base)[q];
        return f32x4{h2f(v[0]), h2f(v[1]), h2f(v[2]), h2f(v[3])};
    }
}

// The dynamic and learned parts of a vector's piece q of batch entry b (the
// learned load re-reads the dynamic piece when there is no learned part, so
// the loads are unconditional and every wait count stays exact).
__device__ __forceinline__ void load_bvec(const bvec & v, int64_t b, int q, f32x4 & dyn, f32x4 & learned) {
    const f32x4 * d = reinterpret_cast<const f32x4 *>(v.dyn + b * v.stride);
    dyn = d[q];
    learned = v.learned ? reinterpret_cast<const f32x4 *>(v.learned)[q] : d[q];
}

template <typename P, int NV, bool kDelta, bool kGate, bool kMod>
__global__ __launch_bounds__(256) void mod_norm_kernel(mod_norm_params p) {
    constexpr int kStage = (NV + 1) / 2;  // pieces of 4 a thread stages: 128 * NV per row / 256 threads
    // Each staged vector spans the 128 * NV pieces a row's lanes address, so
    // LDS reads need no clamp; pieces past the row are never staged and their
    // values are never stored.
    constexpr int kSpan = 128 * NV;
    extern __shared__ f32x4 stage[];
    const int nq = p.dim >> 2;
    f32x4 * s_gate = stage;
    f32x4 * s_gamma = stage + (kGate ? kSpan : 0);
    f32x4 * s_beta = s_gamma + kSpan;
    f32x4 * s_ops = s_beta + kSpan;
    f32x4 * s_shift = s_ops + kSpan;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t batch = blockIdx.x / p.wg_per_batch;
    const int64_t local = static_cast<int64_t>(blockIdx.x % p.wg_per_batch) * 4 + wave;
    // A wave past its batch entry's rows computes on the entry's last row and
    // stores nothing.
    const bool valid = local < p.rows_per_batch;
    const int64_t row = batch * p.rows_per_batch + (valid ? local : p.rows_per_batch - 1);

    // 1. staging loads: piece q of each vector, clamped into the row
    f32x4 gd[kStage], gl[kStage], ga[kStage], be[kStage], sd[kStage], sl[kStage], hd[kStage], hl[kStage];
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int q = min(static_cast<int>(threadIdx.x) + 256 * i, nq - 1);
        if constexpr (kGate) load_bvec(p.gate, batch, q, gd[i], gl[i]);
        ga[i] = load_param4<P>(p.gamma, q);
        be[i] = load_param4<P>(p.beta, q);
        if constexpr (kMod) {
            load_bvec(p.scale, batch, q, sd[i], sl[i]);
            load_bvec(p.shift, batch, q, hd[i], hl[i]);
        }
    }
    asm volatile("" ::: "memory");  // the row loads below are issued after these

    // 2. row loads: group j is pieces lane + 128 j and lane + 128 j + 64, so
    // each 16-byte access of the wave covers one contiguous KiB
    const float * xr = p.x + row * p.dim;
    const float * dr = kDelta ? p.d + row * p.dim : nullptr;
    bool in[NV], in2[NV];
    int q0[NV], q1[NV];
    float xb[NV][kVec], db[NV][kVec];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int a = lane + 128 * j, b = a + 64;
        in[j] = a < nq;
        in2[j] = b < nq;
        q0[j] = in[j] ? a : 0;
        q1[j] = in2[j] ? b : 0;
        load4x2_row(xr + 4 * q0[j], xr + 4 * q1[j], xb[j]);
        if constexpr (kDelta) load4x2_row(dr + 4 * q0[j], dr + 4 * q1[j], db[j]);
    }

    // 3. stage the vectors (waits for the staging loads only)
    consume_now(ga);
    consume_now(be);
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int q = static_cast<int>(threadIdx.x) + 256 * i;
        f32x4 g, ops, sh;
        if constexpr (kGate) g = p.gate.learned ? gd[i] + gl[i] : gd[i];  // ggml_add(dynamic, learned)
        if constexpr (kMod) {
            ops = (p.scale.learned ? sd[i] + sl[i] : sd[i]) + 1.0f;      // ggml_scale_bias(scale, 1, 1)
            sh = p.shift.learned ? hd[i] + hl[i] : hd[i];
        }
        if (q < nq) {
            if constexpr (kGate) s_gate[q] = g;
            s_gamma[q] = ga[i];
            s_beta[q] = be[i];
            if constexpr (kMod) {
                s_ops[q] = ops;
                s_shift[q] = sh;
            }
        }
    }
    lds_barrier();

    // 4. residual: h = (delta * gate) + x, or x + delta
    if constexpr (kDelta) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            if constexpr (kGate) {
                const f32x4 g0 = s_gate[lane + 128 * j], g1 = s_gate[lane + 128 * j + 64];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    xb[j][k] = (db[j][k] * g0[k]) + xb[j][k];
                    xb[j][k + 4] = (db[j][k + 4] * g1[k]) + xb[j][k + 4];
                }
            } else {
#pragma unroll
                for (int k = 0; k < kVec; ++k) xb[j][k] = xb[j][k] + db[j][k];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < NV; ++j) consume_now(xb[j]);  // the whole row has arrived before any store
    float * hr = p.h_out ? p.h_out + row * p.dim : nullptr;
    if (hr && valid) {
#pragma unroll
        for (int j = 0; j < NV; ++j) store4x2_row(hr + 4 * q0[j], hr + 4 * q1[j], xb[j], in[j], in2[j]);
    }

    // 5. LayerNorm statistics, as norm_kernel_wg (pieces past the row left out
    // of the sums)
    float h[NV][kVec];
    const double acc = wave_sum_f64(lane_sum_pieces<NV, false>(xb, in, in2));
    const float mean = static_cast<float>(acc / static_cast<double>(p.dim));
#pragma unroll
    for (int j = 0; j < NV; ++j) {
#pragma unroll
        for (int k = 0; k < kVec; ++k) h[j][k] = xb[j][k] - mean;
    }
    const double acc2 = wave_sum_f64(lane_sum_pieces<NV, true>(h, in, in2));
    const float scale = 1.0f / sqrtf(static_cast<float>(acc2 / static_cast<double>(p.dim)) + p.eps);
    if (!valid) return;

    // 6. output: ((v * scale) * gamma) + beta, then * (scale + 1) + shift
    float * yr = p.y + row * p.dim;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        float o[kVec];
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int q = lane + 128 * j + 64 * half;
            const f32x4 gm = s_gamma[q], bt = s_beta[q];
            f32x4 op, sh;
            if constexpr (kMod) {
                op = s_ops[q];
                sh = s_shift[q];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float t = ((h[j][4 * half + k] * scale) * gm[k]) + bt[k];
                if constexpr (kMod) t = (t * op[k]) + sh[k];
                o[4 * half + k] = t;
            }
        }
        store4x2_row(yr + 4 * q0[j], yr + 4 * q1[j], o, in[j], in2[j]);
    }
}

template <typename P, int NV, bool kDelta, bool kGate, bool kMod>
int launch_mod_norm(const mod_norm_params & p, uint32_t grid, int lds_bytes, hipStream_t stream) {
    const auto kernel = mod_norm_kernel<P, NV, kDelta, kGate, kMod>;
    if (lds_bytes > 64 * 1024) {
        if (const int st = allow_dynamic_lds(reinterpret_cast<const void *>(kernel), lds_bytes,
                                             "levo_hip_residual_layer_norm_modulated");
            st != LEVO_HIP_OK)
            return st;
    }
    kernel<<<grid, 256, lds_bytes, stream>>>(p);
    return launch_status("levo_hip_residual_layer_norm_modulated");
}

template <typename P, int NV>
int launch_mod_norm_nv(const mod_norm_params & p, bool delta, bool gate, bool mod, uint32_t grid, int lds,
                       hipStream_t s) {
    if (gate) return mod ? launch_mod_norm<P, NV, true, true, true>(p, grid, lds, s)
                         : launch_mod_norm<P, NV, true, true, false>(p, grid, lds, s);
    if (delta) return mod ? launch_mod_norm<P, NV, true, false, true>(p, grid, lds, s)
                          : launch_mod_norm<P, NV, true, false, false>(p, grid, lds, s);
    return mod ? launch_mod_norm<P, NV, false, false, true>(p, grid, lds, s)
               : launch_mod_norm<P, NV, false, false, false>(p, grid, lds, s);
}

template <typename P>
int launch_mod_norm_p(const mod_norm_params & p, bool delta, bool gate, bool mod, uint32_t grid, int lds,
                      hipStream_t s) {
    if (p.dim <= 1024) return launch_mod_norm_nv<P, 2>(p, delta, gate, mod, grid, lds, s);
    if (p.dim <= 2560) return launch_mod_norm_nv<P, 5>(p, delta, gate, mod, grid, lds, s);
    return launch_mod_norm_nv<P, 8>(p, delta, gate, mod, grid, lds, s);
}

bool bvec_ok(const levo_hip_batch_vector & v, int64_t dim) {
    return v.dynamic == nullptr ||
           (v.stride >= dim && v.stride % 4 == 0 && aligned16(v.dynamic) && (v.learned == nullptr || aligned16(v.learned)));
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
    // 64 work-items per row, and a launch counts its work-items in 32 bits
    LEVO_REQUIRE(rows < (int64_t{1} << 26), "residual norm: too many rows");
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

extern "C" int levo_hip_residual_layer_norm_modulated(const levo_hip_modulated_norm_args * args,
                                                      levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "modulated norm: null argument block");
    const levo_hip_modulated_norm_args & a = *args;
    LEVO_REQUIRE(a.rows >= 0 && a.dim >= 0, "modulated norm: negative shape");
    if (a.rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(a.x != nullptr && a.y != nullptr && a.gamma != nullptr && a.beta != nullptr,
                 "modulated norm: null input, parameter or output");
    LEVO_REQUIRE(a.param_type == LEVO_HIP_TYPE_F32 || a.param_type == LEVO_HIP_TYPE_F16,
                 "modulated norm: gamma / beta must be F32 or F16");
    LEVO_REQUIRE(a.dim > 0 && a.dim % 4 == 0 && a.dim <= 4096,
                 "modulated norm: row length must be a positive multiple of 4, at most 4096 (got %lld)",
                 static_cast<long long>(a.dim));
    LEVO_REQUIRE(a.rows_per_batch > 0 && a.rows % a.rows_per_batch == 0,
                 "modulated norm: rows (%lld) must be a whole number of batch entries of %lld rows",
                 static_cast<long long>(a.rows), static_cast<long long>(a.rows_per_batch));
    LEVO_REQUIRE(a.eps >= 0.0f, "modulated norm: eps must be non-negative");
    LEVO_REQUIRE(a.gate.dynamic == nullptr || a.delta != nullptr, "modulated norm: a gate needs delta");
    LEVO_REQUIRE((a.scale.dynamic == nullptr) == (a.shift.dynamic == nullptr),
                 "modulated norm: scale and shift come together");
    const size_t palign = a.param_type == LEVO_HIP_TYPE_F16 ? 8 : 16;
    auto al = [](const void * q, size_t n) { return (reinterpret_cast<uintptr_t>(q) & (n - 1)) == 0; };
    LEVO_REQUIRE(aligned16(a.x) && (a.delta == nullptr || aligned16(a.delta)) &&
                     (a.h_out == nullptr || aligned16(a.h_out)) && aligned16(a.y) && al(a.gamma, palign) &&
                     al(a.beta, palign),
                 "modulated norm: rows and parameters must be 16-byte aligned (8-byte for F16 gamma / beta)");
    LEVO_REQUIRE(bvec_ok(a.gate, a.dim) && bvec_ok(a.scale, a.dim) && bvec_ok(a.shift, a.dim),
                 "modulated norm: a batch vector needs 16-byte aligned parts and a stride of at least dim, "
                 "a multiple of 4");
    const int64_t batches = a.rows / a.rows_per_batch;
    const int64_t wg_per_batch = ceil_div(a.rows_per_batch, 4);
    LEVO_REQUIRE(batches * wg_per_batch < (int64_t{1} << 24), "modulated norm: too many rows");
    const bool delta = a.delta != nullptr, gate = a.gate.dynamic != nullptr, mod = a.scale.dynamic != nullptr;
    mod_norm_params p;
    p.x = a.x;
    p.d = a.delta;
    p.gate = bvec{a.gate.dynamic, a.gate.stride, a.gate.learned};
    p.scale = bvec{a.scale.dynamic, a.scale.stride, a.scale.learned};
    p.shift = bvec{a.shift.dynamic, a.shift.stride, a.shift.learned};
    p.gamma = a.gamma;
    p.beta = a.beta;
    p.h_out = a.h_out;
    p.y = a.y;
    p.rows_per_batch = a.rows_per_batch;
    p.wg_per_batch = static_cast<int>(wg_per_batch);
    p.dim = static_cast<int>(a.dim);
    p.eps = a.eps;
    const int nv = a.dim <= 1024 ? 2 : a.dim <= 2560 ? 5 : 8;  // the instance launch_mod_norm_p picks
    const int lds = ((gate ? 1 : 0) + 2 + (mod ? 2 : 0)) * 128 * nv * 16;
    const uint32_t grid = static_cast<uint32_t>(batches * wg_per_batch);
    const hipStream_t s = as_hip(stream);
    return a.param_type == LEVO_HIP_TYPE_F16 ? launch_mod_norm_p<uint16_t>(p, delta, gate, mod, grid, lds, s)
                                             : launch_mod_norm_p<float>(p, delta, gate, mod, grid, lds, s);
}
