// Flow matching Euler step with classifier-free guidance, elementwise CFG
// combine, and the F16 <-> F32 row converters. All streaming kernels with
// dwordx4 accesses and the reference's two-rounding arithmetic (the library
// is compiled with -ffp-contract=off, so a*b+c is never fused here).
//
//   cfg_euler:  state += dt * (u + g * (c - u))   src/levo-flow-renderer.cpp:105, :307
//   incontext:  state  = ns * noise + t * context  src/levo-flow-renderer.cpp:94-101
//   cfg_combine: out   = u + s * (c - u)          src/levo-sampling.cpp:22-28,
//                                                 src/levo-renderer-pattern.cpp:123-135
#include "common.hpp"

namespace levo_hip {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ float cfg(float u, float c, float g) { return u + g * (c - u); }

__device__ __forceinline__ bool finite4(const f32x4 & v) {
    return __builtin_isfinite(v.x) && __builtin_isfinite(v.y) && __builtin_isfinite(v.z) &&
           __builtin_isfinite(v.w);
}

// Records which checked quantity held a non-finite value. Reached only on a
// failure, so the healthy path carries one compare per vector and no atomics.
__device__ __forceinline__ void flag_nonfinite(int32_t * flags, bool bad_v, bool bad_s) {
    const int32_t f = (bad_v ? LEVO_HIP_NONFINITE_VELOCITY : 0) | (bad_s ? LEVO_HIP_NONFINITE_STATE : 0);
    if (f) atomicOr(flags, f);
}

// One dwordx4 per thread; the scalar tail (n % 4) is handled by block 0.
// kCheck: also flag a non-finite combined velocity or updated state
// (src/levo-flow-renderer.cpp:104, :106).
template <bool kCfg, bool kCheck>
__global__ __launch_bounds__(kThreads) void cfg_euler_kernel(float * state, const float * __restrict__ vu,
                                                             const float * __restrict__ vc, int64_t n,
                                                             float g, float dt, int32_t * flags) {
    const int64_t n4 = n / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i < n4) {
        f32x4 s = reinterpret_cast<const f32x4 *>(state)[i];
        const f32x4 u = reinterpret_cast<const f32x4 *>(vu)[i];
        f32x4 v = u;
        if (kCfg) {
            const f32x4 c = reinterpret_cast<const f32x4 *>(vc)[i];
            v.x = cfg(u.x, c.x, g);
            v.y = cfg(u.y, c.y, g);
            v.z = cfg(u.z, c.z, g);
            v.w = cfg(u.w, c.w, g);
        }
        s.x += dt * v.x;
        s.y += dt * v.y;
        s.z += dt * v.z;
        s.w += dt * v.w;
        reinterpret_cast<f32x4 *>(state)[i] = s;
        if (kCheck) flag_nonfinite(flags, !finite4(v), !finite4(s));
    }
    if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
        const int64_t e = n4 * 4 + threadIdx.x;
        const float v = kCfg ? cfg(vu[e], vc[e], g) : vu[e];
        const float s = state[e] + dt * v;
        state[e] = s;
        if (kCheck) flag_nonfinite(flags, !__builtin_isfinite(v), !__builtin_isfinite(s));
    }
}

template <bool kCfg, bool kCheck>
__global__ __launch_bounds__(kThreads) void cfg_euler_scalar(float * state, const float * __restrict__ vu,
                                                             const float * __restrict__ vc, int64_t n,
                                                             float g, float dt, int32_t * flags) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e < n) {
        const float v = kCfg ? cfg(vu[e], vc[e], g) : vu[e];
        const float s = state[e] + dt * v;
        state[e] = s;
        if (kCheck) flag_nonfinite(flags, !__builtin_isfinite(v), !__builtin_isfinite(s));
    }
}

// flags |= bit when any of x[0, n) is NaN or infinite.
__global__ __launch_bounds__(kThreads) void check_finite_kernel(const float * __restrict__ x, int64_t n,
                                                                int32_t * flags, int32_t bit, bool vec) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
    bool bad = false;
    if (vec) {
        const int64_t n4 = n / 4;
        for (int64_t j = i; j < n4; j += stride) bad |= !finite4(reinterpret_cast<const f32x4 *>(x)[j]);
        if (i < (n & 3)) bad |= !__builtin_isfinite(x[n4 * 4 + i]);
    } else {
        for (int64_t j = i; j < n; j += stride) bad |= !__builtin_isfinite(x[j]);
    }
    if (bad) atomicOr(flags, bit);
}

__global__ __launch_bounds__(kThreads) void incontext_kernel(float * state, const float * __restrict__ noise,
                                                             const float * __restrict__ context,
                                                             int64_t n, float ns, float t) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e < n) state[e] = ns * noise[e] + t * context[e];
}

__global__ __launch_bounds__(kThreads) void cfg_combine_kernel(float * out, const float * __restrict__ u,
                                                               const float * __restrict__ c, int64_t n,
                                                               float s, bool vec) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (vec) {
        const int64_t n4 = n / 4;
        if (i < n4) {
            const f32x4 a = reinterpret_cast<const f32x4 *>(u)[i];
            const f32x4 b = reinterpret_cast<const f32x4 *>(c)[i];
            f32x4 r;
            r.x = cfg(a.x, b.x, s);
            r.y = cfg(a.y, b.y, s);
            r.z = cfg(a.z, b.z, s);
            r.w = cfg(a.w, b.w, s);
            reinterpret_cast<f32x4 *>(out)[i] = r;
        }
        if (blockIdx.x == 0 && threadIdx.x < (n & 3)) {
            const int64_t e = n4 * 4 + threadIdx.x;
            out[e] = cfg(u[e], c[e], s);
        }
    } else if (i < n) {
        out[i] = cfg(u[i], c[i], s);
    }
}

__global__ __launch_bounds__(kThreads) void f32_to_f16_kernel(const float * __restrict__ x, uint16_t * y,
                                                              int64_t n) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e < n) y[e] = f2h(x[e]);
}

__global__ __launch_bounds__(kThreads) void f16_to_f32_kernel(const uint16_t * __restrict__ x, float * y,
                                                              int64_t n) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e < n) y[e] = h2f(x[e]);
}

// Eight values per thread, 16-byte aligned rows: two dwordx4 F32 and one
// dwordx4 F16 transaction per thread; the same per-value rounding (RNE
// narrowing, exact widening) as the scalar kernels, which take the tail.
__global__ __launch_bounds__(kThreads) void f32_to_f16_vec8(const float * __restrict__ x, uint16_t * y, int64_t n8) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (i >= n8) return;
    const f32x4 a = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x) + 2 * i);
    const f32x4 b = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x) + 2 * i + 1);
    u32x4 o;
    o[0] = f2h(a[0]) | (static_cast<uint32_t>(f2h(a[1])) << 16);
    o[1] = f2h(a[2]) | (static_cast<uint32_t>(f2h(a[3])) << 16);
    o[2] = f2h(b[0]) | (static_cast<uint32_t>(f2h(b[1])) << 16);
    o[3] = f2h(b[2]) | (static_cast<uint32_t>(f2h(b[3])) << 16);
    __builtin_nontemporal_store(o, reinterpret_cast<u32x4 *>(y) + i);
}

// Widening, four values per lane: each dwordx2 load and dwordx4 store of a
// wave covers one contiguous span; thread t of workgroup g converts groups
// g * 256 * kWidenPer + k * 256 + t, k < kWidenPer.
constexpr int kWidenPer = 2;

__global__ __launch_bounds__(kThreads) void f16_to_f32_vec4(const uint16_t * __restrict__ x, float * y, int64_t n4) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads * kWidenPer + threadIdx.x;
    u32x2 v[kWidenPer];
#pragma unroll
    for (int k = 0; k < kWidenPer; ++k) {
        const int64_t i = i0 + k * kThreads;
        v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(x) + (i < n4 ? i : n4 - 1));
    }
#pragma unroll
    for (int k = 0; k < kWidenPer; ++k) {
        const int64_t i = i0 + k * kThreads;
        if (i >= n4) break;
        f32x4 a;
        a[0] = h2f(static_cast<uint16_t>(v[k][0] & 0xffffu));
        a[1] = h2f(static_cast<uint16_t>(v[k][0] >> 16));
        a[2] = h2f(static_cast<uint16_t>(v[k][1] & 0xffffu));
        a[3] = h2f(static_cast<uint16_t>(v[k][1] >> 16));
        __builtin_nontemporal_store(a, reinterpret_cast<f32x4 *>(y) + i);
    }
}

// Widening, 8 G values per lane: each lane requests G dwordx4 of 8 halves (a
// wave's 512 G halves, G KiB, in G instructions); the wave's block goes
// through its own G KiB of LDS so that each of its 2 G dwordx4 stores covers
// one contiguous KiB of floats (lane l stores floats 4 l .. 4 l + 3 of each
// quarter-KiB of halves). G = 2: 6.7 us for 4096 x 1536 values, 0.98 of the
// streaming ceiling (G = 1 7.8 us; four values per lane with dwordx2 loads,
// the form for 8-byte aligned sources, 8.6 us).
template <int G>
__global__ __launch_bounds__(kThreads) void f16_to_f32_x8(const uint16_t * __restrict__ x, float * y, int64_t n8) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    __shared__ __attribute__((aligned(16))) uint32_t stage[kThreads / 64][256 * G];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * (kThreads / 64) + wave) * 64 * G;  // the wave's first group
    u32x4 v[G];
#pragma unroll
    for (int k = 0; k < G; ++k) {
        const int64_t g = base + 64 * k + lane;
        v[k] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(x) + (g < n8 ? g : n8 - 1));
    }
    uint32_t * st = stage[wave];
#pragma unroll
    for (int k = 0; k < G; ++k) reinterpret_cast<u32x4 *>(st)[64 * k + lane] = v[k];
    // one wave's LDS operations complete in issue order
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int h = 0; h < 2 * G; ++h) {
        const u32x2 w = reinterpret_cast<const u32x2 *>(st)[64 * h + lane];  // halves 256 h + 4 lane ..
        if (base + 32 * h + (lane >> 1) >= n8) continue;
        f32x4 a;
        a[0] = h2f(static_cast<uint16_t>(w[0] & 0xffffu));
        a[1] = h2f(static_cast<uint16_t>(w[0] >> 16));
        a[2] = h2f(static_cast<uint16_t>(w[1] & 0xffffu));
        a[3] = h2f(static_cast<uint16_t>(w[1] >> 16));
        __builtin_nontemporal_store(a, reinterpret_cast<f32x4 *>(y) + 2 * base + 64 * h + lane);
    }
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

namespace {

int launch_euler(float * state, const float * v_uncond, const float * v_cond, int64_t n, float guidance,
                 float dt, int32_t * flags, levo_hip_stream_t stream, const char * what) {
    const bool vec = aligned16(state) && aligned16(v_uncond) && (v_cond == nullptr || aligned16(v_cond));
    const hipStream_t s = as_hip(stream);
    const bool check = flags != nullptr;
    if (vec) {
        const int64_t grid = ceil_div(n / 4 > 0 ? n / 4 : 1, kThreads);
        if (v_cond && check)
            cfg_euler_kernel<true, true><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else if (v_cond)
            cfg_euler_kernel<true, false><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else if (check)
            cfg_euler_kernel<false, true><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else
            cfg_euler_kernel<false, false><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
    } else {
        const int64_t grid = ceil_div(n, kThreads);
        if (v_cond && check)
            cfg_euler_scalar<true, true><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else if (v_cond)
            cfg_euler_scalar<true, false><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else if (check)
            cfg_euler_scalar<false, true><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
        else
            cfg_euler_scalar<false, false><<<grid, kThreads, 0, s>>>(state, v_uncond, v_cond, n, guidance, dt, flags);
    }
    return launch_status(what);
}

}  // namespace

extern "C" int levo_hip_flow_cfg_euler(float * state, const float * v_uncond, const float * v_cond,
                                       int64_t n, float guidance, float dt, levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "LeVo Flow renderer: Euler state size is negative");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(state != nullptr && v_uncond != nullptr,
                 "LeVo Flow renderer: Euler state or velocity is null");
    return launch_euler(state, v_uncond, v_cond, n, guidance, dt, nullptr, stream, "levo_hip_flow_cfg_euler");
}

extern "C" int levo_hip_flow_cfg_euler_checked(float * state, const float * v_uncond, const float * v_cond,
                                               int64_t n, float guidance, float dt, int32_t * nonfinite,
                                               levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "LeVo Flow renderer: Euler state size is negative");
    LEVO_REQUIRE(nonfinite != nullptr, "LeVo Flow renderer: non-finite flag pointer is null");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(state != nullptr && v_uncond != nullptr,
                 "LeVo Flow renderer: Euler state or velocity is null");
    return launch_euler(state, v_uncond, v_cond, n, guidance, dt, nonfinite, stream,
                        "levo_hip_flow_cfg_euler_checked");
}

extern "C" int levo_hip_check_finite(const float * x, int64_t n, int32_t * flags, int32_t bit,
                                     levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "check_finite: negative length");
    LEVO_REQUIRE(flags != nullptr, "check_finite: flag pointer is null");
    LEVO_REQUIRE(bit != 0, "check_finite: flag bit is zero");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(x != nullptr, "check_finite: input is null");
    const bool vec = aligned16(x);
    const int64_t items = vec ? (n / 4 > 0 ? n / 4 : 1) : n;
    // Up to 8 workgroups per CU, each thread then strides over the rest.
    const int64_t grid = ceil_div(items, kThreads) < 2048 ? ceil_div(items, kThreads) : 2048;
    check_finite_kernel<<<grid, kThreads, 0, as_hip(stream)>>>(x, n, flags, bit, vec);
    return launch_status("levo_hip_check_finite");
}

extern "C" int levo_hip_flow_incontext(float * state, const float * noise, const float * context,
                                       int64_t n_prefix, float time, float sigma_min,
                                       levo_hip_stream_t stream) {
    LEVO_REQUIRE(n_prefix >= 0, "LeVo Flow renderer: in-context length is negative");
    if (n_prefix == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(state != nullptr && noise != nullptr && context != nullptr,
                 "LeVo Flow renderer: Euler state, noise or context is null");
    // Host-side scalar exactly as src/levo-flow-renderer.cpp:94 (two roundings).
    const float noise_scale = 1.0f - (1.0f - sigma_min) * time;
    incontext_kernel<<<ceil_div(n_prefix, kThreads), kThreads, 0, as_hip(stream)>>>(
        state, noise, context, n_prefix, noise_scale, time);
    return launch_status("levo_hip_flow_incontext");
}

extern "C" int levo_hip_cfg_combine(float * out, const float * uncond, const float * cond, int64_t n,
                                    float scale, levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "CFG logits have different sizes");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(out != nullptr && uncond != nullptr && cond != nullptr, "CFG: null pointer");
    const bool vec = aligned16(out) && aligned16(uncond) && aligned16(cond);
    const int64_t grid = vec ? ceil_div(n / 4 > 0 ? n / 4 : 1, kThreads) : ceil_div(n, kThreads);
    cfg_combine_kernel<<<grid, kThreads, 0, as_hip(stream)>>>(out, uncond, cond, n, scale, vec);
    return launch_status("levo_hip_cfg_combine");
}

extern "C" int levo_hip_fp32_to_fp16_row(const float * x, uint16_t * y, int64_t n,
                                         levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "fp32_to_fp16_row: negative length");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(x != nullptr && y != nullptr, "fp32_to_fp16_row: null pointer");
    int64_t head = 0;
    if (aligned16(x) && aligned16(y)) {
        const int64_t n8 = n / 8;
        if (n8 > 0) f32_to_f16_vec8<<<ceil_div(n8, kThreads), kThreads, 0, as_hip(stream)>>>(x, y, n8);
        head = n8 * 8;
    }
    if (head < n) f32_to_f16_kernel<<<ceil_div(n - head, kThreads), kThreads, 0, as_hip(stream)>>>(x + head, y + head, n - head);
    return launch_status("levo_hip_fp32_to_fp16_row");
}

extern "C" int levo_hip_fp16_to_fp32_row(const uint16_t * x, float * y, int64_t n,
                                         levo_hip_stream_t stream) {
    LEVO_REQUIRE(n >= 0, "fp16_to_fp32_row: negative length");
    if (n == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(x != nullptr && y != nullptr, "fp16_to_fp32_row: null pointer");
    int64_t head = 0;
    if (aligned16(x) && aligned16(y)) {
        const int64_t n8 = n / 8;
        if (n8 > 0) f16_to_f32_x8<2><<<ceil_div(n8, 2 * kThreads), kThreads, 0, as_hip(stream)>>>(x, y, n8);
        head = n8 * 8;
    }
    if (head == 0 && (reinterpret_cast<uintptr_t>(x) & 7u) == 0 && aligned16(y)) {
        const int64_t n4 = n / 4;
        if (n4 > 0) f16_to_f32_vec4<<<ceil_div(n4, kThreads * kWidenPer), kThreads, 0, as_hip(stream)>>>(x, y, n4);
        head = n4 * 4;
    }
    if (head < n) f16_to_f32_kernel<<<ceil_div(n - head, kThreads), kThreads, 0, as_hip(stream)>>>(x + head, y + head, n - head);
    return launch_status("levo_hip_fp16_to_fp32_row");
}
