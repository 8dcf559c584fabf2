// Shared helpers of the gfx950 kernels: status reporting, launch checks,
// vector types, wave64 reductions and F16 bit conversions.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "levo_hip.h"

namespace levo_hip {

// ---- status ---------------------------------------------------------------

void set_error(const char * fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

#define LEVO_REQUIRE(cond, ...)                        \
    do {                                               \
        if (!(cond)) {                                 \
            ::levo_hip::set_error(__VA_ARGS__);        \
            return LEVO_HIP_ERR_INVALID;               \
        }                                              \
    } while (0)

// Checks the launch that was just enqueued.
int launch_status(const char * what);

// Raises `kernel`'s dynamic LDS limit to `bytes` on the current device, once
// per (kernel, device); thread-safe. LEVO_HIP_OK or LEVO_HIP_ERR_RUNTIME.
int allow_dynamic_lds(const void * kernel, int bytes, const char * what);

inline hipStream_t as_hip(levo_hip_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device (queried once per device; 0 if the
// query fails).
int device_cu_count();

// K-quant helpers shared by the quantizer entry points (kquant.hip).
bool is_kquant(levo_hip_type type);
int64_t kquant_block_bytes(levo_hip_type type);  // Q4_K / Q5_K / Q6_K / Q8_K per 256 values; 0 otherwise
// ggml's quantize_row_q{4,5,6}_K_ref over rows of src (F32 or F16, src_cols
// values each, src_stride apart, zero-padded to dst_cols, a multiple of 256).
int quantize_kquant_rows(levo_hip_type type, const void * src, levo_hip_type src_type, int64_t src_cols,
                         int64_t src_stride, void * dst, int64_t nrows, int64_t dst_cols, hipStream_t stream);
int dequantize_kquant(levo_hip_type type, const void * src, void * dst, levo_hip_type dst_type, int64_t k,
                      hipStream_t stream);

// One VAE residual unit, y = x + conv_1(snake_post(conv_0(snake_pre(x)))),
// conv_0 k = 7 at dilation d (padding 3d), conv_1 k = 1 (src/levo-vae.cpp:91-100),
// as a single launch (snake_conv.hip). Applies to 128 channels with 16-byte
// aligned weights and both SnakeBeta parameter sets; returns kNotFused
// otherwise (nothing launched). x and y are [128][t] with row stride t and
// must not overlap.
constexpr int kNotFused = 1;

// levo_hip_snake_conv1d_split on contiguous rows (x, y: row stride t) with a
// SnakeBeta of its own applied to the output (after the bias):
// y = snake_post(conv(snake(x)) + bias). The decoder's residual units store
// their k = 1 conv's activated input this way, one SnakeBeta per sample.
int snake_conv1d_post(const float * x, int64_t c_in, int64_t t, const void * alpha_log, const void * beta_log,
                      levo_hip_type param_type, const float * weight, int64_t c_out, int64_t kernel,
                      const float * bias, int64_t padding, int64_t dilation, float * y, const void * post_alpha_log,
                      const void * post_beta_log, float * ws, int64_t ws_floats, hipStream_t stream);
int launch_residual_unit_fused(const float * x, int64_t c, int64_t t, const void * pre_alpha_log,
                               const void * pre_beta_log, const float * w0, const float * b0,
                               const void * post_alpha_log, const void * post_beta_log, const float * w1,
                               const float * b1, int64_t dilation, levo_hip_type param_type, float * y,
                               hipStream_t stream);

inline bool aligned16(const void * p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- vector types (dwordx4 global accesses) --------------------------------

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// ---- F16 bit conversions (IEEE round-to-nearest-even, exact widening) -----

__device__ __forceinline__ float h2f(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// ---- order-preserving float key (+0 and -0 map to the same key) -----------

__device__ __forceinline__ uint32_t float_key(float v) {
    uint32_t b = __builtin_bit_cast(uint32_t, v + 0.0f);  // -0 -> +0 (RNE)
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---- wave64 reductions ------------------------------------------------------
// All-reduce over the 64 lanes: DPP within each row of 16 lanes (quad
// butterflies, then rotations by 4 and 8), then the four row totals are read
// with v_readlane and combined in a fixed order, so every lane returns the same
// value. Each DPP step is a few cycles; an LDS-routed shuffle costs ~100.

namespace dpp {
constexpr int kQuadXor1 = 0xB1;  // quad_perm [1, 0, 3, 2]
constexpr int kQuadXor2 = 0x4E;  // quad_perm [2, 3, 0, 1]
constexpr int kRowRor4 = 0x124;  // row_ror:4
constexpr int kRowRor8 = 0x128;  // row_ror:8
constexpr int kRowMirror = 0x140;      // row_mirror: lane i of each 16 takes lane 15 - i
constexpr int kRowHalfMirror = 0x141;  // row_half_mirror: lane i of each 8 takes lane 7 - i

// Every control used through mov (quad permutes, row rotations and mirrors)
// gives each lane a source inside its row, so no "old" value is needed: v_mov_b32_dpp
// without one spares the register a zero (or a copy) would take.
template <int kCtrl>
__device__ __forceinline__ uint32_t mov(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl>
__device__ __forceinline__ float mov(float v) {
    return __builtin_bit_cast(float, mov<kCtrl>(__builtin_bit_cast(uint32_t, v)));
}
template <int kCtrl>
__device__ __forceinline__ int mov(int v) {
    return static_cast<int>(mov<kCtrl>(static_cast<uint32_t>(v)));
}
template <int kCtrl>
__device__ __forceinline__ double mov(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = mov<kCtrl>(static_cast<uint32_t>(b));
    const uint64_t hi = mov<kCtrl>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(double, lo | (hi << 32));
}

template <int kCtrl>
__device__ __forceinline__ uint64_t mov(uint64_t v) {
    const uint64_t lo = mov<kCtrl>(static_cast<uint32_t>(v));
    const uint64_t hi = mov<kCtrl>(static_cast<uint32_t>(v >> 32));
    return lo | (hi << 32);
}

__device__ __forceinline__ uint32_t lane(uint32_t v, int l) {
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}
__device__ __forceinline__ float lane(float v, int l) {
    return __builtin_bit_cast(float, lane(__builtin_bit_cast(uint32_t, v), l));
}
__device__ __forceinline__ int lane(int v, int l) { return static_cast<int>(lane(static_cast<uint32_t>(v), l)); }
__device__ __forceinline__ uint64_t lane(uint64_t v, int l) {
    return lane(static_cast<uint32_t>(v), l) | (static_cast<uint64_t>(lane(static_cast<uint32_t>(v >> 32), l)) << 32);
}
__device__ __forceinline__ double lane(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = lane(static_cast<uint32_t>(b), l);
    const uint64_t hi = lane(static_cast<uint32_t>(b >> 32), l);
    return __builtin_bit_cast(double, lo | (hi << 32));
}

constexpr int kRowShr1 = 0x111;     // row_shr:1
constexpr int kRowShr2 = 0x112;     // row_shr:2
constexpr int kRowShr4 = 0x114;     // row_shr:4
constexpr int kRowShr8 = 0x118;     // row_shr:8
constexpr int kRowBcast15 = 0x142;  // row_bcast:15
constexpr int kRowBcast31 = 0x143;  // row_bcast:31

// v from the DPP source lane, or 0 where the source lies outside the row
// (bound_ctrl) or the destination row is masked off.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ int mov_or_zero(int v) {
    return __builtin_amdgcn_update_dpp(0, v, kCtrl, kRowMask, 0xF, true);
}

template <class T, class Op>
__device__ __forceinline__ T allreduce(T v, Op op) {
    v = op(v, mov<kQuadXor1>(v));
    v = op(v, mov<kQuadXor2>(v));
    v = op(v, mov<kRowRor4>(v));
    v = op(v, mov<kRowRor8>(v));
    return op(op(lane(v, 0), lane(v, 16)), op(lane(v, 32), lane(v, 48)));
}
}  // namespace dpp

// Sum over each group of LPR consecutive lanes (16, 32 or 64), in every lane
// of the group: DPP steps within each row of 16, then the row totals.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp::mov<dpp::kQuadXor1>(v);
    v += dpp::mov<dpp::kQuadXor2>(v);
    v += dpp::mov<dpp::kRowRor4>(v);
    v += dpp::mov<dpp::kRowRor8>(v);
    if constexpr (LPR == 16) {
        return v;
    } else if constexpr (LPR == 32) {
        const float lo = dpp::lane(v, 0) + dpp::lane(v, 16);
        const float hi = dpp::lane(v, 32) + dpp::lane(v, 48);
        return (threadIdx.x & 63) < 32 ? lo : hi;
    } else {
        return (dpp::lane(v, 0) + dpp::lane(v, 16)) + (dpp::lane(v, 32) + dpp::lane(v, 48));
    }
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    return dpp::allreduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ double wave_sum_f64(double v) {
    return dpp::allreduce(v, [](double a, double b) { return a + b; });
}
__device__ __forceinline__ float wave_max_f32(float v) {
    return dpp::allreduce(v, [](float a, float b) { return fmaxf(a, b); });
}
__device__ __forceinline__ int wave_sum_i32(int v) {
    return dpp::allreduce(v, [](int a, int b) { return a + b; });
}
__device__ __forceinline__ int wave_min_i32(int v) {
    return dpp::allreduce(v, [](int a, int b) { return a < b ? a : b; });
}
// Inclusive prefix sum over the 64 lanes: Hillis-Steele shifts within each row
// of 16, then row 0's total into row 1 and row 2's into row 3 (row_bcast:15),
// then lane 31's running total into rows 2 and 3 (row_bcast:31).
__device__ __forceinline__ int wave_inclusive_scan_i32(int v) {
    v += dpp::mov_or_zero<dpp::kRowShr1>(v);
    v += dpp::mov_or_zero<dpp::kRowShr2>(v);
    v += dpp::mov_or_zero<dpp::kRowShr4>(v);
    v += dpp::mov_or_zero<dpp::kRowShr8>(v);
    v += dpp::mov_or_zero<dpp::kRowBcast15, 0xA>(v);
    v += dpp::mov_or_zero<dpp::kRowBcast31, 0xC>(v);
    return v;
}

// The same over doubles: each DPP step moves both halves of the 64-bit value;
// lanes outside a step's source row receive +0.0, which leaves sums unchanged.
template <int kCtrl, int kRowMask = 0xF>
__device__ __forceinline__ double scan_step_f64(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint64_t lo = static_cast<uint32_t>(dpp::mov_or_zero<kCtrl, kRowMask>(static_cast<int>(static_cast<uint32_t>(b))));
    const uint64_t hi =
        static_cast<uint32_t>(dpp::mov_or_zero<kCtrl, kRowMask>(static_cast<int>(static_cast<uint32_t>(b >> 32))));
    return x + __builtin_bit_cast(double, lo | (hi << 32));
}
__device__ __forceinline__ double wave_inclusive_scan_f64(double v) {
    v = scan_step_f64<dpp::kRowShr1>(v);
    v = scan_step_f64<dpp::kRowShr2>(v);
    v = scan_step_f64<dpp::kRowShr4>(v);
    v = scan_step_f64<dpp::kRowShr8>(v);
    v = scan_step_f64<dpp::kRowBcast15, 0xA>(v);
    v = scan_step_f64<dpp::kRowBcast31, 0xC>(v);
    return v;
}

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Workgroup barrier that orders LDS accesses only: global loads in flight
// (a prefetch of the next row) and earlier global stores are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Makes the values of `v` present in registers at this point: the wait for the
// loads that produced them (and any conversion) happens here, not where they
// are first used. Stores and loads share one vector-memory counter on this
// GPU, so a wait for a load issued before a store also waits until that store
// has completed; calling this after the last load is issued and before the
// first store keeps every load wait ahead of every store. The memory clobber
// keeps loads above and stores below this point.
template <typename T, int N>
__device__ __forceinline__ void consume_now(T (&v)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) asm volatile("" : "+v"(v[k])::"memory");
}

// Bits of lanes below the calling lane in a 64-bit ballot mask.
__device__ __forceinline__ int rank_in_mask(uint64_t mask) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u));
}

}  // namespace levo_hip
