// Shared device helpers of the Q8_0 / Q4_0 kernels: the source-block loader
// and ggml's reference Q8_0 block quantizer (quantize_row_q8_0_ref as reached
// from ggml_quantize_chunk, tools/levo-quantize.cpp:386-388), bit-exact
// including the x86-64 conversions of out-of-range and non-finite values.
#pragma once

#include "common.hpp"

#include <type_traits>

namespace levo_hip {

// Loads one 32-value block starting at column col0 of a source row, zero
// beyond src_cols (row padding, write_tensor :375-384). kVec: the row start is
// 16-byte aligned, so a block that lies wholly inside the row takes dwordx4
// loads (4 for F16, 8 for F32).
template <typename S, bool kVec>
__device__ __forceinline__ void load_block(const S * row, int64_t col0, int64_t src_cols, float (&x)[32]) {
    if (kVec && col0 + 32 <= src_cols) {
        if constexpr (std::is_same<S, uint16_t>::value) {
            const u16x8 * p = reinterpret_cast<const u16x8 *>(row + col0);
            u16x8 v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = __builtin_nontemporal_load(p + i);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int k = 0; k < 8; ++k) x[i * 8 + k] = h2f(v[i][k]);
        } else {
            const f32x4 * p = reinterpret_cast<const f32x4 *>(row + col0);
            f32x4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = __builtin_nontemporal_load(p + i);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                x[i * 4 + 0] = v[i].x;
                x[i * 4 + 1] = v[i].y;
                x[i * 4 + 2] = v[i].z;
                x[i * 4 + 3] = v[i].w;
            }
        }
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const int64_t c = col0 + k;
            if (c < src_cols) {
                if constexpr (std::is_same<S, uint16_t>::value) x[k] = h2f(row[c]);
                else x[k] = row[c];
            } else {
                x[k] = 0.0f;
            }
        }
    }
}

// roundf (half away from zero) is trunc(v + copysign(0.5 - 2^-25, v)): the
// two agree for every non-NaN float (checked exhaustively), and NaN stays NaN.
// low_byte_i8 truncates toward zero itself, so callers pass the sum and the
// trunc is left to the conversion.
__device__ __forceinline__ float half_away_offset(float v) {
    return v + __builtin_copysignf(0x1.fffffep-2f, v);
}

// (int8_t)v as the reference's x86-64 build computes it: truncation to int32
// (cvttss2si), low byte kept. v_cvt_i32_f32 truncates too and gives 0 for NaN
// where cvttss2si gives 0x80000000 (low byte 0 as well); the two differ only
// beyond +-2^31, which the callers exclude or handle (see quantize_block).
// Inline asm because a C++ float -> int conversion of NaN is undefined.
__device__ __forceinline__ uint32_t low_byte_i8(float v) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return static_cast<uint32_t>(r) & 0xffu;
}

// id = 1/d is +inf only when d underflows; then every x * id is +-inf or NaN
// and the reference's (int8_t) conversion yields 0 for each (cvttss2si gives
// 0x80000000). Replacing such an id by NaN makes every product NaN, which
// low_byte_i8 maps to 0 as well, so the per-value code needs no special case.
__device__ __forceinline__ float nan_if_inf(float id) {
    return __builtin_isinf(id) ? __builtin_nanf("") : id;
}

__device__ __forceinline__ uint32_t pack4(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return a | (b << 8) | (c << 16) | (d << 24);
}

// v_cvt_i32_f32 of v (truncation; 0 for NaN), all 32 bits.
__device__ __forceinline__ uint32_t trunc_i32(float v) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return static_cast<uint32_t>(r);
}

// The low bytes of a, b, c, d as one little-endian dword, by two byte
// permutes (selector byte s takes byte s of {hi:lo}, 0x0c gives 0) and an OR.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);  // a0, b0, 0, 0
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x04000c0cu);  // 0, 0, c0, d0
    return ab | cd;
}

// Quantizes one block of 32 values as quantize_row_q8_0_ref does:
// amax = MAX(amax, |x|) in index order, d = amax / 127, id = d ? 1 / d : 0,
// q = (int8_t)roundf(x * id). Writes the quants as 8 little-endian dwords and
// returns d rounded to F16 (RNE).
__device__ __forceinline__ uint16_t quantize_q8_0_block(const float (&x)[32], uint32_t (&pk)[8]) {
    // |x| as an unsigned bit pattern orders like |x|, with every NaN above
    // +inf: the integer maximum is amax whenever the block holds no NaN, and
    // then the index-order MAX of the reference gives the same value.
    uint32_t bits_max = 0u;
#pragma unroll
    for (int k = 0; k < 32; ++k) bits_max = __builtin_elementwise_max(bits_max, __float_as_uint(x[k]) & 0x7fffffffu);
    const bool has_nan = bits_max > 0x7f800000u;
    float amax = __uint_as_float(bits_max);
    if (has_nan) {
        amax = 0.0f;  // ggml's MAX(amax, fabsf(v)) in index order: a NaN resets it
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float v = fabsf(x[k]);
            amax = amax > v ? amax : v;
        }
    }
    const float d = amax / 127.0f;
    const float id = nan_if_inf(d != 0.0f ? 1.0f / d : 0.0f);
    if (!has_nan) {
        // every |x| <= amax: |x * id| stays within 128 (or is NaN), so the
        // low byte of the truncated int32 is the reference's (int8_t)
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = trunc_i32(half_away_offset(x[4 * w + k] * id));
            pk[w] = pack_low_bytes(q[0], q[1], q[2], q[3]);
        }
    } else {
        // A NaN reset the running MAX, so earlier values may exceed amax
        // and x * id may leave the int32 range: there cvttss2si gives
        // 0x80000000 (low byte 0).
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float v = half_away_offset(x[4 * w + k] * id);
                q[k] = __builtin_fabsf(v) < 0x1p31f ? low_byte_i8(v) : 0u;
            }
            pk[w] = pack4(q[0], q[1], q[2], q[3]);
        }
    }
    return f2h(d);
}

}  // namespace levo_hip
