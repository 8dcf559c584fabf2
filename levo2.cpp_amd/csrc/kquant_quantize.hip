// K-quant block quantizers: ggml's quantize_row_q{4,5,6}_K_ref as the
// conversion tool reaches them, ggml_quantize_chunk(type, src, dst, start,
// nrows, n_per_row, NULL) (tools/levo-quantize.cpp:386-388, the Q6_K /
// Q5_K_M / Q4_K_M profiles of src/levo-quantization.h:47-55, 96-118).
//
// The searches are sequential float loops whose rounding order decides the
// chosen scale, so one lane runs one sub-block's search exactly in ggml's
// order (single roundings, no contraction; ggml builds these routines for
// the baseline x86-64 ISA, without FMA):
//   Q4_K / Q5_K: a lane per 32-value sub-block, eight lanes per super-block,
//     make_qkx2_quants (weights sqrt(mean x^2) + |x|; nmax 15 / 31; trial
//     inverse scales (rmin + 0.1 is + nmax) / (max - min), is = 0..20 / 0..15,
//     each refined by a weighted least-squares fit of scale and min);
//   Q6_K: a lane per 16-value sub-block, sixteen lanes per super-block,
//     make_qx_quants(16, 32, x, L, 1, NULL) (weights x^2, trial inverse
//     scales -(32 + 0.1 is) / max, is = -9..9).
// The lanes of a super-block then meet in LDS: the largest scale (and min)
// in sub-block order, the 6-bit (Q4_K / Q5_K) or 8-bit (Q6_K) sub-block
// scales against it, the F16 super-block scale(s), every value re-coded
// against the quantized scales (a sub-block whose quantized scale is 0 keeps
// its search codes), and the block bytes packed as ggml lays them out.
// The codes of a search are not kept per trial: the accepted trial's inverse
// scale and offset are, and the codes are recomputed from them (the same
// float operations give the same integers).
#include "common.hpp"

#include <type_traits>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ int nearest_int(float fval) {
    const float val = fval + 12582912.0f;  // 1.5 * 2^23: the integer lands in the mantissa (ties to even)
    return static_cast<int>(__builtin_bit_cast(uint32_t, val) & 0x007fffffu) - 0x00400000;
}

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

// N source values of one row from column col0 (zero past src_cols: the
// tool's row padding, tools/levo-quantize.cpp:375-384).
template <typename S, int N>
__device__ __forceinline__ void load_values(const S * row, int64_t col0, int64_t src_cols, float (&x)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int64_t c = col0 + k;
        if (c < src_cols) {
            if constexpr (std::is_same<S, uint16_t>::value) x[k] = h2f(row[c]);
            else x[k] = row[c];
        } else {
            x[k] = 0.0f;
        }
    }
}

// The code of a search value v, clamp(nearest_int(v), lo, hi), as a float.
// nearest_int rounds by adding 1.5 * 2^23: for |v| < 2^22 the sum stays in
// [2^23, 2^24), where the float spacing is 1, so it is v rounded to nearest,
// ties to even (the sum's parity is v's, 1.5 * 2^23 being even), which is
// v_rndne_f32; the clamp of the integer and its conversion back equal a
// float median of three. kFast takes that form (four instructions per code
// with the product instead of seven); its callers establish |v| < 2^22 for
// every value of a trial beforehand (in_trial_range), and a lane where that
// fails repeats its search in the integer form.
template <bool kFast>
__device__ __forceinline__ float code_of(float v, float lo, float hi) {
    if constexpr (kFast) return __builtin_amdgcn_fmed3f(__builtin_rintf(v), lo, hi);
    else return static_cast<float>(clampi(nearest_int(v), static_cast<int>(lo), static_cast<int>(hi)));
}

// Every v = iscale * (x - min) of a trial has |v| < 2^22 when this holds, for
// finite x in [xlo, xhi]: rounding is monotonic, so fl(x - min) lies between
// fl(xlo - min) and fl(xhi - min), and |fl(iscale * d)| <= fl(|iscale| * |d|).
// NaN or infinite scales or bounds fail it.
__device__ __forceinline__ bool in_trial_range(float iscale, float min, float xlo, float xhi) {
    const float d = fmaxf(__builtin_fabsf(xhi - min), __builtin_fabsf(min - xlo));
    return __builtin_fabsf(iscale) * d < 0x1p22f;
}

// make_qkx2_quants(32, NMAX, x, w, L, &the_min, Laux, rmin, 0.1, NSTEP, false).
// Returns the scale, -min in the_min, and the inverse scale and offset that
// produced the winning codes (code = clamp(nearest_int(iscale_l * (x - min_l)))).
// A trial's codes (Laux) are kept in registers for its error sum, as ggml
// keeps them in Laux; every float operation is ggml's, in its order. kFast
// (finite x only) clears in_range when a trial's values may leave the float
// code form's range; the caller then repeats the search with kFast false.
template <int NMAX, int NSTEP, bool kFast>
__device__ __forceinline__ float make_qkx2(const float (&x)[32], const float (&w)[32], float rmin, float & the_min,
                                           float & iscale_l, float & min_l, bool & zero_codes, bool & in_range) {
    constexpr float kMax = static_cast<float>(NMAX);
    float min = x[0];
    float max = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    const float xlo = min;
    if (min > 0) min = 0;
    zero_codes = false;
    if (max == min) {
        zero_codes = true;
        the_min = -min;
        iscale_l = 0.0f;
        min_l = 0.0f;
        return 0.f;
    }
    float iscale = NMAX / (max - min);
    float scale = 1 / iscale;
    float best_mad = 0;
    if (kFast) in_range = in_range && in_trial_range(iscale, min, xlo, max);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const float l = code_of<kFast>(iscale * (x[i] - min), 0.0f, kMax);
        float diff = scale * l + min - x[i];
        diff = diff * diff;
        best_mad += w[i] * diff;
    }
    iscale_l = iscale;
    min_l = min;
    // one trial per iteration, not unrolled: the trials are sequential (each
    // may move min) and an unrolled copy per trial would not fit the registers
#pragma unroll 1
    for (int is = 0; is <= NSTEP; ++is) {
        iscale = (rmin + 0.1f * static_cast<float>(is) + static_cast<float>(NMAX)) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        float laux[32];
        if (kFast) in_range = in_range && in_trial_range(iscale, min, xlo, max);
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            laux[i] = code_of<kFast>(iscale * (x[i] - min), 0.0f, kMax);
            const float wl = w[i] * laux[i];
            sum_l += wl;
            sum_l2 += wl * laux[i];
            sum_xl += wl * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                // the integer form recomputes the trial's codes (fewer live registers)
                const float l = kFast ? laux[i] : code_of<false>(iscale * (x[i] - min), 0.0f, kMax);
                float diff = this_scale * l + this_min - x[i];
                diff = diff * diff;
                mad += w[i] * diff;
            }
            if (mad < best_mad) {
                iscale_l = iscale;
                min_l = min;
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    the_min = -min;
    return scale;
}

// make_qx_quants(16, 32, x, L, rmse_type 1, NULL). Returns the scale and the
// inverse scale of the winning codes (code = clamp(nearest_int(iscale_l * x),
// -32, 31) + 32), or zero_codes for an all-zero group. The weights x^2 and
// their products with x (ggml's w * x[i] * l is (w * x[i]) * l) are formed
// once, outside the trials. For finite x every |iscale * x| stays within
// 32.9 (|x| <= |max|), so kFast needs only finite values (the caller's check).
template <bool kFast>
__device__ __forceinline__ float make_qx(const float (&x)[16], float & iscale_l, bool & zero_codes) {
    constexpr int nmax = 32;
    float max = 0;
    float amax = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    zero_codes = amax < 1e-15f;
    iscale_l = 0.0f;
    if (zero_codes) return 0.f;
    float w[16], wx[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        w[i] = x[i] * x[i];
        wx[i] = w[i] * x[i];
    }
    float iscale = static_cast<float>(-nmax) / max;
    float sumlx = 0;
    float suml2 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float l = code_of<kFast>(iscale * x[i], -32.0f, 31.0f);
        sumlx += wx[i] * l;
        suml2 += (w[i] * l) * l;
    }
    iscale_l = iscale;
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -(static_cast<float>(nmax) + 0.1f * static_cast<float>(is)) / max;
        sumlx = suml2 = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float l = code_of<kFast>(iscale * x[i], -32.0f, 31.0f);
            sumlx += wx[i] * l;
            suml2 += (w[i] * l) * l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            iscale_l = iscale;
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// LDS of one wave: per super-block group, the 256 codes and the per-lane
// scale data.
template <int GROUPS, int LANES>
struct kq_lds {
    uint8_t codes[GROUPS][256];
    float scale[GROUPS][LANES];
    float min[GROUPS][LANES];
    int q6s[GROUPS][LANES];
    uint8_t ls[GROUPS][8];
    uint8_t lm[GROUPS][8];
};

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One lane's sub-block of a Q4_K / Q5_K super-block: ggml's search over its
// 32 values with the weights sqrt(mean x^2) + |x|. kFast returns false when a
// lane of the wave met a code value outside the float form's range; the
// caller then runs the integer form, which loads the values again (so
// nothing of the first run stays live across it).
template <bool Q5, typename S, bool kFast>
__device__ __forceinline__ bool q45_search(const S * row, int64_t col0, int64_t src_cols, float & scale,
                                           float & the_min, float & iscale_l, float & min_l, bool & zero_codes) {
    // a compiler barrier: the values are loaded here, not reused from an
    // earlier load of the same addresses (which would keep them live)
    asm volatile("" ::: "memory");
    float x[32];
    load_values<S, 32>(row, col0, src_cols, x);
    float sum_x2 = 0;
#pragma unroll
    for (int l = 0; l < 32; ++l) sum_x2 += x[l] * x[l];
    const float av_x = sqrtf(sum_x2 / 32);
    float w[32];
#pragma unroll
    for (int l = 0; l < 32; ++l) w[l] = av_x + fabsf(x[l]);
    // the float code form needs finite values (a NaN or inf in x, or squares
    // that overflow, make sum_x2 NaN or inf)
    bool in_range = __builtin_isfinite(sum_x2);
    scale = make_qkx2<Q5 ? 31 : 15, Q5 ? 15 : 20, kFast>(x, w, Q5 ? -0.5f : -1.f, the_min, iscale_l, min_l,
                                                         zero_codes, in_range);
    return !kFast || __ballot(!in_range) == 0;
}

// Q4_K (Q5 = false) / Q5_K: eight lanes per super-block, eight super-blocks
// per wave. Super-block sb is row sb / nsb_row, columns (sb % nsb_row) * 256.
template <bool Q5, typename S>
__global__ __launch_bounds__(kThreads, 3) void quantize_q45_k_kernel(const S * __restrict__ src, int64_t src_cols,
                                                                  int64_t src_stride, uint8_t * __restrict__ dst,
                                                                  int64_t nsb_row, int64_t nsb) {
    constexpr int NMAX = Q5 ? 31 : 15;
    constexpr int QB = Q5 ? 176 : 144;
    __shared__ kq_lds<8, 8> lds_all[kWaves];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    kq_lds<8, 8> & L = lds_all[wave];
    const int g = lane >> 3;  // super-block group of the wave
    const int j = lane & 7;   // sub-block
    const int64_t sb = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 8 + g;
    const bool valid = sb < nsb;
    const int64_t sbc = valid ? sb : nsb - 1;
    const int64_t r = sbc / nsb_row;
    const int64_t col0 = (sbc - r * nsb_row) * 256 + 32 * j;

    float scale, the_min, iscale_l, min_l;
    bool zero_codes;
    if (!q45_search<Q5, S, true>(src + r * src_stride, col0, src_cols, scale, the_min, iscale_l, min_l, zero_codes))
        q45_search<Q5, S, false>(src + r * src_stride, col0, src_cols, scale, the_min, iscale_l, min_l, zero_codes);
    asm volatile("" ::: "memory");
    float x[32];  // the values again (a cache hit), for the codes
    load_values<S, 32>(src + r * src_stride, col0, src_cols, x);
    L.scale[g][j] = scale;
    L.min[g][j] = the_min;
    wave_lds_sync();
    float max_scale = 0, max_min = 0;  // in sub-block order, as ggml
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float s = L.scale[g][q];
        const float m = L.min[g][q];
        if (s > max_scale) max_scale = s;
        if (m > max_min) max_min = m;
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    uint32_t ls = static_cast<uint8_t>(nearest_int(inv_scale * scale));
    uint32_t lm = static_cast<uint8_t>(nearest_int(inv_min * the_min));
    ls = ls < 63u ? ls : 63u;
    lm = lm < 63u ? lm : 63u;
    const uint16_t d16 = f2h(max_scale / 63.f);
    const uint16_t dmin16 = f2h(max_min / 63.f);
    // the codes: re-coded against the quantized scales, or the search's own
    const float d = h2f(d16) * static_cast<float>(ls);
    const float dm = h2f(dmin16) * static_cast<float>(lm);
#pragma unroll
    for (int l = 0; l < 32; ++l) {
        int c;
        if (d != 0.0f) c = clampi(nearest_int((x[l] + dm) / d), 0, NMAX);
        else c = zero_codes ? 0 : clampi(nearest_int(iscale_l * (x[l] - min_l)), 0, NMAX);
        L.codes[g][32 * j + l] = static_cast<uint8_t>(c);
    }
    L.ls[g][j] = static_cast<uint8_t>(ls);
    L.lm[g][j] = static_cast<uint8_t>(lm);
    wave_lds_sync();
    if (!valid) return;
    uint8_t * out = dst + sb * QB;
    const uint8_t * cd = L.codes[g];
    for (int t = j; t < QB; t += 8) {
        uint32_t b;
        if (t < 2) {
            b = (d16 >> (8 * t)) & 0xffu;
        } else if (t < 4) {
            b = (dmin16 >> (8 * (t - 2))) & 0xffu;
        } else if (t < 16) {
            const int s = t - 4;  // packed 6-bit scales and mins (get_scale_min_k4's layout)
            if (s < 4) b = L.ls[g][s] | ((L.ls[g][s + 4] >> 4) << 6);
            else if (s < 8) b = L.lm[g][s - 4] | ((L.lm[g][s] >> 4) << 6);
            else b = (L.ls[g][s - 4] & 0xFu) | ((L.lm[g][s - 4] & 0xFu) << 4);
        } else if (!Q5) {
            const int u = t - 16;  // qs[32p + l] = code[64p + l] | code[64p + 32 + l] << 4
            const int p = u >> 5, l = u & 31;
            b = cd[64 * p + l] | (cd[64 * p + 32 + l] << 4);
        } else if (t < 48) {
            const int l = t - 16;  // qh[l]: bit 2p from code[64p + l] > 15, bit 2p + 1 from code[64p + 32 + l] > 15
            b = 0;
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                b |= (cd[64 * p + l] > 15 ? 1u : 0u) << (2 * p);
                b |= (cd[64 * p + 32 + l] > 15 ? 1u : 0u) << (2 * p + 1);
            }
        } else {
            const int u = t - 48;
            const int p = u >> 5, l = u & 31;
            b = (cd[64 * p + l] & 0xFu) | ((cd[64 * p + 32 + l] & 0xFu) << 4);
        }
        out[t] = static_cast<uint8_t>(b);
    }
}

// Q6_K: sixteen lanes per super-block, four super-blocks per wave.
template <typename S>
__global__ __launch_bounds__(kThreads) void quantize_q6_k_kernel(const S * __restrict__ src, int64_t src_cols,
                                                                 int64_t src_stride, uint8_t * __restrict__ dst,
                                                                 int64_t nsb_row, int64_t nsb) {
    constexpr int QB = 210;
    __shared__ kq_lds<4, 16> lds_all[kWaves];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    kq_lds<4, 16> & L = lds_all[wave];
    const int g = lane >> 4;
    const int j = lane & 15;
    const int64_t sb = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 4 + g;
    const bool valid = sb < nsb;
    const int64_t sbc = valid ? sb : nsb - 1;
    const int64_t r = sbc / nsb_row;
    const int64_t col0 = (sbc - r * nsb_row) * 256 + 16 * j;

    float x[16];
    load_values<S, 16>(src + r * src_stride, col0, src_cols, x);
    float iscale_l;
    bool zero_codes;
    float abs_sum = 0.0f;  // NaN or inf when a value is not finite (or the sum overflows)
#pragma unroll
    for (int l = 0; l < 16; ++l) abs_sum += fabsf(x[l]);
    float scale;
    if (__ballot(!__builtin_isfinite(abs_sum)) == 0) scale = make_qx<true>(x, iscale_l, zero_codes);
    else scale = make_qx<false>(x, iscale_l, zero_codes);
    L.scale[g][j] = scale;
    wave_lds_sync();
    float max_scale = 0, max_abs_scale = 0;  // first of the largest magnitudes, as ggml
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float s = L.scale[g][q];
        const float a = fabsf(s);
        if (a > max_abs_scale) {
            max_abs_scale = a;
            max_scale = s;
        }
    }
    const bool zero_block = max_abs_scale < 1e-15f;
    const float iscale = -128.f / max_scale;
    const uint16_t d16 = zero_block ? f2h(0.f) : f2h(1 / iscale);
    const int sc = zero_block ? 0 : min(127, nearest_int(iscale * scale));
    const float d = h2f(d16) * static_cast<float>(sc);
#pragma unroll
    for (int l = 0; l < 16; ++l) {
        int c;
        if (zero_block) c = 0;
        else if (d != 0.0f) c = clampi(nearest_int(x[l] / d), -32, 31) + 32;
        else c = zero_codes ? 0 : clampi(nearest_int(iscale_l * x[l]), -32, 31) + 32;
        L.codes[g][16 * j + l] = static_cast<uint8_t>(c);
    }
    L.q6s[g][j] = sc;
    wave_lds_sync();
    if (!valid) return;
    uint8_t * out = dst + sb * QB;
    const uint8_t * cd = L.codes[g];
    for (int t = j; t < QB; t += 16) {
        uint32_t b;
        if (zero_block) {
            b = t < 208 ? 0u : (d16 >> (8 * (t - 208))) & 0xffu;
        } else if (t < 128) {
            const int h = t >> 6, u = t & 63;  // ql of half h
            const int base = 128 * h + (u & 31) + (u < 32 ? 0 : 32);
            b = (cd[base] & 0xFu) | ((cd[base + 64] & 0xFu) << 4);
        } else if (t < 192) {
            const int h = (t - 128) >> 5, l = (t - 128) & 31;
            const int base = 128 * h + l;
            b = (cd[base] >> 4) | ((cd[base + 32] >> 4) << 2) | ((cd[base + 64] >> 4) << 4) | ((cd[base + 96] >> 4) << 6);
        } else if (t < 208) {
            b = static_cast<uint32_t>(L.q6s[g][t - 192]) & 0xffu;
        } else {
            b = (d16 >> (8 * (t - 208))) & 0xffu;
        }
        out[t] = static_cast<uint8_t>(b);
    }
}

template <typename S>
int launch_kquant_quantize(levo_hip_type type, const S * src, int64_t src_cols, int64_t src_stride, uint8_t * dst,
                           int64_t nrows, int64_t dst_cols, hipStream_t stream) {
    const int64_t nsb_row = dst_cols / 256;
    const int64_t nsb = nrows * nsb_row;
    if (type == LEVO_HIP_TYPE_Q6_K) {
        const int64_t grid = ceil_div(nsb, 4 * kWaves);
        quantize_q6_k_kernel<S><<<grid, kThreads, 0, stream>>>(src, src_cols, src_stride, dst, nsb_row, nsb);
    } else {
        const int64_t grid = ceil_div(nsb, 8 * kWaves);
        if (type == LEVO_HIP_TYPE_Q5_K)
            quantize_q45_k_kernel<true, S><<<grid, kThreads, 0, stream>>>(src, src_cols, src_stride, dst, nsb_row, nsb);
        else
            quantize_q45_k_kernel<false, S><<<grid, kThreads, 0, stream>>>(src, src_cols, src_stride, dst, nsb_row, nsb);
    }
    return launch_status("levo_hip_quantize (K-quant)");
}

}  // namespace

int quantize_kquant_rows(levo_hip_type type, const void * src, levo_hip_type src_type, int64_t src_cols,
                         int64_t src_stride, void * dst, int64_t nrows, int64_t dst_cols, hipStream_t stream) {
    uint8_t * d = static_cast<uint8_t *>(dst);
    if (src_type == LEVO_HIP_TYPE_F16)
        return launch_kquant_quantize(type, static_cast<const uint16_t *>(src), src_cols, src_stride, d, nrows,
                                      dst_cols, stream);
    return launch_kquant_quantize(type, static_cast<const float *>(src), src_cols, src_stride, d, nrows, dst_cols,
                                  stream);
}

}  // namespace levo_hip
