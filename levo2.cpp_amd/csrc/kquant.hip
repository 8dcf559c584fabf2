// K-quant super-blocks (ggml's Q4_K / Q5_K / Q6_K, QK_K = 256) on the decode
// path: the Q8_K activation quantizer (ggml's vec_dot_type for the K-quants,
// quantize_row_q8_K_ref), the dequantizers (dequantize_row_q{4,5,6}_K) and
// the mat-vec of ggml_mul_mat(W, x) with K-quant weights
// (ggml_vec_dot_q{4,5,6}_K_q8_K). These are the matrices the Q6_K, Q5_K_M
// and Q4_K_M profiles write (src/levo-quantization.h:47-55, 96-118).
//
// Block layouts (ggml, little-endian):
//   block_q4_K {f16 d; f16 dmin; u8 scales[12]; u8 qs[128]}            144 B
//   block_q5_K {f16 d; f16 dmin; u8 scales[12]; u8 qh[32]; u8 qs[128]} 176 B
//   block_q6_K {u8 ql[128]; u8 qh[64]; i8 scales[16]; f16 d}           210 B
//   block_q8_K {f32 d; i8 qs[256]; i16 bsums[16]}                      292 B
// Q4_K / Q5_K: eight sub-blocks of 32 with 6-bit scale and min (packed in
// 12 bytes); value = d * sc * q - dmin * m. Q6_K: sixteen sub-blocks of 16
// with int8 scales; value = d * sc * (q - 32).
#include "common.hpp"
#include "span_load.hpp"

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kQK = 256;

// ggml's nearest_int: fval + 1.5 * 2^23 leaves the integer (ties to even) in
// the mantissa for |fval| < 2^22.
__device__ __forceinline__ int nearest_int(float fval) {
    const float val = fval + 12582912.0f;
    return static_cast<int>(__builtin_bit_cast(uint32_t, val) & 0x007fffffu) - 0x00400000;
}

// get_scale_min_k4: sub-block j's 6-bit scale and min, without a branch
// (the lanes of a block take sub-blocks on both sides of j = 4; a branch ran
// both paths: Q4_K / Q5_K mat-vecs 2-4 % slower): with a, b, c byte j % 4 of
// the three dwords (bytes j % 4, 4 + j % 4, 8 + j % 4 of the twelve), j < 4
// takes sc = a & 63, m = b & 63; j >= 4 takes sc = (c & 15) | (a >> 6) << 4,
// m = (c >> 4) | (b >> 6) << 4.
__device__ __forceinline__ void scale_min_k4(uint32_t s0, uint32_t s1, uint32_t s2, int j, int & sc, int & m) {
    const uint32_t sh = 8u * static_cast<uint32_t>(j & 3);
    const int a = static_cast<int>((s0 >> sh) & 0xffu);
    const int b = static_cast<int>((s1 >> sh) & 0xffu);
    const int c = static_cast<int>((s2 >> sh) & 0xffu);
    const bool lo = j < 4;
    sc = lo ? (a & 63) : ((c & 0xF) | ((a >> 6) << 4));
    m = lo ? (b & 63) : ((c >> 4) | ((b >> 6) << 4));
}

// Two dwords at byte offset `off` of a block whose start is 2 mod 4 when
// `odd` (Q6_K's 210-byte blocks): aligned dword loads and a funnel shift of
// 16 bits (odd) or none, with no branch (lanes of one wave hold blocks of
// both kinds; a branch ran both paths: Q6_K mat-vecs 3-6 % slower). Odd
// blocks read three dwords, even ones the second dword again, so nothing
// past the block is read. off is a multiple of 4 and off + 10 <= 210; for
// odd blocks the two bytes before the block (the previous block's tail: the
// buffer itself is 16-byte aligned, so its first block is never odd) are
// read and discarded.
__device__ __forceinline__ void load_u32x2(const uint8_t * blk, int off, bool odd, uint32_t & a, uint32_t & b) {
    const uint32_t * p = reinterpret_cast<const uint32_t *>(blk + off - (odd ? 2 : 0));
    const uint32_t w0 = p[0], w1 = p[1], w2 = p[odd ? 2 : 1];
    const uint32_t sh = odd ? 16u : 0u;
    a = __builtin_amdgcn_alignbit(w1, w0, sh);
    b = __builtin_amdgcn_alignbit(w2, w1, sh);
}

__device__ __forceinline__ uint32_t load_u32(const uint8_t * blk, int off, bool odd) {
    const uint32_t * p = reinterpret_cast<const uint32_t *>(blk + off - (odd ? 2 : 0));
    return odd ? __builtin_amdgcn_alignbit(p[1], p[0], 16) : p[0];
}

// Bytes b in [0, 63] to the signed bytes b - 32 (no borrow between bytes).
__device__ __forceinline__ uint32_t minus32(uint32_t b) {
    return ((b | 0x80808080u) - 0x20202020u) ^ 0x80808080u;
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// ---- Q8_K quantizer: sixteen lanes per 256-value block -----------------------

// quantize_row_q8_K_ref for the block whose values 16 s .. 16 s + 15 this
// lane holds (s = lane % 16: sixteen lanes per block, four blocks per wave):
// its 16 quants as 4 dwords, its bsum s (elements 16 s .. 16 s + 15 are this
// lane's own) and the block's scale d. Every reduction stays inside the
// lane's row of 16, as DPP steps: the largest |x| bits (NaN counting as 0,
// so it never compares larger, as the reference's `if (ax > amax)` scan),
// the first index holding it, and that value's sign. A block of zeros gives
// d = 0, zero quants and a zero bsum. Every lane of the wave runs it.
__device__ __forceinline__ void q8_K_block16(const f32x4 (&v)[4], int s, uint32_t (&pk)[4], int & bsum,
                                             float & d) {
    uint32_t lmax = 0u, lval = 0u;
    int lidx = 0;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float x = v[q >> 2][q & 3];
        const float ax = __builtin_fabsf(x);
        const uint32_t bits = ax == ax ? __builtin_bit_cast(uint32_t, ax) : 0u;
        const bool more = bits > lmax;
        lmax = more ? bits : lmax;
        lidx = more ? q : lidx;
        lval = more ? __builtin_bit_cast(uint32_t, x) : lval;
    }
    uint32_t gmax = lmax;
    gmax = __builtin_elementwise_max(gmax, dpp::mov<dpp::kQuadXor1>(gmax));
    gmax = __builtin_elementwise_max(gmax, dpp::mov<dpp::kQuadXor2>(gmax));
    gmax = __builtin_elementwise_max(gmax, dpp::mov<dpp::kRowHalfMirror>(gmax));
    gmax = __builtin_elementwise_max(gmax, dpp::mov<dpp::kRowMirror>(gmax));
    const uint32_t mine = static_cast<uint32_t>(16 * s + lidx);
    uint32_t gidx = lmax == gmax ? mine : 256u;
    gidx = __builtin_elementwise_min(gidx, dpp::mov<dpp::kQuadXor1>(gidx));
    gidx = __builtin_elementwise_min(gidx, dpp::mov<dpp::kQuadXor2>(gidx));
    gidx = __builtin_elementwise_min(gidx, dpp::mov<dpp::kRowHalfMirror>(gidx));
    gidx = __builtin_elementwise_min(gidx, dpp::mov<dpp::kRowMirror>(gidx));
    uint32_t mbits = mine == gidx ? lval : 0u;
    mbits |= dpp::mov<dpp::kQuadXor1>(mbits);
    mbits |= dpp::mov<dpp::kQuadXor2>(mbits);
    mbits |= dpp::mov<dpp::kRowHalfMirror>(mbits);
    mbits |= dpp::mov<dpp::kRowMirror>(mbits);
    const bool zero = gmax == 0u;  // amax == 0: an all-zero (or all-NaN) block
    const float iscale = -127.0f / __builtin_bit_cast(float, mbits);
    int sum = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t packed = 0u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            int l = nearest_int(iscale * v[w][q]);
            l = l < 127 ? l : 127;
            l = zero ? 0 : l;
            sum += l;
            packed |= (static_cast<uint32_t>(l) & 0xffu) << (8 * q);
        }
        pk[w] = packed;
    }
    bsum = sum;
    d = zero ? 0.0f : 1.0f / iscale;
}

// Sixteen blocks per workgroup, sixteen lanes each (q8_K_block16); a group
// past the last block computes on the last one and stores nothing.
__global__ __launch_bounds__(kThreads) void quantize_q8_K_kernel(const float * __restrict__ x, uint8_t * y,
                                                                  int64_t nb) {
    const int s = threadIdx.x & 15;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * (kThreads / 16) + (threadIdx.x >> 4);
    const int64_t ic = i < nb ? i : nb - 1;
    const f32x4 * src = reinterpret_cast<const f32x4 *>(x + ic * kQK + 16 * s);
    const f32x4 v[4] = {src[0], src[1], src[2], src[3]};
    uint32_t pk[4];
    int bsum;
    float d;
    q8_K_block16(v, s, pk, bsum, d);
    if (i >= nb) return;
    uint8_t * blk = y + i * 292;
    uint32_t * q = reinterpret_cast<uint32_t *>(blk + 4 + 16 * s);  // 4-byte aligned (292 i + 4)
#pragma unroll
    for (int w = 0; w < 4; ++w) q[w] = pk[w];
    reinterpret_cast<int16_t *>(blk + 260)[s] = static_cast<int16_t>(bsum);
    if (s == 0) *reinterpret_cast<float *>(blk) = d;
}

// ---- dequantizers: 8 outputs per thread --------------------------------------

template <int TYPE, typename Out>
__global__ __launch_bounds__(kThreads) void dequantize_kquant_kernel(const uint8_t * __restrict__ src, Out * dst,
                                                                      int64_t nb) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t i = t >> 5;
    if (i >= nb) return;
    const int r = static_cast<int>(t & 31);
    const int j = r >> 2;         // 32-element group of the block (Q4_K / Q5_K: the sub-block)
    const int p = r & 3;          // 8-element part of it
    constexpr int kBytes = TYPE == LEVO_HIP_TYPE_Q4_K ? 144 : TYPE == LEVO_HIP_TYPE_Q5_K ? 176 : 210;
    const uint8_t * blk = src + i * kBytes;
    float out[8];
    if constexpr (TYPE == LEVO_HIP_TYPE_Q6_K) {
        const bool odd = (reinterpret_cast<uintptr_t>(blk) & 3u) != 0;
        const int n = j >> 2, quarter = j & 3, l0 = 8 * p;
        uint32_t ql0, ql1, qh0, qh1;
        load_u32x2(blk, 64 * n + 32 * (quarter & 1) + l0, odd, ql0, ql1);
        load_u32x2(blk, 128 + 32 * n + l0, odd, qh0, qh1);
        const float d = h2f(*reinterpret_cast<const uint16_t *>(blk + 208));  // 2-byte load: stays in the block
        const int sub = 8 * n + 2 * quarter + (p >> 1);
        const uint32_t sw = load_u32(blk, 192 + (sub & ~3), odd);
        const int sc = static_cast<int8_t>((sw >> (8 * (sub & 3))) & 0xffu);
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const uint32_t qlw = l < 4 ? ql0 : ql1, qhw = l < 4 ? qh0 : qh1;
            const int byte = static_cast<int>((qlw >> (8 * (l & 3))) & 0xffu);
            const int nib = quarter < 2 ? (byte & 0xF) : (byte >> 4);
            const int hi = static_cast<int>((qhw >> (8 * (l & 3) + 2 * quarter)) & 3u);
            out[l] = d * static_cast<float>(sc) * static_cast<float>((nib | (hi << 4)) - 32);
        }
    } else {
        const uint32_t * hw = reinterpret_cast<const uint32_t *>(blk);
        const uint32_t h0 = hw[0], s0 = hw[1], s1 = hw[2], s2 = hw[3];
        const float d = h2f(static_cast<uint16_t>(h0 & 0xffffu));
        const float dmin = h2f(static_cast<uint16_t>(h0 >> 16));
        int sc, m;
        scale_min_k4(s0, s1, s2, j, sc, m);
        const float d1 = d * static_cast<float>(sc);
        const float m1 = dmin * static_cast<float>(m);
        const int g = j >> 1, high = j & 1;
        const uint8_t * qs = blk + (TYPE == LEVO_HIP_TYPE_Q5_K ? 48 : 16) + 32 * g + 8 * p;
        const uint2 q = *reinterpret_cast<const uint2 *>(qs);
        uint2 qh = uint2{0u, 0u};
        if constexpr (TYPE == LEVO_HIP_TYPE_Q5_K) qh = *reinterpret_cast<const uint2 *>(blk + 16 + 8 * p);
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const uint32_t qw = l < 4 ? q.x : q.y;
            const int byte = static_cast<int>((qw >> (8 * (l & 3))) & 0xffu);
            int code = high ? (byte >> 4) : (byte & 0xF);
            if constexpr (TYPE == LEVO_HIP_TYPE_Q5_K) {
                const uint32_t hw2 = l < 4 ? qh.x : qh.y;
                code += ((hw2 >> (8 * (l & 3) + j)) & 1u) ? 16 : 0;
            }
            out[l] = d1 * static_cast<float>(code) - m1;
        }
    }
    Out * o = dst + i * kQK + 32 * j + 8 * p;
#pragma unroll
    for (int l = 0; l < 8; ++l) {
        if constexpr (sizeof(Out) == 4) {
            o[l] = out[l];
        } else {
            o[l] = f2h(out[l]);
        }
    }
}

// ---- mat-vec: one wave per row, 8 lanes per super-block ----------------------

constexpr int kMaxVec = 8;
constexpr int kXVec = 6;         // activation dwordx4 a thread requests up front (24 KiB per workgroup)
constexpr int kMaxMats = 4;      // matrices of one launch
constexpr int kFusedBlocks = 16; // F32 activations quantized in the launch: n_vec * k / 256 <= 16

// One matrix of a launch: workgroups [first_wg, next matrix's first_wg).
struct kq_mat {
    const uint8_t * w;      // [rows][nb] blocks, 16-byte aligned
    float * y;              // [n_vec][y_pitch]
    int64_t y_pitch;
    int64_t rows;
    int64_t row_bytes;
    int64_t w_bytes;        // rows * row_bytes
    int32_t type;
    int32_t first_wg;
};

struct kq_params {
    kq_mat m[kMaxMats];
    int32_t n_mats;
    const uint8_t * x;      // [n_vec][nb] block_q8_K, or null
    const float * xf;       // F32 activations [n_vec][xf_pitch] (quantized in the launch), or null
    int64_t xf_pitch;
    int32_t nb;
    int32_t n_vec;
    int32_t x_lds_bytes;    // staged activations, 16-byte multiple
    int32_t stage_bytes;    // LDS bytes per wave for its weight span
};

// Registers of one unit (block ib, eighth u) of a row, read from the block's
// bytes in the wave's LDS stage (Q6_K: `odd` when the block starts 2 mod 4).
template <int TYPE>
struct kq_unit;

template <>
struct kq_unit<LEVO_HIP_TYPE_Q4_K> {
    u32x4 hd, qs;  // d, dmin, scales; 16 bytes of quants (32 weights)
    __device__ __forceinline__ void load(const uint8_t * blk, int u, bool) {
        hd = *reinterpret_cast<const u32x4 *>(blk);
        qs = *reinterpret_cast<const u32x4 *>(blk + 16 + 32 * (u >> 1) + 16 * (u & 1));
    }
};

template <>
struct kq_unit<LEVO_HIP_TYPE_Q5_K> {
    u32x4 hd, qh, qs;
    __device__ __forceinline__ void load(const uint8_t * blk, int u, bool) {
        hd = *reinterpret_cast<const u32x4 *>(blk);
        qh = *reinterpret_cast<const u32x4 *>(blk + 16 + 16 * (u & 1));
        qs = *reinterpret_cast<const u32x4 *>(blk + 48 + 32 * (u >> 1) + 16 * (u & 1));
    }
};

template <>
struct kq_unit<LEVO_HIP_TYPE_Q6_K> {
    uint32_t a0, a1, b0, b1, h0, h1, sw0, sw1;  // ql[l], ql[l + 32], qh[l] (8 l each), scales
    uint16_t d;
    __device__ __forceinline__ void load(const uint8_t * blk, int u, bool odd) {
        const int n = u >> 2, l0 = 8 * (u & 3);
        load_u32x2(blk, 64 * n + l0, odd, a0, a1);
        load_u32x2(blk, 64 * n + 32 + l0, odd, b0, b1);
        load_u32x2(blk, 128 + 32 * n + l0, odd, h0, h1);
        load_u32x2(blk, 192 + 8 * n, odd, sw0, sw1);
        d = *reinterpret_cast<const uint16_t *>(blk + 208);  // 2-byte load: stays in the block
    }
};

// Adds one unit's terms for every activation column to acc_d / acc_m.
// Q4_K / Q5_K unit u = (g = u / 2, h = u % 2): quants of sub-blocks 2 g (low
// nibbles) and 2 g + 1 (high), elements 64 g + 16 h + [0, 16) and + 32.
template <int TYPE, int NV>
__device__ __forceinline__ void kq_compute(const kq_unit<TYPE> & w, int ib, int u, int nb, int n_vec,
                                           const int8_t * xq, const float * xd, const int16_t * xs,
                                           float (&acc_d)[NV], float (&acc_m)[NV]) {
    if constexpr (TYPE == LEVO_HIP_TYPE_Q6_K) {
        const int n = u >> 2, l0 = 8 * (u & 3);
        const float dw = h2f(w.d);
        // scales of sub-blocks 8 n + 2 quarter + (u & 3) / 2
        const int sh = 8 * ((u & 3) >> 1);
        const int sc0 = static_cast<int8_t>((w.sw0 >> sh) & 0xffu);
        const int sc1 = static_cast<int8_t>((w.sw0 >> (sh + 16)) & 0xffu);
        const int sc2 = static_cast<int8_t>((w.sw1 >> sh) & 0xffu);
        const int sc3 = static_cast<int8_t>((w.sw1 >> (sh + 16)) & 0xffu);
        const uint32_t c00 = minus32((w.a0 & 0x0F0F0F0Fu) | ((w.h0 & 0x03030303u) << 4));
        const uint32_t c01 = minus32((w.a1 & 0x0F0F0F0Fu) | ((w.h1 & 0x03030303u) << 4));
        const uint32_t c10 = minus32((w.b0 & 0x0F0F0F0Fu) | (((w.h0 >> 2) & 0x03030303u) << 4));
        const uint32_t c11 = minus32((w.b1 & 0x0F0F0F0Fu) | (((w.h1 >> 2) & 0x03030303u) << 4));
        const uint32_t c20 = minus32(((w.a0 >> 4) & 0x0F0F0F0Fu) | (((w.h0 >> 4) & 0x03030303u) << 4));
        const uint32_t c21 = minus32(((w.a1 >> 4) & 0x0F0F0F0Fu) | (((w.h1 >> 4) & 0x03030303u) << 4));
        const uint32_t c30 = minus32(((w.b0 >> 4) & 0x0F0F0F0Fu) | (((w.h0 >> 6) & 0x03030303u) << 4));
        const uint32_t c31 = minus32(((w.b1 >> 4) & 0x0F0F0F0Fu) | (((w.h1 >> 6) & 0x03030303u) << 4));
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if (v < n_vec) {
                const int8_t * q8 = xq + (static_cast<int64_t>(v) * nb + ib) * kQK + 128 * n + l0;
                const uint2 x0 = *reinterpret_cast<const uint2 *>(q8);
                const uint2 x1 = *reinterpret_cast<const uint2 *>(q8 + 32);
                const uint2 x2 = *reinterpret_cast<const uint2 *>(q8 + 64);
                const uint2 x3 = *reinterpret_cast<const uint2 *>(q8 + 96);
                const int isum = __mul24(sc0, dot4(c00, x0.x, dot4(c01, x0.y, 0))) +
                                 __mul24(sc1, dot4(c10, x1.x, dot4(c11, x1.y, 0))) +
                                 __mul24(sc2, dot4(c20, x2.x, dot4(c21, x2.y, 0))) +
                                 __mul24(sc3, dot4(c30, x3.x, dot4(c31, x3.y, 0)));
                acc_d[v] += (dw * xd[v * nb + ib]) * static_cast<float>(isum);
            }
        }
    } else {
        const int g = u >> 1, h = u & 1;
        u32x4 lo, hi;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            lo[q] = w.qs[q] & 0x0F0F0F0Fu;
            hi[q] = (w.qs[q] >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (TYPE == LEVO_HIP_TYPE_Q5_K) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lo[q] |= ((w.qh[q] >> (2 * g)) & 0x01010101u) << 4;
                hi[q] |= ((w.qh[q] >> (2 * g + 1)) & 0x01010101u) << 4;
            }
        }
        int sc0, m0, sc1, m1;
        scale_min_k4(w.hd[1], w.hd[2], w.hd[3], 2 * g, sc0, m0);
        scale_min_k4(w.hd[1], w.hd[2], w.hd[3], 2 * g + 1, sc1, m1);
        const float dw = h2f(static_cast<uint16_t>(w.hd[0] & 0xffffu));
        const float dminw = h2f(static_cast<uint16_t>(w.hd[0] >> 16));
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if (v < n_vec) {
                const int64_t base = (static_cast<int64_t>(v) * nb + ib) * kQK + 64 * g + 16 * h;
                const u32x4 x0 = *reinterpret_cast<const u32x4 *>(xq + base);
                const u32x4 x1 = *reinterpret_cast<const u32x4 *>(xq + base + 32);
                int dl = 0, dh = 0;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    dl = dot4(lo[q], x0[q], dl);
                    dh = dot4(hi[q], x1[q], dh);
                }
                const int16_t * bs = xs + (v * nb + ib) * 16;
                const int isum = __mul24(sc0, dl) + __mul24(sc1, dh);
                const int msum = __mul24(m0, static_cast<int>(bs[4 * g + h])) + __mul24(m1, static_cast<int>(bs[4 * g + 2 + h]));
                const float dx = xd[v * nb + ib];
                acc_d[v] += (dw * dx) * static_cast<float>(isum);
                acc_m[v] += (dminw * dx) * static_cast<float>(msum);
            }
        }
    }
}

// LPR lanes per row, 64 / LPR rows per wave; lane li of its row's group
// takes the units li + LPR i (i < U) of the row's 8 nb units (unit = eighth of
// a 256-value block, 32 weights). Per workgroup (4 waves, 4 * 64 / LPR rows):
//   1. each wave requests its rows' contiguous weight bytes with coalesced
//      dwordx4 loads (CH chunks per lane, all in flight);
//   2. meanwhile the workgroup stages the Q8_K activations in LDS, re-laid out
//      so that each lane's quants are aligned: xq [n_vec][256 nb] int8, then
//      xd [n_vec][nb] float, xs [n_vec][16 nb] int16 (the bsums);
//   3. each wave stores its span to its LDS stage area; each lane parses its
//      units there and adds their terms; a reduction over the row's LPR lanes
//      gives y.
// WPR > 1 (LPR = 64): WPR waves share a row, each a contiguous part of its
// super-blocks; their partial sums meet in LDS and are added in wave order.
// The units of the wave's rows that lane li of row group g takes, parsed
// from the wave's LDS stage (the row's blocks kb0 .. kb0 + units / 8).
template <int TYPE, int LPR, int U, int NV>
__device__ __forceinline__ void kq_units(const uint8_t * stage, int lead, int g, int li, int row_bytes, int units,
                                         int kb0, int nb, int n_vec, const int8_t * xq, const float * xd,
                                         const int16_t * xs, float (&acc_d)[NV], float (&acc_m)[NV]) {
    constexpr int kBytes = TYPE == LEVO_HIP_TYPE_Q4_K ? 144 : TYPE == LEVO_HIP_TYPE_Q5_K ? 176 : 210;
#pragma unroll
    for (int i = 0; i < U; ++i) {
        const int unit = li + LPR * i;
        if (unit < units) {
            const int off = lead + g * row_bytes + (unit >> 3) * kBytes;
            kq_unit<TYPE> w;
            w.load(stage + off, unit & 7, (off & 2) != 0);
            kq_compute<TYPE, NV>(w, kb0 + (unit >> 3), unit & 7, nb, n_vec, xq, xd, xs, acc_d, acc_m);
        }
    }
}

// LPR lanes per row, 64 / LPR rows per wave; lane li of its row's group
// takes the units li + LPR i (i < U) of the row's 8 nb units (unit = eighth of
// a 256-value block, 32 weights). Per workgroup (4 waves, 4 * 64 / LPR rows of
// one matrix, the matrix's type chosen once per workgroup):
//   1. each wave requests its rows' contiguous weight bytes with coalesced
//      dwordx4 loads (CH chunks per lane, all in flight);
//   2. meanwhile the workgroup stages the Q8_K activations in LDS, laid out
//      so that each lane's quants are aligned: xq [n_vec][256 nb] int8, then
//      xd [n_vec][nb] float, xs [n_vec][16 nb] int16 (the bsums); FUSED: it
//      quantizes F32 activations into that layout itself, sixteen lanes per
//      block as levo_hip_quantize_q8_K does;
//   3. each wave stores its span to its LDS stage area; each lane parses its
//      units there and adds their terms; a reduction over the row's LPR lanes
//      gives y.
// WPR > 1 (LPR = 64): WPR waves share a row, each a contiguous part of its
// super-blocks; their partial sums meet in LDS and are added in wave order.
// TYPE: the weight type when every matrix of the launch has it, else 0 (the
// type read per workgroup from its matrix). ONE: a launch of one matrix (no
// per-workgroup matrix lookup: its fields load with the other arguments).
template <int TYPE, int LPR, int U, int CH, int WPR, bool FUSED, bool ONE, int NV>
__global__ __launch_bounds__(kThreads) void mul_mat_kquant_kernel(const kq_params p) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
    const int nb = p.nb;
    const int nblk = p.n_vec * nb;
    int8_t * xq = reinterpret_cast<int8_t *>(lds_raw);
    float * xd = reinterpret_cast<float *>(lds_raw + static_cast<size_t>(nblk) * kQK);
    int16_t * xs = reinterpret_cast<int16_t *>(xd + ((nblk + 3) & ~3));
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    uint8_t * stage = lds_raw + p.x_lds_bytes + wave * p.stage_bytes;
    constexpr int kRowsPerWave = 64 / LPR;
    // this workgroup's matrix (uniform) and its index within the matrix
    int mi = 0;
    if constexpr (!ONE) {
#pragma unroll
        for (int i = 1; i < kMaxMats; ++i) {
            if (i < p.n_mats && static_cast<int>(blockIdx.x) >= p.m[i].first_wg) mi = i;
        }
    }
    const kq_mat & M = p.m[mi];
    const int64_t lb = static_cast<int64_t>(blockIdx.x) - M.first_wg;
    const int kbytes = TYPE == LEVO_HIP_TYPE_Q4_K   ? 144
                       : TYPE == LEVO_HIP_TYPE_Q5_K ? 176
                       : TYPE == LEVO_HIP_TYPE_Q6_K ? 210
                                                    : static_cast<int>(M.row_bytes / nb);
    // 1. the wave's rows [row0, row0 + nrows): bytes [sb0, sb1); with WPR > 1
    //    the WPR waves of a row each take a contiguous part of its blocks,
    //    [kb0, kb1)
    int64_t row0;
    int nrows, kb0, kb1;
    if constexpr (WPR > 1) {
        row0 = lb * (kThreads / 64 / WPR) + wave / WPR;
        nrows = row0 < M.rows ? 1 : 0;
        const int qb = (nb + WPR - 1) / WPR;
        kb0 = (wave % WPR) * qb;
        kb1 = kb0 + qb < nb ? kb0 + qb : nb;
        if (kb0 >= kb1) nrows = 0;
    } else {
        row0 = (lb * (kThreads / 64) + wave) * kRowsPerWave;
        const int64_t left = M.rows - row0;
        nrows = left < kRowsPerWave ? (left > 0 ? static_cast<int>(left) : 0) : kRowsPerWave;
        kb0 = 0;
        kb1 = nb;
    }
    const int64_t sb0 = row0 * M.row_bytes + static_cast<int64_t>(kb0) * kbytes;
    const int64_t sb1 = WPR > 1 ? row0 * M.row_bytes + static_cast<int64_t>(kb1) * kbytes
                                : sb0 + nrows * M.row_bytes;
    u32x4 regs[CH];
    if constexpr (FUSED) {
        // F32 activations, block b = (vector b / nb, super-block b % nb),
        // sixteen lanes per block (q8_K_block16): block 4 wave + lane / 16,
        // requested first, then the weights; a group past the last block
        // computes on it and stores nothing
        const int fb = 4 * wave + (lane >> 4);
        const int fs = lane & 15;
        const int fbc = min(fb, nblk - 1);
        const f32x4 * fsrc = reinterpret_cast<const f32x4 *>(p.xf + (fbc / nb) * p.xf_pitch + (fbc % nb) * kQK + 16 * fs);
        const f32x4 xv[4] = {fsrc[0], fsrc[1], fsrc[2], fsrc[3]};
        load_span<CH>(M.w, M.w_bytes, sb0 & ~int64_t{15}, sb1, nrows > 0, lane, regs);
        {
            uint32_t pk[4];
            int bsum;
            float d;
            q8_K_block16(xv, fs, pk, bsum, d);
            if (fb < nblk) {
                reinterpret_cast<u32x4 *>(xq)[fb * 16 + fs] = u32x4{pk[0], pk[1], pk[2], pk[3]};
                xs[fb * 16 + fs] = static_cast<int16_t>(bsum);
                if (fs == 0) xd[fb] = d;
            }
        }
    } else {
        // The activations: n_vec * nb block_q8_K of 292 bytes (f32 d, int8
        // qs[256], int16 bsums[16]) go to LDS by whole pieces: 16 quant
        // chunks, the scale and 2 bsum chunks per block, chunk c of a region
        // at byte 16 c (LDS stores stay 16-byte aligned; the global reads are
        // 4-byte aligned). The first chunks are requested before the weights,
        // with no branch around them (surplus requests re-read the last
        // chunk): loads complete in issue order, so they are stored while the
        // weights are in flight.
        const uint8_t * xg = p.x;
        const auto qchunk = [&](int c) {
            return *reinterpret_cast<const u32x4 *>(xg + 292 * static_cast<int64_t>(c >> 4) + 4 + 16 * (c & 15));
        };
        const auto schunk = [&](int c) {
            return *reinterpret_cast<const u32x4 *>(xg + 292 * static_cast<int64_t>(c >> 1) + 260 + 16 * (c & 1));
        };
        const auto dword = [&](int b) {
            return *reinterpret_cast<const uint32_t *>(xg + 292 * static_cast<int64_t>(b));
        };
        const int n_q = 16 * nblk;
        u32x4 xr[kXVec];
#pragma unroll
        for (int j = 0; j < kXVec; ++j) xr[j] = qchunk(min(tid + kThreads * j, n_q - 1));
        const uint32_t d0 = dword(min(tid, nblk - 1));
        const u32x4 s0 = schunk(min(tid, 2 * nblk - 1));
        load_span<CH>(M.w, M.w_bytes, sb0 & ~int64_t{15}, sb1, nrows > 0, lane, regs);
        // 2. store them (and fetch any the first requests did not cover)
#pragma unroll
        for (int j = 0; j < kXVec; ++j) {
            const int c = tid + kThreads * j;
            if (c < n_q) reinterpret_cast<u32x4 *>(xq)[c] = xr[j];
        }
        if (tid < nblk) xd[tid] = __builtin_bit_cast(float, d0);
        if (tid < 2 * nblk) reinterpret_cast<u32x4 *>(xs)[tid] = s0;
        for (int c = tid + kThreads * kXVec; c < n_q; c += kThreads) reinterpret_cast<u32x4 *>(xq)[c] = qchunk(c);
        for (int b = tid + kThreads; b < nblk; b += kThreads) xd[b] = __builtin_bit_cast(float, dword(b));
        for (int c = tid + kThreads; c < 2 * nblk; c += kThreads) reinterpret_cast<u32x4 *>(xs)[c] = schunk(c);
    }
    lds_barrier();  // LDS only: the weight loads stay in flight
    // 3. parse and sum
    store_span<CH>(stage, M.w, M.w_bytes, sb0 & ~int64_t{15}, sb1, nrows > 0, lane, regs);
    wave_lds_fence();
    const int g = lane / LPR;
    const int li = lane % LPR;
    const bool live = g < nrows;
    const int lead = static_cast<int>(sb0 & 15);
    const int units = (kb1 - kb0) * 8;
    float acc_d[NV], acc_m[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc_d[v] = acc_m[v] = 0.0f;
    if (live) {
        const int rb = static_cast<int>(M.row_bytes);
        if constexpr (TYPE != 0) {
            kq_units<TYPE, LPR, U, NV>(stage, lead, g, li, rb, units, kb0, nb, p.n_vec, xq, xd, xs, acc_d, acc_m);
        } else if (M.type == LEVO_HIP_TYPE_Q4_K) {
            kq_units<LEVO_HIP_TYPE_Q4_K, LPR, U, NV>(stage, lead, g, li, rb, units, kb0, nb, p.n_vec, xq, xd, xs, acc_d,
                                                 acc_m);
        } else if (M.type == LEVO_HIP_TYPE_Q5_K) {
            kq_units<LEVO_HIP_TYPE_Q5_K, LPR, U, NV>(stage, lead, g, li, rb, units, kb0, nb, p.n_vec, xq, xd, xs, acc_d,
                                                 acc_m);
        } else {
            kq_units<LEVO_HIP_TYPE_Q6_K, LPR, U, NV>(stage, lead, g, li, rb, units, kb0, nb, p.n_vec, xq, xd, xs, acc_d,
                                                 acc_m);
        }
    }
    // every lane of the wave takes part in the shuffles (acc_m stays 0 for Q6_K)
    if constexpr (WPR > 1) {
        // the row's parts meet in LDS, each at the start of its wave's own
        // stage area (no longer read once the wave has computed), summed in
        // wave order
        float * part = reinterpret_cast<float *>(stage);
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if (v < p.n_vec) {
                const float sd = group_sum<LPR>(acc_d[v]);
                const float sm = group_sum<LPR>(acc_m[v]);
                if (lane == 0) {
                    part[2 * v] = sd;
                    part[2 * v + 1] = sm;
                }
            }
        }
        __syncthreads();
        if (wave % WPR == 0 && lane < p.n_vec && row0 < M.rows) {
            float sd = part[2 * lane], sm = part[2 * lane + 1];
#pragma unroll
            for (int w = 1; w < WPR; ++w) {
                const float * other = reinterpret_cast<const float *>(stage + w * p.stage_bytes);
                sd += other[2 * lane];
                sm += other[2 * lane + 1];
            }
            M.y[lane * M.y_pitch + row0] = sd - sm;
        }
    } else {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if (v < p.n_vec) {
                const float sd = group_sum<LPR>(acc_d[v]);
                const float sm = group_sum<LPR>(acc_m[v]);
                if (live && li == 0) M.y[v * M.y_pitch + row0 + g] = sd - sm;
            }
        }
    }
}

// NV: the accumulators per lane, 2 for the CFG pair (n_vec <= 2: the
// decode case, 3-6 % faster than the general instance), else 8.
template <int TYPE, int LPR, int U, int CH, int WPR, bool FUSED, int NV>
auto pick_kernel(const kq_params & p) {
    return TYPE != 0 && p.n_mats == 1 ? mul_mat_kquant_kernel<TYPE, LPR, U, CH, WPR, FUSED, true, NV>
                                      : mul_mat_kquant_kernel<TYPE, LPR, U, CH, WPR, FUSED, false, NV>;
}

template <int TYPE, int LPR, int U, int CH, int WPR, bool FUSED>
int launch_mul_mat_t(kq_params p, int64_t max_row_bytes, hipStream_t st) {
    const auto kernel = p.n_vec <= 2 ? pick_kernel<TYPE, LPR, U, CH, WPR, FUSED, 2>(p)
                                     : pick_kernel<TYPE, LPR, U, CH, WPR, FUSED, kMaxVec>(p);
    if (const int rc = allow_dynamic_lds(reinterpret_cast<const void *>(kernel), 160 * 1024, "levo_hip_mul_mat_kquant");
        rc != LEVO_HIP_OK)
        return rc;
    constexpr int kRowsPerWave = 64 / LPR;
    const int64_t span = WPR > 1 ? ceil_div(p.nb, WPR) * (max_row_bytes / p.nb) : kRowsPerWave * max_row_bytes;
    LEVO_REQUIRE(span + 15 <= int64_t{CH} * 64 * 16, "mul_mat_kquant: row span exceeds the wave's registers");
    LEVO_REQUIRE(WPR == 1 || ceil_div(p.nb, WPR) * 8 <= int64_t{U} * LPR, "mul_mat_kquant: row part exceeds the lanes");
    LEVO_REQUIRE(WPR > 1 || int64_t{p.nb} * 8 <= int64_t{U} * LPR, "mul_mat_kquant: row exceeds the lanes");
    p.stage_bytes = static_cast<int32_t>((span + 15 + 15) & ~int64_t{15});
    const size_t lds = static_cast<size_t>(p.x_lds_bytes) + static_cast<size_t>(kThreads / 64) * p.stage_bytes;
    LEVO_REQUIRE(lds <= 160 * 1024, "mul_mat_kquant: n_vec * k too large for the workgroup's LDS");
    const int64_t rows_per_block = WPR > 1 ? (kThreads / 64) / WPR : (kThreads / 64) * kRowsPerWave;
    int64_t wgs = 0;
    for (int i = 0; i < p.n_mats; ++i) {
        p.m[i].first_wg = static_cast<int32_t>(wgs);
        wgs += ceil_div(p.m[i].rows, rows_per_block);
    }
    LEVO_REQUIRE(wgs < (int64_t{1} << 31) / kThreads, "mul_mat_kquant: too many rows");
    kernel<<<dim3(static_cast<uint32_t>(wgs)), kThreads, lds, st>>>(p);
    return launch_status("levo_hip_mul_mat_kquant");
}

// The instance for the launch's types (one shared type, or mixed) and
// activation source. F32 activations (at most 16 blocks, so k <= 4096) only
// reach the geometries of up to 16 units per lane row.
template <int LPR, int U, int CH, int WPR = 1>
int launch_mul_mat_u(kq_params p, int64_t max_row_bytes, hipStream_t st) {
    int type = p.m[0].type;
    for (int i = 1; i < p.n_mats; ++i) type = p.m[i].type == type ? type : 0;
    constexpr bool kFusable = WPR == 1 && U * LPR <= 128;
    if (p.xf != nullptr) {
        if constexpr (kFusable) {
            switch (type) {
                case LEVO_HIP_TYPE_Q4_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q4_K, LPR, U, CH, WPR, true>(p, max_row_bytes, st);
                case LEVO_HIP_TYPE_Q5_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q5_K, LPR, U, CH, WPR, true>(p, max_row_bytes, st);
                case LEVO_HIP_TYPE_Q6_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q6_K, LPR, U, CH, WPR, true>(p, max_row_bytes, st);
                default: return launch_mul_mat_t<0, LPR, U, CH, WPR, true>(p, max_row_bytes, st);
            }
        } else {
            LEVO_REQUIRE(false, "mul_mat_kquant: F32 activations need k <= 4096");
        }
    }
    switch (type) {
        case LEVO_HIP_TYPE_Q4_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q4_K, LPR, U, CH, WPR, false>(p, max_row_bytes, st);
        case LEVO_HIP_TYPE_Q5_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q5_K, LPR, U, CH, WPR, false>(p, max_row_bytes, st);
        case LEVO_HIP_TYPE_Q6_K: return launch_mul_mat_t<LEVO_HIP_TYPE_Q6_K, LPR, U, CH, WPR, false>(p, max_row_bytes, st);
        default: return launch_mul_mat_t<0, LPR, U, CH, WPR, false>(p, max_row_bytes, st);
    }
}

// Lanes per row, units per lane and span chunks per lane by the row's 8 nb
// units (k <= 16384) and the largest matrix's rows: a wave's span is 64 / LPR
// rows, or half a row. Spans are sized for the largest row of the launch.
int launch_mul_mat(kq_params & p, hipStream_t st) {
    int64_t rows = 0, rb = 0;
    for (int i = 0; i < p.n_mats; ++i) {
        rows = p.m[i].rows > rows ? p.m[i].rows : rows;
        rb = p.m[i].row_bytes > rb ? p.m[i].row_bytes : rb;
    }
    const int units = p.nb * 8;
    if (units <= 64) {
        // K <= 2048: the fewest lanes per row (the most rows per workgroup,
        // each workgroup staging the activations once) that still give 256
        // workgroups or more: 16 rows per workgroup from 4096 rows, 8 from
        // 2048, else 4 (1536 x 1536 Q4_K 4.69 -> 3.68 us, Q6_K 5.29 -> 3.99;
        // at 8960 and 16385 rows 16 lanes per row stay fastest)
        // Instances sized to the span where it is smaller: every lane issues
        // all CH chunk loads and U unit iterations, so surplus ones cost
        // issue slots (K = 1536: 3 units and 5 chunks instead of 4 and 8,
        // 3-5 % at 8960 and 16385 rows; K = 2304 / 4608 below 11-13 %); the
        // lanes' units, and so the sums, stay the same.
        if (rows >= 4096) {
            if (units <= 48 && 4 * rb + 30 <= 5 * 64 * 16) return launch_mul_mat_u<16, 3, 5>(p, rb, st);
            return launch_mul_mat_u<16, 4, 8>(p, rb, st);
        }
        if (rows >= 2048) return launch_mul_mat_u<32, 2, 4>(p, rb, st);
        return launch_mul_mat_u<64, 1, 2>(p, rb, st);
    }
    if (units <= 128) {
        if (units <= 80 && 4 * rb + 30 <= 8 * 64 * 16) return launch_mul_mat_u<16, 5, 8>(p, rb, st);
        return launch_mul_mat_u<16, 8, 16>(p, rb, st);
    }
    if (units <= 256) {
        if (units <= 160 && 2 * rb + 30 <= 8 * 64 * 16) return launch_mul_mat_u<32, 5, 8>(p, rb, st);
        return launch_mul_mat_u<32, 8, 16>(p, rb, st);
    }
    // K > 8192 (LeLM's ffn_down, K = 8960): a row over two waves, each half
    // its super-blocks, so each lane takes ~2 units instead of ~4 (Q4_K
    // 10.2 -> 9.4 us). Up to 38 super-blocks the half-row spans fit 4 chunks
    // per lane and 3 units per lane (Q4_K 6.75 -> 6.40 us, Q6_K 7.9 -> 7.6 us
    // against 7 chunks and 4 units); one row per wave measured 6.9 / 8.8 us
    // and four waves per row 6.95 / 8.2 us.
    if (p.nb <= 38) return launch_mul_mat_u<64, 3, 4, 2>(p, rb, st);
    return launch_mul_mat_u<64, 4, 7, 2>(p, rb, st);
}

}  // namespace

bool is_kquant(levo_hip_type type) {
    return type == LEVO_HIP_TYPE_Q4_K || type == LEVO_HIP_TYPE_Q5_K || type == LEVO_HIP_TYPE_Q6_K;
}

int64_t kquant_block_bytes(levo_hip_type type) {
    switch (type) {
        case LEVO_HIP_TYPE_Q4_K: return 144;
        case LEVO_HIP_TYPE_Q5_K: return 176;
        case LEVO_HIP_TYPE_Q6_K: return 210;
        case LEVO_HIP_TYPE_Q8_K: return 292;
        default: return 0;
    }
}

// Dequantize k values (a multiple of 256) of a K-quant type; arguments checked by the caller.
int dequantize_kquant(levo_hip_type type, const void * src, void * dst, levo_hip_type dst_type, int64_t k,
                      hipStream_t st) {
    const int64_t nb = k / kQK;
    if (nb == 0) return LEVO_HIP_OK;
    const dim3 grid(static_cast<uint32_t>(ceil_div(nb * 32, kThreads)));
    const uint8_t * s = static_cast<const uint8_t *>(src);
    const bool f32 = dst_type == LEVO_HIP_TYPE_F32;
#define LEVO_DEQ(T)                                                                                         \
    if (f32) dequantize_kquant_kernel<T, float><<<grid, kThreads, 0, st>>>(s, static_cast<float *>(dst), nb); \
    else dequantize_kquant_kernel<T, uint16_t><<<grid, kThreads, 0, st>>>(s, static_cast<uint16_t *>(dst), nb)
    switch (type) {
        case LEVO_HIP_TYPE_Q4_K: LEVO_DEQ(LEVO_HIP_TYPE_Q4_K); break;
        case LEVO_HIP_TYPE_Q5_K: LEVO_DEQ(LEVO_HIP_TYPE_Q5_K); break;
        default: LEVO_DEQ(LEVO_HIP_TYPE_Q6_K); break;
    }
#undef LEVO_DEQ
    return launch_status("levo_hip_dequantize");
}

}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_quantize_q8_K(const float * x, void * y, int64_t k, levo_hip_stream_t stream) {
    LEVO_REQUIRE(k >= 0 && k % kQK == 0, "quantize_q8_K: k must be a multiple of 256");
    LEVO_REQUIRE(k < (int64_t{1} << 40), "quantize_q8_K: k too large");
    if (k == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(x != nullptr && y != nullptr, "quantize_q8_K: null pointer");
    LEVO_REQUIRE(aligned16(x), "quantize_q8_K: x must be 16-byte aligned");
    LEVO_REQUIRE((reinterpret_cast<uintptr_t>(y) & 3u) == 0, "quantize_q8_K: y must be 4-byte aligned");
    const int64_t nb = k / kQK;
    quantize_q8_K_kernel<<<static_cast<uint32_t>(ceil_div(nb, kThreads / 16)), kThreads, 0, as_hip(stream)>>>(
            x, static_cast<uint8_t *>(y), nb);
    return launch_status("levo_hip_quantize_q8_K");
}

namespace {

int mul_mat_kquant_launch(const levo_hip_mat_kquant * mats, int32_t n_mats, const void * x_blocks, const float * x,
                          int64_t x_pitch, int64_t k, int64_t n_vec, hipStream_t st) {
    LEVO_REQUIRE(n_mats >= 1 && n_mats <= kMaxMats, "mul_mat_kquant: 1 to 4 matrices per launch");
    LEVO_REQUIRE(mats != nullptr, "mul_mat_kquant: null matrix list");
    LEVO_REQUIRE(k > 0 && k % kQK == 0, "mul_mat_kquant: k must be a positive multiple of 256");
    LEVO_REQUIRE(k <= 16384, "mul_mat_kquant: k must be at most 16384");
    LEVO_REQUIRE(n_vec >= 1 && n_vec <= kMaxVec, "mul_mat_kquant: n_vec must be 1..8");
    const int64_t nb = k / kQK;
    const int64_t nblk = n_vec * nb;
    kq_params p{};
    p.n_mats = 0;
    for (int i = 0; i < n_mats; ++i) {
        const levo_hip_mat_kquant & m = mats[i];
        LEVO_REQUIRE(is_kquant(m.type), "mul_mat_kquant: weight type must be Q4_K, Q5_K or Q6_K");
        LEVO_REQUIRE(m.rows >= 0 && m.rows < (int64_t{1} << 31), "mul_mat_kquant: bad row count");
        LEVO_REQUIRE(m.y_pitch >= m.rows, "mul_mat_kquant: y_pitch smaller than rows");
        if (m.rows == 0) continue;
        LEVO_REQUIRE(m.weight != nullptr && m.y != nullptr, "mul_mat_kquant: null pointer");
        LEVO_REQUIRE(aligned16(m.weight), "mul_mat_kquant: weight must be 16-byte aligned");
        kq_mat & q = p.m[p.n_mats++];
        q.w = static_cast<const uint8_t *>(m.weight);
        q.y = m.y;
        q.y_pitch = m.y_pitch;
        q.rows = m.rows;
        q.row_bytes = nb * kquant_block_bytes(m.type);
        q.w_bytes = m.rows * q.row_bytes;
        q.type = static_cast<int32_t>(m.type);
        q.first_wg = 0;
    }
    if (p.n_mats == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE((x_blocks == nullptr) != (x == nullptr), "mul_mat_kquant: pass exactly one of x_blocks and x");
    if (x_blocks != nullptr) {
        LEVO_REQUIRE((reinterpret_cast<uintptr_t>(x_blocks) & 3u) == 0,
                     "mul_mat_kquant: x_blocks must be 4-byte aligned");
    } else {
        LEVO_REQUIRE(nblk <= kFusedBlocks,
                     "mul_mat_kquant: F32 activations take n_vec * k <= 4096 (quantize larger ones to Q8_K first)");
        LEVO_REQUIRE(aligned16(x) && x_pitch >= k && x_pitch % 4 == 0,
                     "mul_mat_kquant: x must be 16-byte aligned with x_pitch >= k, a multiple of 4");
    }
    p.x = static_cast<const uint8_t *>(x_blocks);
    p.xf = x;
    p.xf_pitch = x_pitch;
    p.nb = static_cast<int32_t>(nb);
    p.n_vec = static_cast<int32_t>(n_vec);
    // xq, then xd padded to 16 bytes, then xs (the kernel's layout)
    p.x_lds_bytes = static_cast<int32_t>(nblk * kQK + ((4 * nblk + 15) & ~int64_t{15}) + 32 * nblk);
    p.stage_bytes = 0;
    return launch_mul_mat(p, st);
}

}  // namespace

extern "C" int levo_hip_mul_mat_kquant(levo_hip_type type, const void * weight, const void * x_blocks, float * y,
                                       int64_t y_pitch, int64_t rows, int64_t k, int64_t n_vec,
                                       levo_hip_stream_t stream) {
    LEVO_REQUIRE(x_blocks != nullptr || rows == 0, "mul_mat_kquant: null pointer");
    const levo_hip_mat_kquant m{type, weight, y, y_pitch, rows};
    return mul_mat_kquant_launch(&m, 1, x_blocks, nullptr, 0, k, n_vec, as_hip(stream));
}

extern "C" int levo_hip_mul_mat_kquant_multi(const levo_hip_mat_kquant * mats, int32_t n_mats, const void * x_blocks,
                                             const float * x, int64_t x_pitch, int64_t k, int64_t n_vec,
                                             levo_hip_stream_t stream) {
    return mul_mat_kquant_launch(mats, n_mats, x_blocks, x, x_pitch, k, n_vec, as_hip(stream));
}
