// Q8_0 / Q4_0 per-32-value block quantization and dequantization.
//
// Bit-exact restatement of ggml's reference block quantizers as reached from
// ggml_quantize_chunk (tools/levo-quantize.cpp:386-388):
//   Q8_0: amax = max|x|; d = amax/127; id = d ? 1/d : 0; qs = roundf(x*id)
//   Q4_0: max = first value of largest |x|; d = max/-8; id = d ? 1/d : 0;
//         q = min(15, (int8)(x*id + 8.5)); qs[j] = q[j] | q[j+16] << 4
// with d stored as IEEE F16 (RNE). Blocks are 34 / 18 bytes and therefore not
// naturally aligned.
//
// Quantize: packed rows take two lanes per block, other layouts one lane per
// block; a wave's consecutive blocks (32 or 64: a 16-byte-aligned byte range)
// are assembled in LDS and written with streaming (nontemporal) dwordx4
// stores. Dequantize: a wave stages 32 blocks in LDS and writes their values
// as contiguous 16-byte chunks.
#include "common.hpp"
#include "quant_block.hpp"

#include <type_traits>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kQ8Bytes = 34;
constexpr int kQ4Bytes = 18;

template <int QT>
struct qtraits;
template <>
struct qtraits<LEVO_HIP_TYPE_Q8_0> {
    static constexpr int bytes = kQ8Bytes;
};
template <>
struct qtraits<LEVO_HIP_TYPE_Q4_0> {
    static constexpr int bytes = kQ4Bytes;
};

// Writes one block (F16 scale d16, then NW little-endian dwords of packed
// quants) to LDS at byte offset base = lane * (2 + 4 * NW) with 4-byte aligned
// stores only: base is 4-aligned for even lanes and 2 mod 4 for odd ones, so
// odd lanes store d16 and then the dwords as they are, even lanes store
// dwords shifted by 16 bits (d16 first) and the last half-word on its own.
template <int NW>
__device__ __forceinline__ void stage_block(uint8_t * lds, int lane, uint32_t d16, const uint32_t (&pk)[NW]) {
    constexpr int QB = 2 + 4 * NW;
    const int base = lane * QB;
    const bool odd = lane & 1;
    uint32_t * words = reinterpret_cast<uint32_t *>(lds + base + (odd ? 2 : 0));
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const uint32_t shifted = i == 0 ? (d16 | (pk[0] << 16)) : __builtin_amdgcn_alignbit(pk[i], pk[i - 1], 16);
        words[i] = odd ? pk[i] : shifted;
    }
    *reinterpret_cast<uint16_t *>(lds + base + (odd ? 0 : QB - 2)) =
            static_cast<uint16_t>(odd ? d16 : (pk[NW - 1] >> 16));
}

// Quantizes one block of 32 values in ggml's reference order and stages it
// in LDS (stage_block) for lane `lane`.
template <int QT>
__device__ __forceinline__ void quantize_block(const float (&x)[32], uint8_t * lds, int lane) {
    if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
        uint32_t pk[8];
        const uint16_t d16 = quantize_q8_0_block(x, pk);
        stage_block<8>(lds, lane, d16, pk);
    } else {
        // ggml's scan (the first value of largest |x|, NaN never taken) as
        // four independent scans of 8 values joined in order: the strict
        // comparison keeps the earliest quarter on ties, as the single scan
        // keeps the earliest value. The scan's amax is always |max|, so only
        // the signed value is kept and compared through |.| (a compare with
        // absolute-value operands and one select per value).
        float qv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            qv[q] = 0.0f;
#pragma unroll
            for (int k = 8 * q; k < 8 * q + 8; ++k) qv[q] = fabsf(qv[q]) < fabsf(x[k]) ? x[k] : qv[q];
        }
        float vmax = qv[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) vmax = fabsf(vmax) < fabsf(qv[q]) ? qv[q] : vmax;
        const float d = vmax / -8.0f;
        const float id = nan_if_inf(d != 0.0f ? 1.0f / d : 0.0f);
        uint32_t pk[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t b[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = 4 * w + k;
                const uint32_t c0 = low_byte_i8(x[j] * id + 8.5f);
                const uint32_t c1 = low_byte_i8(x[j + 16] * id + 8.5f);
                const uint32_t q0 = c0 < 15u ? c0 : 15u;
                const uint32_t q1 = c1 < 15u ? c1 : 15u;
                b[k] = q0 | (q1 << 4);
            }
            pk[w] = pack4(b[0], b[1], b[2], b[3]);
        }
        stage_block<4>(lds, lane, f2h(d), pk);
    }
}

__device__ __forceinline__ void wave_lds_fence() {
    // Only this wave touches its LDS region, and one wave's LDS operations
    // complete in issue order: a wavefront-scope fence is enough.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Packed rows (source value i of block b is src[32 b + i]), 16-byte aligned
// source, two lanes per block: lane 2 b + h of a wave quantizes half of
// block b of the wave's 32 (Q8_0: values 16 h .. 16 h + 15; Q4_0: values
// 8 h .. 8 h + 7 and 16 + 8 h .. 16 + 8 h + 7, the two of each packed byte),
// so each lane's chain from its loads to its stores is half as long as with a
// lane per block. The wave's 32 blocks are read with coalesced dwordx4 loads
// and transposed through LDS (each block in a 16-byte-padded slot). The
// halves meet with DPP swaps: their partial maxima (with the reference's
// index-order rule, below) and, at the end, the second half's quants, which
// the first lane stages with the block's scale.
template <int QT, typename S>
__global__ __launch_bounds__(kThreads) void quantize_pair_kernel(const S * __restrict__ src,
                                                                 uint8_t * __restrict__ dst, int64_t nblocks,
                                                                 bool dst_vec) {
    constexpr int QB = qtraits<QT>::bytes;
    constexpr int CPB = 32 * static_cast<int>(sizeof(S)) / 16;  // 16-byte chunks per block: 4 (F16) or 8 (F32)
    constexpr int CPL = CPB / 2;                                // chunks per lane
    constexpr int VPC = 16 / static_cast<int>(sizeof(S));       // values per chunk
    constexpr int SLOT = (CPB + 1) * 16;                        // padded block slot in LDS
    constexpr int STAGE = 32 * SLOT;                            // >= 32 * QB output bytes
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][STAGE];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int b = lane >> 1;
    const int h = lane & 1;
    const int64_t b0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 32;
    uint8_t * lds = stage[wave];
    const u32x4 * in = reinterpret_cast<const u32x4 *>(src);
    const int64_t last = nblocks * CPB - 1;  // last valid chunk of the source

    // Every load is issued before any is used: chunks past the end read the
    // last valid chunk (no branch around a load) and are zeroed afterwards.
    u32x4 v[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t g = b0 * CPB + lane + 64 * j;
        v[j] = __builtin_nontemporal_load(in + (g < last ? g : last));
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        if (b0 * CPB + lane + 64 * j > last) v[j] = u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        *reinterpret_cast<u32x4 *>(lds + (c / CPB) * SLOT + (c % CPB) * 16) = v[j];
    }
    wave_lds_fence();
    // this lane's 16 values, x[i] = block value at(i)
    float x[16];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        // Q8_0: chunks CPL h + j; Q4_0: the chunks of values 8 h .. and 16 + 8 h ..
        const int chunk = QT == LEVO_HIP_TYPE_Q8_0 ? CPL * h + j
                                                   : (j < CPL / 2 ? (8 * h) / VPC + j : (16 + 8 * h) / VPC + j - CPL / 2);
        const u32x4 w = *reinterpret_cast<const u32x4 *>(lds + b * SLOT + chunk * 16);
        if constexpr (std::is_same<S, uint16_t>::value) {
            const u16x8 hv = __builtin_bit_cast(u16x8, w);
#pragma unroll
            for (int k = 0; k < 8; ++k) x[j * 8 + k] = h2f(hv[k]);
        } else {
            // Cast the whole vector: ROCm 7.2's clang lowers a bit_cast of a
            // single ext_vector element (w.y, ...) as a cast of element 0.
            const f32x4 f = __builtin_bit_cast(f32x4, w);
            x[j * 4 + 0] = f.x;
            x[j * 4 + 1] = f.y;
            x[j * 4 + 2] = f.z;
            x[j * 4 + 3] = f.w;
        }
    }
    // The output reuses the stage: the fence keeps every read above ahead of
    // the writes below, and the wave's LDS operations execute in that order.
    wave_lds_fence();

    uint16_t d16;
    uint32_t pk[8];  // Q8_0: 4 dwords of this half's quants (8 once the halves meet); Q4_0: 2 (4)
    if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
        // amax = MAX(amax, |x|) in index order. Without a NaN that is the
        // largest |x|: the |x| bit patterns order like the values. A NaN makes
        // the running MAX restart at the next value, so a half holding one
        // ends the same whatever came before it: the block's amax is the
        // second half's own scan from 0 if it holds a NaN, else the first
        // half's scan continued over the second (restarting if the first
        // half's scan ended on its NaN).
        uint32_t bm = 0u;
#pragma unroll
        for (int k = 0; k < 16; ++k) bm = __builtin_elementwise_max(bm, __float_as_uint(x[k]) & 0x7fffffffu);
        const uint32_t bm_o = dpp::mov<dpp::kQuadXor1>(bm);
        const uint32_t bits_max = bm > bm_o ? bm : bm_o;
        const bool has_nan = bits_max > 0x7f800000u;  // the pair's (both lanes agree)
        float amax = __uint_as_float(bits_max);
        if (has_nan) {
            float fold = 0.0f;
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float a = fabsf(x[k]);
                fold = fold > a ? fold : a;
            }
            const float fold_o = dpp::mov<dpp::kQuadXor1>(fold);
            const float first = h ? fold_o : fold;          // the first half's scan from 0
            const uint32_t bm1 = h ? bm : bm_o;             // the second half's |x| maximum
            const float second = h ? fold : fold_o;         // the second half's scan from 0
            amax = bm1 > 0x7f800000u ? second
                                     : (first != first ? __uint_as_float(bm1) : fmaxf(first, __uint_as_float(bm1)));
        }
        const float d = amax / 127.0f;
        const float id = nan_if_inf(d != 0.0f ? 1.0f / d : 0.0f);
        if (!has_nan) {
            // |x * id| <= 128 (or NaN): the truncated int32's low byte is the
            // reference's (int8_t)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t q[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) q[k] = trunc_i32(half_away_offset(x[4 * w + k] * id));
                pk[w] = pack_low_bytes(q[0], q[1], q[2], q[3]);
            }
        } else {
            // earlier values may exceed amax and leave the int32 range:
            // there cvttss2si gives 0x80000000 (low byte 0)
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t q[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float vq = half_away_offset(x[4 * w + k] * id);
                    q[k] = __builtin_fabsf(vq) < 0x1p31f ? trunc_i32(vq) : 0u;
                }
                pk[w] = pack_low_bytes(q[0], q[1], q[2], q[3]);
            }
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) pk[4 + w] = dpp::mov<dpp::kQuadXor1>(pk[w]);
        d16 = f2h(d);
    } else {
        // ggml's scan (the first value of largest |x|, NaN never taken) in
        // the four quarters of 8 values, joined in order with strict
        // comparisons (the earliest quarter wins a tie, as the single scan
        // keeps the earliest value): this lane scans quarters h and 2 + h.
        float qa = 0.0f, qb = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) qa = fabsf(qa) < fabsf(x[k]) ? x[k] : qa;
#pragma unroll
        for (int k = 8; k < 16; ++k) qb = fabsf(qb) < fabsf(x[k]) ? x[k] : qb;
        const float oa = dpp::mov<dpp::kQuadXor1>(qa);
        const float ob = dpp::mov<dpp::kQuadXor1>(qb);
        const float q0 = h ? oa : qa, q1 = h ? qa : oa, q2 = h ? ob : qb, q3 = h ? qb : ob;
        float vmax = q0;
        vmax = fabsf(vmax) < fabsf(q1) ? q1 : vmax;
        vmax = fabsf(vmax) < fabsf(q2) ? q2 : vmax;
        vmax = fabsf(vmax) < fabsf(q3) ? q3 : vmax;
        const float d = vmax / -8.0f;
        const float id = nan_if_inf(d != 0.0f ? 1.0f / d : 0.0f);
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            uint32_t bq[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = 4 * w + k;  // byte 8 h + i: values 8 h + i and 16 + 8 h + i
                const uint32_t c0 = low_byte_i8(x[i] * id + 8.5f);
                const uint32_t c1 = low_byte_i8(x[8 + i] * id + 8.5f);
                bq[k] = (c0 < 15u ? c0 : 15u) | ((c1 < 15u ? c1 : 15u) << 4);
            }
            pk[w] = pack4(bq[0], bq[1], bq[2], bq[3]);
        }
#pragma unroll
        for (int w = 0; w < 2; ++w) pk[2 + w] = dpp::mov<dpp::kQuadXor1>(pk[w]);
        d16 = f2h(d);
    }
    if (h == 0) {
        if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
            stage_block<8>(lds, b, d16, pk);
        } else {
            const uint32_t q4[4] = {pk[0], pk[1], pk[2], pk[3]};
            stage_block<4>(lds, b, d16, q4);
        }
    }
    wave_lds_fence();

    uint8_t * out = dst + b0 * QB;
    const int64_t nvalid = nblocks - b0;
    if (nvalid >= 32 && dst_vec) {
        for (int i = lane; i < 32 * QB / 16; i += 64)
            __builtin_nontemporal_store(reinterpret_cast<const u32x4 *>(lds)[i], reinterpret_cast<u32x4 *>(out) + i);
    } else if (nvalid > 0) {
        const int nbytes = static_cast<int>(nvalid < 32 ? nvalid : 32) * QB;
        for (int i = lane; i < nbytes / 2; i += 64)
            reinterpret_cast<uint16_t *>(out)[i] = reinterpret_cast<const uint16_t *>(lds)[i];
    }
}

// QT block type; S source element; kVec: dwordx4 source loads.
// One lane quantizes one 32-value block, scanning it in index order exactly as
// ggml's reference quantizer (so the max, its first occurrence and NaN
// handling match); the wave's 64 blocks are assembled in LDS and written as
// 16-byte stores (64 * 34 and 64 * 18 bytes are multiples of 16).
template <int QT, typename S, bool kVec>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const S * __restrict__ src, int64_t src_cols,
                                                            int64_t src_stride, uint8_t * __restrict__ dst,
                                                            int64_t nblocks_row, int64_t nblocks, bool dense,
                                                            bool dst_vec) {
    constexpr int QB = qtraits<QT>::bytes;
    constexpr int GB = 64 * QB;
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][GB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t b0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * 64;
    const int64_t blk = b0 + lane;

    float x[32];
    if (blk < nblocks) {
        if (dense) {
            load_block<S, kVec>(src + blk * 32, 0, 32, x);
        } else {
            const int64_t r = blk / nblocks_row;
            const int64_t cb = blk - r * nblocks_row;
            load_block<S, kVec>(src + r * src_stride, cb * 32, src_cols, x);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 32; ++k) x[k] = 0.0f;
    }

    quantize_block<QT>(x, stage[wave], lane);
    wave_lds_fence();

    uint8_t * out = dst + b0 * QB;
    const uint8_t * lds = stage[wave];
    const int64_t nvalid = nblocks - b0;
    if (nvalid >= 64 && dst_vec) {
        for (int i = lane; i < GB / 16; i += 64)
            __builtin_nontemporal_store(reinterpret_cast<const u32x4 *>(lds)[i], reinterpret_cast<u32x4 *>(out) + i);
    } else if (nvalid > 0) {
        const int nbytes = static_cast<int>(nvalid < 64 ? nvalid : 64) * QB;
        for (int i = lane; i < nbytes / 2; i += 64)
            reinterpret_cast<uint16_t *>(out)[i] = reinterpret_cast<const uint16_t *>(lds)[i];
    }
}

// Dequantize: a wave expands 32 consecutive blocks. Their 32 * QB bytes (a
// 16-byte-aligned range) are staged in LDS; the output is written as 16-byte
// chunks with lane l taking chunks l, l + 64, ..., so every store instruction
// covers one contiguous 1 KiB span. Chunk c holds values (c % CPB) * VPC ..
// of block c / CPB.
template <int QT, typename D>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t * __restrict__ src, D * __restrict__ dst,
                                                              int64_t nblocks, bool src_vec, bool dst_vec) {
    constexpr int QB = qtraits<QT>::bytes;
    constexpr int BPW = 32;
    constexpr int GB = BPW * QB;
    constexpr int VPC = 16 / static_cast<int>(sizeof(D));  // values per 16-byte chunk: 4 (F32) or 8 (F16)
    constexpr int CPB = 32 / VPC;                          // chunks per block
    constexpr int CPL = BPW * CPB / 64;                    // chunks per lane
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][GB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t b0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * BPW;
    const int64_t nvalid = nblocks - b0;
    if (nvalid <= 0) return;  // whole wave; no barrier follows
    uint8_t * lds = stage[wave];
    const uint8_t * in = src + b0 * QB;
    if (nvalid >= BPW && src_vec) {
        for (int i = lane; i < GB / 16; i += 64)
            reinterpret_cast<u32x4 *>(lds)[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(in) + i);
    } else {
        const int nbytes = static_cast<int>(nvalid < BPW ? nvalid : BPW) * QB;
        for (int i = lane; i < nbytes / 2; i += 64)
            reinterpret_cast<uint16_t *>(lds)[i] = reinterpret_cast<const uint16_t *>(in)[i];
    }
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int c = lane + 64 * j;
        const int bi = c / CPB;
        const int part = c % CPB;
        if (bi >= nvalid) break;
        const uint8_t * blk = lds + bi * QB;
        const float d = h2f(*reinterpret_cast<const uint16_t *>(blk));
        float y[VPC];
#pragma unroll
        for (int k = 0; k < VPC; k += 2) {
            const int v = part * VPC + k;  // first of the two values
            if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
                const uint16_t two = *reinterpret_cast<const uint16_t *>(blk + 2 + v);
                y[k] = static_cast<float>(static_cast<int8_t>(two & 0xffu)) * d;
                y[k + 1] = static_cast<float>(static_cast<int8_t>(two >> 8)) * d;
            } else {
                // values 0..15: low nibbles of qs[0..15]; 16..31: high nibbles
                const uint16_t two = *reinterpret_cast<const uint16_t *>(blk + 2 + (v & 15));
                const int shift = (v >> 4) * 4;
                y[k] = static_cast<float>(static_cast<int>((two >> shift) & 0xfu) - 8) * d;
                y[k + 1] = static_cast<float>(static_cast<int>((two >> (8 + shift)) & 0xfu) - 8) * d;
            }
        }
        const int64_t e0 = (b0 + bi) * 32 + part * VPC;
        if (dst_vec) {
            if constexpr (std::is_same<D, float>::value) {
                f32x4 o;
                o.x = y[0];
                o.y = y[1];
                o.z = y[2];
                o.w = y[3];
                __builtin_nontemporal_store(o, reinterpret_cast<f32x4 *>(dst + e0));
            } else {
                u16x8 h;
#pragma unroll
                for (int k = 0; k < 8; ++k) h[k] = f2h(y[k]);
                __builtin_nontemporal_store(h, reinterpret_cast<u16x8 *>(dst + e0));
            }
        } else {
#pragma unroll
            for (int k = 0; k < VPC; ++k) {
                if constexpr (std::is_same<D, float>::value) dst[e0 + k] = y[k];
                else dst[e0 + k] = f2h(y[k]);
            }
        }
    }
}

int64_t block_bytes(levo_hip_type t) {
    if (t == LEVO_HIP_TYPE_Q8_0) return kQ8Bytes;
    if (t == LEVO_HIP_TYPE_Q4_0) return kQ4Bytes;
    return -1;
}

template <int QT, typename S>
int launch_quant(const void * src, int64_t src_cols, int64_t src_stride, void * dst, int64_t nrows,
                 int64_t dst_cols, hipStream_t stream) {
    const int64_t nb_row = dst_cols / 32;
    const int64_t nblocks = nrows * nb_row;
    const int64_t grid = ceil_div(nblocks, 64 * kWaves);
    // dwordx4 loads need every row start 16-byte aligned
    const bool vec = aligned16(src) && (src_stride * static_cast<int64_t>(sizeof(S))) % 16 == 0;
    // rows packed back to back with no padding: block b is source values 32b..32b+31
    const bool dense = src_cols == dst_cols && src_stride == src_cols;
    const S * s = static_cast<const S *>(src);
    uint8_t * d = static_cast<uint8_t *>(dst);
    const bool dst_vec = aligned16(dst);
    if (vec && dense)
        quantize_pair_kernel<QT, S><<<ceil_div(nblocks, 32 * kWaves), kThreads, 0, stream>>>(s, d, nblocks, dst_vec);
    else if (vec)
        quantize_kernel<QT, S, true><<<grid, kThreads, 0, stream>>>(s, src_cols, src_stride, d, nb_row, nblocks, dense, dst_vec);
    else
        quantize_kernel<QT, S, false><<<grid, kThreads, 0, stream>>>(s, src_cols, src_stride, d, nb_row, nblocks, dense, dst_vec);
    return launch_status("levo_hip_quantize");
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int64_t levo_hip_row_size(levo_hip_type type, int64_t n_per_row) {
    if (const int64_t kb = kquant_block_bytes(type)) {
        LEVO_REQUIRE(n_per_row >= 0 && n_per_row % 256 == 0, "row_size: row length must be a multiple of 256");
        return n_per_row / 256 * kb;
    }
    const int64_t bb = block_bytes(type);
    LEVO_REQUIRE(bb > 0, "row_size: unsupported type %d", static_cast<int>(type));
    LEVO_REQUIRE(n_per_row >= 0 && n_per_row % 32 == 0, "row_size: row length must be a multiple of 32");
    return n_per_row / 32 * bb;
}

extern "C" int64_t levo_hip_quantize_rows(levo_hip_type type, const void * src, levo_hip_type src_type,
                                          int64_t src_cols, int64_t src_row_stride, void * dst,
                                          int64_t nrows, int64_t dst_cols, levo_hip_stream_t stream) {
    if (type == LEVO_HIP_TYPE_Q4_K || type == LEVO_HIP_TYPE_Q5_K || type == LEVO_HIP_TYPE_Q6_K) {
        LEVO_REQUIRE(src_type == LEVO_HIP_TYPE_F32 || src_type == LEVO_HIP_TYPE_F16,
                     "quantize: source must be F32 or F16");
        LEVO_REQUIRE(nrows >= 0 && src_cols >= 0 && dst_cols >= 0, "quantize: negative shape");
        LEVO_REQUIRE(dst_cols % 256 == 0, "quantize: K-quant storage width must be a multiple of 256");
        LEVO_REQUIRE(dst_cols >= src_cols, "quantize: storage width is smaller than the source width");
        LEVO_REQUIRE(src_row_stride >= src_cols, "quantize: source row stride is smaller than the width");
        const int64_t bytes = nrows * (dst_cols / 256) * kquant_block_bytes(type);
        if (bytes == 0) return 0;
        LEVO_REQUIRE(src != nullptr && dst != nullptr, "quantize: null pointer");
        LEVO_REQUIRE((reinterpret_cast<uintptr_t>(src) & (src_type == LEVO_HIP_TYPE_F16 ? 1u : 3u)) == 0,
                     "quantize: source is not aligned to its element size");
        const int r = quantize_kquant_rows(type, src, src_type, src_cols, src_row_stride, dst, nrows, dst_cols,
                                           as_hip(stream));
        return r == LEVO_HIP_OK ? bytes : r;
    }
    LEVO_REQUIRE(type == LEVO_HIP_TYPE_Q8_0 || type == LEVO_HIP_TYPE_Q4_0,
                 "quantize: unsupported block type %d", static_cast<int>(type));
    LEVO_REQUIRE(src_type == LEVO_HIP_TYPE_F32 || src_type == LEVO_HIP_TYPE_F16,
                 "quantize: source must be F32 or F16");
    LEVO_REQUIRE(nrows >= 0 && src_cols >= 0 && dst_cols >= 0, "quantize: negative shape");
    LEVO_REQUIRE(dst_cols % 32 == 0, "quantize: storage width must be a multiple of 32");
    LEVO_REQUIRE(dst_cols >= src_cols, "quantize: storage width is smaller than the source width");
    LEVO_REQUIRE(src_row_stride >= src_cols, "quantize: source row stride is smaller than the width");
    const int64_t bytes = nrows * (dst_cols / 32) * block_bytes(type);
    if (bytes == 0) return 0;
    LEVO_REQUIRE(nrows * (dst_cols / 32) < (int64_t{1} << 31), "quantize: more than 2^31 - 1 blocks in one call");
    LEVO_REQUIRE(src != nullptr && dst != nullptr, "quantize: null pointer");
    LEVO_REQUIRE((reinterpret_cast<uintptr_t>(dst) & 1u) == 0, "quantize: destination must be 2-byte aligned");
    LEVO_REQUIRE((reinterpret_cast<uintptr_t>(src) & (src_type == LEVO_HIP_TYPE_F16 ? 1u : 3u)) == 0,
                 "quantize: source is not aligned to its element size");
    const hipStream_t st = as_hip(stream);
    int r;
    if (type == LEVO_HIP_TYPE_Q8_0) {
        r = src_type == LEVO_HIP_TYPE_F16
                ? launch_quant<LEVO_HIP_TYPE_Q8_0, uint16_t>(src, src_cols, src_row_stride, dst, nrows, dst_cols, st)
                : launch_quant<LEVO_HIP_TYPE_Q8_0, float>(src, src_cols, src_row_stride, dst, nrows, dst_cols, st);
    } else {
        r = src_type == LEVO_HIP_TYPE_F16
                ? launch_quant<LEVO_HIP_TYPE_Q4_0, uint16_t>(src, src_cols, src_row_stride, dst, nrows, dst_cols, st)
                : launch_quant<LEVO_HIP_TYPE_Q4_0, float>(src, src_cols, src_row_stride, dst, nrows, dst_cols, st);
    }
    return r == LEVO_HIP_OK ? bytes : r;
}

extern "C" int64_t levo_hip_quantize_chunk(levo_hip_type type, const float * src, void * dst, int64_t start,
                                           int64_t nrows, int64_t n_per_row, const float * imatrix,
                                           levo_hip_stream_t stream) {
    const bool kq = type == LEVO_HIP_TYPE_Q4_K || type == LEVO_HIP_TYPE_Q5_K || type == LEVO_HIP_TYPE_Q6_K;
    LEVO_REQUIRE(type == LEVO_HIP_TYPE_Q8_0 || type == LEVO_HIP_TYPE_Q4_0 || kq,
                 "quantize_chunk: unsupported block type %d", static_cast<int>(type));
    LEVO_REQUIRE(type == LEVO_HIP_TYPE_Q8_0 || imatrix == nullptr,
                 "quantize_chunk: this block type with an importance matrix is not implemented");
    LEVO_REQUIRE(n_per_row > 0 && n_per_row % (kq ? 256 : 32) == 0,
                 kq ? "quantize_chunk: K-quant row length must be a multiple of 256"
                    : "quantize_chunk: row length must be a multiple of 32");
    LEVO_REQUIRE(start >= 0 && start % n_per_row == 0, "quantize_chunk: start must be a row boundary");
    const int64_t row_size = kq ? n_per_row / 256 * kquant_block_bytes(type) : n_per_row / 32 * block_bytes(type);
    uint8_t * d = dst ? static_cast<uint8_t *>(dst) + (start / n_per_row) * row_size : nullptr;
    return levo_hip_quantize_rows(type, src ? src + start : nullptr, LEVO_HIP_TYPE_F32, n_per_row, n_per_row, d,
                                  nrows, n_per_row, stream);
}

extern "C" int levo_hip_dequantize(levo_hip_type type, const void * src, void * dst, levo_hip_type dst_type,
                                   int64_t k, levo_hip_stream_t stream) {
    if (is_kquant(type)) {
        LEVO_REQUIRE(dst_type == LEVO_HIP_TYPE_F32 || dst_type == LEVO_HIP_TYPE_F16,
                     "dequantize: destination must be F32 or F16");
        LEVO_REQUIRE(k >= 0 && k % 256 == 0 && k < (int64_t{1} << 40), "dequantize: k must be a multiple of 256");
        if (k == 0) return LEVO_HIP_OK;
        LEVO_REQUIRE(src != nullptr && dst != nullptr, "dequantize: null pointer");
        LEVO_REQUIRE(aligned16(src), "dequantize: K-quant source must be 16-byte aligned");
        LEVO_REQUIRE((reinterpret_cast<uintptr_t>(dst) & (dst_type == LEVO_HIP_TYPE_F16 ? 1u : 3u)) == 0,
                     "dequantize: destination is not aligned to its element size");
        return dequantize_kquant(type, src, dst, dst_type, k, as_hip(stream));
    }
    LEVO_REQUIRE(type == LEVO_HIP_TYPE_Q8_0 || type == LEVO_HIP_TYPE_Q4_0,
                 "dequantize: unsupported block type %d", static_cast<int>(type));
    LEVO_REQUIRE(dst_type == LEVO_HIP_TYPE_F32 || dst_type == LEVO_HIP_TYPE_F16,
                 "dequantize: destination must be F32 or F16");
    LEVO_REQUIRE(k >= 0 && k % 32 == 0, "dequantize: k must be a multiple of 32");
    if (k == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(src != nullptr && dst != nullptr, "dequantize: null pointer");
    LEVO_REQUIRE((reinterpret_cast<uintptr_t>(src) & 1u) == 0, "dequantize: source must be 2-byte aligned");
    LEVO_REQUIRE((reinterpret_cast<uintptr_t>(dst) & (dst_type == LEVO_HIP_TYPE_F16 ? 1u : 3u)) == 0,
                 "dequantize: destination is not aligned to its element size");
    const bool src_vec = aligned16(src);
    const bool dst_vec = aligned16(dst);
    const int64_t nblocks = k / 32;
    const int64_t grid = ceil_div(ceil_div(nblocks, 32), kWaves);
    const hipStream_t st = as_hip(stream);
    const uint8_t * s = static_cast<const uint8_t *>(src);
    if (type == LEVO_HIP_TYPE_Q8_0) {
        if (dst_type == LEVO_HIP_TYPE_F32)
            dequantize_kernel<LEVO_HIP_TYPE_Q8_0, float><<<grid, kThreads, 0, st>>>(s, static_cast<float *>(dst), nblocks, src_vec, dst_vec);
        else
            dequantize_kernel<LEVO_HIP_TYPE_Q8_0, uint16_t><<<grid, kThreads, 0, st>>>(s, static_cast<uint16_t *>(dst), nblocks, src_vec, dst_vec);
    } else {
        if (dst_type == LEVO_HIP_TYPE_F32)
            dequantize_kernel<LEVO_HIP_TYPE_Q4_0, float><<<grid, kThreads, 0, st>>>(s, static_cast<float *>(dst), nblocks, src_vec, dst_vec);
        else
            dequantize_kernel<LEVO_HIP_TYPE_Q4_0, uint16_t><<<grid, kThreads, 0, st>>>(s, static_cast<uint16_t *>(dst), nblocks, src_vec, dst_vec);
    }
    return launch_status("levo_hip_dequantize");
}
