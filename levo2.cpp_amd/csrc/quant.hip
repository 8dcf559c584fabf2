// Q8_0 / Q4_0 per-32-value block quantization and dequantization.
//
// Bit-exact restatement of ggml's reference block quantizers as reached from
// ggml_quantize_chunk (tools/levo-quantize.cpp:386-388):
//   Q8_0: amax = max|x|; d = amax/127; id = d ? 1/d : 0; qs = roundf(x*id)
//   Q4_0: max = first value of largest |x|; d = max/-8; id = d ? 1/d : 0;
//         q = min(15, (int8)(x*id + 8.5)); qs[j] = q[j] | q[j+16] << 4
// with d stored as IEEE F16 (RNE). Blocks are 34 / 18 bytes and therefore not
// naturally aligned; each wave quantizes a group of 8 or 16 consecutive blocks
// (a 16-byte-aligned byte range), assembles them in LDS and writes the group
// with dwordx4 stores, so every HBM access is coalesced and aligned.
//
// Source layout: lanes own 16 contiguous source bytes each (8 F16 or 4 F32
// values); 4 (F16) or 8 (F32) lanes form one block and reduce its max with
// cross-lane shuffles.
#include "common.hpp"

#include <type_traits>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kQ8Bytes = 34;
constexpr int kQ4Bytes = 18;

// (int8_t)f as x86-64 computes it for the reference: truncation, with the
// invalid (non-finite / out-of-int32) case giving 0x80000000 -> low byte 0.
__device__ __forceinline__ int trunc_i8(float f) {
    if (!(fabsf(f) < 2147483648.0f)) return 0;
    return static_cast<int8_t>(static_cast<int32_t>(f));
}

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

// Loads this lane's N source values (N = 8 for F16, 4 for F32) of column
// col0.. of one row, zero beyond src_cols (row padding, write_tensor :375-384).
template <typename S, int N, bool kVec>
__device__ __forceinline__ void load_src(const S * row, int64_t col0, int64_t src_cols, float (&x)[N]) {
    if constexpr (kVec) {
        if (col0 < src_cols) {
            if constexpr (std::is_same<S, uint16_t>::value) {
                const u16x8 v = *reinterpret_cast<const u16x8 *>(row + col0);
#pragma unroll
                for (int k = 0; k < N; ++k) x[k] = h2f(v[k]);
            } else {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(row + col0);
                x[0] = v.x;
                x[1] = v.y;
                x[2] = v.z;
                x[3] = v.w;
            }
        } else {
#pragma unroll
            for (int k = 0; k < N; ++k) x[k] = 0.0f;
        }
    } else {
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
}

__device__ __forceinline__ void lds_put16(uint8_t * lds, int off, uint32_t v16) {
    *reinterpret_cast<uint16_t *>(lds + off) = static_cast<uint16_t>(v16);
}

// QT block type; S source element; kVec = dwordx4 source path.
template <int QT, typename S, bool kVec>
__global__ __launch_bounds__(kThreads) void quantize_kernel(const S * __restrict__ src, int64_t src_cols,
                                                            int64_t src_stride, uint8_t * __restrict__ dst,
                                                            int64_t nblocks_row, int64_t nblocks, bool dst_vec) {
    constexpr bool kF16 = std::is_same<S, uint16_t>::value;
    constexpr int N = kF16 ? 8 : 4;           // values per lane
    constexpr int LPB = 32 / N;               // lanes per block
    constexpr int BPW = 64 / LPB;             // blocks per wave group
    constexpr int QB = qtraits<QT>::bytes;
    constexpr int GB = BPW * QB;              // group bytes (multiple of 16)
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][GB];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const int64_t b0 = group * BPW;
    const int part = lane % LPB;
    const int64_t blk = b0 + lane / LPB;
    const bool valid = blk < nblocks;
    uint8_t * lds = stage[wave];

    float x[N];
    if (valid) {
        const int64_t r = blk / nblocks_row;
        const int64_t cb = blk - r * nblocks_row;
        load_src<S, N, kVec>(src + r * src_stride, cb * 32 + part * N, src_cols, x);
    } else {
#pragma unroll
        for (int k = 0; k < N; ++k) x[k] = 0.0f;
    }
    const int lb = (lane / LPB) * QB;  // block offset in the group

    if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
        float amax = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k) amax = amax > fabsf(x[k]) ? amax : fabsf(x[k]);
#pragma unroll
        for (int o = 1; o < LPB; o <<= 1) {
            const float t = __shfl_xor(amax, o, 64);
            amax = amax > t ? amax : t;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        if (part == 0) lds_put16(lds, lb, f2h(d));
        uint32_t q[N];
#pragma unroll
        for (int k = 0; k < N; ++k) q[k] = static_cast<uint8_t>(trunc_i8(roundf(x[k] * id)));
#pragma unroll
        for (int k = 0; k < N; k += 2) lds_put16(lds, lb + 2 + part * N + k, q[k] | (q[k + 1] << 8));
    } else {
        // signed value of the first largest |x| (strictly greater replaces)
        float amax = 0.0f, vmax = 0.0f;
#pragma unroll
        for (int k = 0; k < N; ++k) {
            if (amax < fabsf(x[k])) {
                amax = fabsf(x[k]);
                vmax = x[k];
            }
        }
        int owner = part;
#pragma unroll
        for (int o = 1; o < LPB; o <<= 1) {
            const float ta = __shfl_xor(amax, o, 64);
            const float tv = __shfl_xor(vmax, o, 64);
            const int to = __shfl_xor(owner, o, 64);
            if (ta > amax || (ta == amax && to < owner)) {
                amax = ta;
                vmax = tv;
                owner = to;
            }
        }
        const float d = vmax / -8.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        if (part == 0) lds_put16(lds, lb, f2h(d));
        uint32_t nib = 0;  // this lane's N nibbles, value k at bits 4k
#pragma unroll
        for (int k = 0; k < N; ++k) {
            int qi = trunc_i8(x[k] * id + 8.5f);
            qi = qi < 15 ? qi : 15;
            nib |= (static_cast<uint32_t>(qi) & 0xfu) << (4 * k);
        }
        // values j (parts < LPB/2) pair with j + 16 (parts >= LPB/2)
        const uint32_t hi = __shfl_down(nib, LPB / 2, 64);
        if (part < LPB / 2) {
#pragma unroll
            for (int k = 0; k < N; k += 2) {
                const uint32_t b_lo = ((nib >> (4 * k)) & 0xfu) | (((hi >> (4 * k)) & 0xfu) << 4);
                const uint32_t b_hi = ((nib >> (4 * k + 4)) & 0xfu) | (((hi >> (4 * k + 4)) & 0xfu) << 4);
                lds_put16(lds, lb + 2 + part * N + k, b_lo | (b_hi << 8));
            }
        }
    }
    __syncthreads();

    // write the group: dwordx4 when the whole group is valid and dst is
    // 16-byte aligned (groups start at multiples of 16 bytes), u16 otherwise
    uint8_t * out = dst + b0 * QB;
    const int64_t nvalid = nblocks - b0;
    if (nvalid >= BPW && dst_vec) {
        if (lane < GB / 16)
            reinterpret_cast<u32x4 *>(out)[lane] = reinterpret_cast<const u32x4 *>(lds)[lane];
    } else if (nvalid > 0) {
        const int nbytes = static_cast<int>(nvalid < BPW ? nvalid : BPW) * QB;
        for (int i = lane; i < nbytes / 2; i += 64)
            reinterpret_cast<uint16_t *>(out)[i] = reinterpret_cast<const uint16_t *>(lds)[i];
    }
}

// Dequantize: each wave reads a group of 16 blocks (16-byte aligned range),
// stages it in LDS, and each lane expands 8 values of one block.
template <int QT, typename D>
__global__ __launch_bounds__(kThreads) void dequantize_kernel(const uint8_t * __restrict__ src, D * __restrict__ dst,
                                                              int64_t nblocks, bool src_vec, bool dst_vec) {
    constexpr int QB = qtraits<QT>::bytes;
    constexpr int BPW = 16;
    constexpr int GB = BPW * QB;
    __shared__ __attribute__((aligned(16))) uint8_t stage[kWaves][GB];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t group = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const int64_t b0 = group * BPW;
    const int64_t nvalid = nblocks - b0;
    uint8_t * lds = stage[wave];
    const uint8_t * in = src + b0 * QB;
    if (nvalid >= BPW && src_vec) {
        if (lane < GB / 16)
            reinterpret_cast<u32x4 *>(lds)[lane] = reinterpret_cast<const u32x4 *>(in)[lane];
    } else if (nvalid > 0) {
        const int nbytes = static_cast<int>(nvalid < BPW ? nvalid : BPW) * QB;
        for (int i = lane; i < nbytes / 2; i += 64)
            reinterpret_cast<uint16_t *>(lds)[i] = reinterpret_cast<const uint16_t *>(in)[i];
    }
    __syncthreads();
    const int bi = lane >> 2;
    const int part = lane & 3;
    if (bi >= nvalid) return;
    const uint8_t * blk = lds + bi * QB;
    const float d = h2f(*reinterpret_cast<const uint16_t *>(blk));
    float y[8];
    if constexpr (QT == LEVO_HIP_TYPE_Q8_0) {
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const uint16_t two = *reinterpret_cast<const uint16_t *>(blk + 2 + part * 8 + k);
            y[k] = static_cast<float>(static_cast<int8_t>(two & 0xffu)) * d;
            y[k + 1] = static_cast<float>(static_cast<int8_t>(two >> 8)) * d;
        }
    } else {
        const int j0 = (part & 1) * 8;     // qs byte index
        const int shift = (part >> 1) * 4;  // low nibbles: values 0..15, high: 16..31
#pragma unroll
        for (int k = 0; k < 8; k += 2) {
            const uint16_t two = *reinterpret_cast<const uint16_t *>(blk + 2 + j0 + k);
            y[k] = static_cast<float>(static_cast<int>((two >> shift) & 0xfu) - 8) * d;
            y[k + 1] = static_cast<float>(static_cast<int>((two >> (8 + shift)) & 0xfu) - 8) * d;
        }
    }
    // output values of this lane: block (b0+bi), values part*8 .. part*8+7
    // (Q4_0 part p holds values 8p..8p+7 too: parts 0,1 low nibbles, 2,3 high)
    const int64_t e0 = (b0 + bi) * 32 + part * 8;
    if (!dst_vec) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            if constexpr (std::is_same<D, float>::value) dst[e0 + k] = y[k];
            else dst[e0 + k] = f2h(y[k]);
        }
    } else if constexpr (std::is_same<D, float>::value) {
        f32x4 a, b;
        a.x = y[0]; a.y = y[1]; a.z = y[2]; a.w = y[3];
        b.x = y[4]; b.y = y[5]; b.z = y[6]; b.w = y[7];
        reinterpret_cast<f32x4 *>(dst + e0)[0] = a;
        reinterpret_cast<f32x4 *>(dst + e0)[1] = b;
    } else {
        u16x8 h;
#pragma unroll
        for (int k = 0; k < 8; ++k) h[k] = f2h(y[k]);
        *reinterpret_cast<u16x8 *>(dst + e0) = h;
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
    constexpr int N = std::is_same<S, uint16_t>::value ? 8 : 4;
    constexpr int BPW = 64 / (32 / N);
    const int64_t nb_row = dst_cols / 32;
    const int64_t nblocks = nrows * nb_row;
    const int64_t groups = ceil_div(nblocks, BPW);
    const int64_t grid = ceil_div(groups, kWaves);
    const bool vec = src_cols % N == 0 && src_stride % N == 0 && aligned16(src);
    const S * s = static_cast<const S *>(src);
    uint8_t * d = static_cast<uint8_t *>(dst);
    const bool dst_vec = aligned16(dst);
    if (vec)
        quantize_kernel<QT, S, true><<<grid, kThreads, 0, stream>>>(s, src_cols, src_stride, d, nb_row, nblocks, dst_vec);
    else
        quantize_kernel<QT, S, false><<<grid, kThreads, 0, stream>>>(s, src_cols, src_stride, d, nb_row, nblocks, dst_vec);
    return launch_status("levo_hip_quantize");
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int64_t levo_hip_row_size(levo_hip_type type, int64_t n_per_row) {
    const int64_t bb = block_bytes(type);
    LEVO_REQUIRE(bb > 0, "row_size: unsupported type %d", static_cast<int>(type));
    LEVO_REQUIRE(n_per_row >= 0 && n_per_row % 32 == 0, "row_size: row length must be a multiple of 32");
    return n_per_row / 32 * bb;
}

extern "C" int64_t levo_hip_quantize_rows(levo_hip_type type, const void * src, levo_hip_type src_type,
                                          int64_t src_cols, int64_t src_row_stride, void * dst,
                                          int64_t nrows, int64_t dst_cols, levo_hip_stream_t stream) {
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
    LEVO_REQUIRE(type == LEVO_HIP_TYPE_Q8_0 || type == LEVO_HIP_TYPE_Q4_0,
                 "quantize_chunk: unsupported block type %d", static_cast<int>(type));
    LEVO_REQUIRE(type != LEVO_HIP_TYPE_Q4_0 || imatrix == nullptr,
                 "quantize_chunk: Q4_0 with an importance matrix is not implemented");
    LEVO_REQUIRE(n_per_row > 0 && n_per_row % 32 == 0, "quantize_chunk: row length must be a multiple of 32");
    LEVO_REQUIRE(start >= 0 && start % n_per_row == 0, "quantize_chunk: start must be a row boundary");
    const int64_t row_size = n_per_row / 32 * block_bytes(type);
    uint8_t * d = dst ? static_cast<uint8_t *>(dst) + (start / n_per_row) * row_size : nullptr;
    return levo_hip_quantize_rows(type, src ? src + start : nullptr, LEVO_HIP_TYPE_F32, n_per_row, n_per_row, d,
                                  nrows, n_per_row, stream);
}

extern "C" int levo_hip_dequantize(levo_hip_type type, const void * src, void * dst, levo_hip_type dst_type,
                                   int64_t k, levo_hip_stream_t stream) {
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
    const int64_t grid = ceil_div(ceil_div(nblocks, 16), kWaves);
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
