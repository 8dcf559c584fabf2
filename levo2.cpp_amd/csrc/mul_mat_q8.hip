// Decode mat-vec with Q8_0 weights and Q8_0 activations:
// y[v][r] = sum_b (float)sumi(W[r][b], X[v][b]) * (d_w * d_x), the
// ggml_vec_dot_q8_0_q8_0 that ggml's CPU mul_mat runs for a Q8_0 weight once
// the activation columns are quantized to Q8_0 (its vec_dot_type); the
// quantized LeLM / Flow matrices (src/levo-quantization.h:96-118) take it at
// every decode step. sumi is the exact int32 dot of the two blocks' quants;
// the F32 terms are summed in a different order than ggml's loop, so outputs
// agree to F32 rounding. The activations come quantized (for example by
// levo_hip_quantize_chunk), once per input vector, so the GEMVs that share an
// input (q / k / v, gate / up) share the quantization too.
//
// One 256-thread workgroup (4 waves) per group of rows, all launched at
// once so that the whole matrix is requested up front; per workgroup:
//   1. each wave issues coalesced dwordx4 loads of its span of weight blocks
//      (contiguous bytes, at most 256 blocks = 8704 B);
//   2. while they are in flight the workgroup stages the activation blocks
//      and unpacks them in LDS (quants as aligned dwords, scales as F32);
//   3. the wave stores its span in LDS and computes: a group of LPR lanes
//      per row, each lane a strided subset of the row's blocks, v_dot4 for
//      sumi, then the F32 term; a shuffle reduction over the group gives y.
// Geometry by blocks per row nb: nb <= 64: 16 lanes per row (16 rows per
// workgroup); nb <= 128: 32 lanes (8 rows); nb <= 256: 64 lanes (4 rows);
// nb <= 512 / 1024: a row is split over 2 / 4 waves (2 / 1 rows per
// workgroup), whose partial sums meet in LDS in wave order (LeLM's
// ffn_down, K = 8960 / 11008).
//
// levo_hip_mul_mat_q8_0_multi runs up to four matrices that read the same
// activation columns (q / k / v, gate / up) in one launch: each matrix owns
// a contiguous range of workgroups. It can also take the activations in F32
// and quantize them inside the launch (the block function of
// levo_hip_quantize_chunk, two lanes per block up to 128 blocks, one lane
// per block up to 256; requested before the weights and computed while they
// are in flight), for n_vec * K / 32 <= 256 blocks; the results equal
// levo_hip_quantize_chunk + levo_hip_mul_mat_q8_0 bit for bit.
#include "common.hpp"
#include "quant_block.hpp"
#include "span_load.hpp"

#include <algorithm>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kQ8Bytes = 34;
constexpr int kSpanBlocks = 256;
constexpr int kChunksPerLane = (kSpanBlocks * kQ8Bytes + 15 + 15) / 16 / 64 + 1;
constexpr int kMaxVectors = 8;
constexpr int kXChunks = 5;  // activation chunks per thread loaded up front (20 KiB per workgroup)
constexpr int kMaxBlocksPerRow = 1024;

constexpr int kMaxMats = 4;
// The activations' form: Q8_0 blocks, F32 values quantized in the launch, or
// columns (levo_hip_quantize_q8_0_columns: quants in value order, then F32 scales).
constexpr int kXBlocks = 0;
constexpr int kXF32 = 1;
constexpr int kXColumns = 2;
constexpr int kXF32Pair = 3;  // F32 values, two lanes per block (n_vec * K / 32 <= 128)

struct mm_params {
    const uint8_t * w;    // [rows][nb] weight blocks, 16-byte aligned
    const uint8_t * x;    // [n_vec][nb] activation blocks, 16-byte aligned
    float * y;            // [n_vec][y_pitch]
    int64_t rows;
    int64_t w_bytes;      // rows * nb * 34
    int64_t y_pitch;
    int32_t nb;           // blocks per row (K / 32)
    int32_t n_vec;
    int32_t stage_bytes;  // LDS bytes per wave for its weight span
};

// One launch over n_mats matrices sharing the activations: matrix m takes
// workgroups [first[m], first[m + 1]). p holds the shared fields (x, nb,
// n_vec, stage_bytes); w / y / rows / y_pitch are per matrix. With xf the
// activations come in F32 ([n_vec][x_pitch], 16-byte aligned rows) and are
// quantized in the workgroup.
struct mm_launch {
    mm_params p;
    const uint8_t * w[kMaxMats];
    float * y[kMaxMats];
    int64_t rows[kMaxMats];
    int64_t y_pitch[kMaxMats];
    int32_t first[kMaxMats + 1];
    int32_t n_mats;
    const float * xf;
    int64_t x_pitch;
};

// Block at LDS byte offset `off` (even): its F16 scale and 8 quant dwords.
// The quants start at off + 2; the dwords read from (off + 2) & ~3 hold them
// shifted by 0 (off = 2 mod 4) or 16 bits (off = 0 mod 4).
__device__ __forceinline__ float read_block(const uint8_t * stage, int off, uint32_t (&q)[8]) {
    const int qa = (off + 2) & ~3;
    const uint32_t * wd = reinterpret_cast<const uint32_t *>(stage + qa);
    uint32_t w[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) w[i] = wd[i];
    const uint32_t shift = (off & 2) ? 0u : 16u;
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = __builtin_amdgcn_alignbit(w[i + 1], w[i], shift);
    return h2f(*reinterpret_cast<const uint16_t *>(stage + off));
}

// The dwords of chunk c below xbytes (a multiple of 4), global -> LDS.
__device__ __forceinline__ void copy_tail_dwords(uint8_t * dst, const uint8_t * src, int64_t xbytes, int c) {
    const int64_t at = 16 * static_cast<int64_t>(c);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (at + 4 * k + 4 <= xbytes) {
            *reinterpret_cast<uint32_t *>(dst + at + 4 * k) = *reinterpret_cast<const uint32_t *>(src + at + 4 * k);
        }
    }
}

// 16-byte chunk c of the activation blocks (xbytes long); the last, partial
// chunk is read as half-words so nothing past the buffer is touched.
__device__ __forceinline__ u32x4 load_x_chunk(const uint8_t * x, int64_t xbytes, int c) {
    const int64_t at = 16 * static_cast<int64_t>(c);
    if (at + 16 <= xbytes) return *reinterpret_cast<const u32x4 *>(x + at);
    uint32_t h[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) h[k] = at + 2 * k + 2 <= xbytes ? *reinterpret_cast<const uint16_t *>(x + at + 2 * k) : 0u;
    return u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
}

// Rows and blocks of wave `wave` in workgroup `grp`: WPR waves share a row
// (each a contiguous part of its blocks), a wave of a WPR = 1 geometry takes
// 64 / LPR whole rows. Returns false when the wave has nothing to do.
template <int LPR, int WPR>
__device__ __forceinline__ bool wave_span(const mm_params & p, int64_t grp, int wave, int64_t & row0, int & nrows,
                                          int & kb0, int & kb1) {
    if constexpr (WPR > 1) {
        row0 = grp * (kWaves / WPR) + wave / WPR;
        nrows = 1;
        const int q = (p.nb + WPR - 1) / WPR;
        kb0 = (wave % WPR) * q;
        kb1 = kb0 + q < p.nb ? kb0 + q : p.nb;
        return row0 < p.rows && kb0 < kb1;
    } else {
        constexpr int RPW = 64 / LPR;
        row0 = (grp * kWaves + wave) * RPW;
        const int64_t left = p.rows - row0;
        nrows = left < RPW ? (left > 0 ? static_cast<int>(left) : 0) : RPW;
        kb0 = 0;
        kb1 = p.nb;
        return nrows > 0;
    }
}

// One block's terms for every activation column: sumi by 8 v_dot4 over the
// block's quant dwords q, then acc[v] += sumi * (d_w * d_x).
template <int NV>
__device__ __forceinline__ void block_terms(const uint32_t (&q)[8], float dw, const uint32_t * xq, const float * dx,
                                            int nb, int kb, int n_vec, float (&acc)[NV]) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        if (v >= n_vec) break;
        const u32x4 * xb = reinterpret_cast<const u32x4 *>(xq + (v * nb + kb) * 8);
        const u32x4 x0 = xb[0];
        const u32x4 x1 = xb[1];
        int s = 0;
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[0]), static_cast<int>(x0.x), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[1]), static_cast<int>(x0.y), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[2]), static_cast<int>(x0.z), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[3]), static_cast<int>(x0.w), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[4]), static_cast<int>(x1.x), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[5]), static_cast<int>(x1.y), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[6]), static_cast<int>(x1.z), s, false);
        s = __builtin_amdgcn_sdot4(static_cast<int>(q[7]), static_cast<int>(x1.w), s, false);
        acc[v] += static_cast<float>(s) * (dw * dx[v * nb + kb]);
    }
}

// quantize_q8_0_block over the two lanes of a pair (lane h of the pair
// holds values 16 h .. 16 h + 15 in v): the |x| maximum joined by one DPP
// step, the index-order NaN scan (rare) reading the pair's values lane by
// lane; each lane's 16 quants as 4 dwords; d as F16 in both lanes. The
// same bits as quantize_q8_0_block; half its dependent chain per lane and
// half the loads per thread (ffn gate/up 8960 x 1536 with its input
// quantized in the launch 6.16 -> 5.54 us). Every lane of the wave runs it
// (the DPP step reads the partner lane).
__device__ __forceinline__ uint16_t quantize_q8_0_block_x2(const u32x4 (&v)[4], uint32_t (&pk)[4]) {
    float x[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[4 * i] = __uint_as_float(v[i].x);
        x[4 * i + 1] = __uint_as_float(v[i].y);
        x[4 * i + 2] = __uint_as_float(v[i].z);
        x[4 * i + 3] = __uint_as_float(v[i].w);
    }
    uint32_t bits_max = 0u;
#pragma unroll
    for (int k = 0; k < 16; ++k) bits_max = __builtin_elementwise_max(bits_max, __float_as_uint(x[k]) & 0x7fffffffu);
    bits_max = __builtin_elementwise_max(bits_max, dpp::mov<dpp::kQuadXor1>(bits_max));
    const bool has_nan = bits_max > 0x7f800000u;
    float amax = __uint_as_float(bits_max);
    if (has_nan) {
        const int base = static_cast<int>(__lane_id()) & ~1;
        amax = 0.0f;
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                const float w = fabsf(__shfl(x[k], base + t, 64));
                amax = amax > w ? amax : w;
            }
        }
    }
    const float d = amax / 127.0f;
    const float id = nan_if_inf(d != 0.0f ? 1.0f / d : 0.0f);
    if (!has_nan) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = trunc_i32(half_away_offset(x[4 * w + k] * id));
            pk[w] = pack_low_bytes(q[0], q[1], q[2], q[3]);
        }
    } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t q[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float t = half_away_offset(x[4 * w + k] * id);
                q[k] = __builtin_fabsf(t) < 0x1p31f ? low_byte_i8(t) : 0u;
            }
            pk[w] = pack4(q[0], q[1], q[2], q[3]);
        }
    }
    return f2h(d);
}

// XF: the activations' form. PB > 0: the weights in the packed layout
// (levo_hip_repack_q8_0): lane li of a row group loads blocks
// kb0 + li + LPR * i (i < PB, the same blocks in the same order as the
// block-layout path; PB = the span's blocks per lane, rounded up: every
// geometry gives a lane at most 4) straight into registers: the first 16
// quants, the last 16 and the F16 scale, each an aligned load; no LDS
// stage, no realignment. PB = 0: Q8_0 blocks.
// NV: accumulators per lane, 2 for the CFG pair (n_vec <= 2), else 8.
// CH: chunk loads per lane of the block layout's span (1 for packed weights).
template <int LPR, int WPR, int XF, int PB, int NV, int CH>
__global__ __launch_bounds__(kThreads) void mul_mat_q8_0_kernel(const mm_launch ml) {
    constexpr bool FUSED = XF == kXF32;
    constexpr bool PAIR = XF == kXF32Pair;
    constexpr bool PACKED = PB > 0;
    constexpr int kPB = PACKED ? PB : 1;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    // this workgroup's matrix, selected among arguments read at fixed
    // offsets (an index into the argument arrays would make the weight
    // addresses wait for a second, dependent argument load)
    mm_params p = ml.p;
    p.w = ml.w[0];
    p.y = ml.y[0];
    p.rows = ml.rows[0];
    p.y_pitch = ml.y_pitch[0];
    int first = 0;
#pragma unroll
    for (int i = 1; i < kMaxMats; ++i) {
        if (i < ml.n_mats && static_cast<int>(blockIdx.x) >= ml.first[i]) {
            p.w = ml.w[i];
            p.y = ml.y[i];
            p.rows = ml.rows[i];
            p.y_pitch = ml.y_pitch[i];
            first = ml.first[i];
        }
    }
    p.w_bytes = p.rows * p.nb * kQ8Bytes;
    const int64_t grp = static_cast<int64_t>(blockIdx.x) - first;
    const int nvb = p.n_vec * p.nb;
    uint32_t * xq = reinterpret_cast<uint32_t *>(smem);                   // [n_vec][nb][8]
    float * dx = reinterpret_cast<float *>(smem + nvb * 32);               // [n_vec][nb]
    float * part = dx + nvb;                                               // [kWaves][kMaxVectors]
    uint8_t * stages = smem + ((nvb * 36 + kWaves * kMaxVectors * 4 + 15) & ~15);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint8_t * stage = stages + wave * p.stage_bytes;

    // 1. the activation blocks' first chunks, then this wave's weight loads:
    //    loads complete in issue order, so the activations (a few KiB, from
    //    L2) are unpacked while the weights are still in flight; columns
    //    (kXColumns) already have the LDS form and are copied as they are
    const int64_t xbytes = static_cast<int64_t>(nvb) * (XF == kXColumns ? 36 : kQ8Bytes);
    const int nchunks = static_cast<int>((xbytes + 15) >> 4);
    // FUSED: thread t < nvb quantizes activation block t (column t / nb,
    // block t % nb); other threads read block 0 and drop it
    const int xt = static_cast<int>(threadIdx.x) < nvb ? static_cast<int>(threadIdx.x) : 0;
    constexpr int kXr = FUSED ? 8 : PAIR ? 4 : kXChunks;
    const int xp = min(static_cast<int>(threadIdx.x) >> 1, nvb - 1);
    u32x4 xr[kXr];  // unconditional (see load_span): chunks past the end re-read chunk 0
#pragma unroll
    for (int i = 0; i < kXr; ++i) {
        if constexpr (PAIR) {
            const float * src = ml.xf + (xp / p.nb) * ml.x_pitch + (xp % p.nb) * 32 + 16 * (threadIdx.x & 1);
            xr[i] = *reinterpret_cast<const u32x4 *>(src + 4 * i);
        } else if constexpr (FUSED) {
            const float * src = ml.xf + (xt / p.nb) * ml.x_pitch + (xt % p.nb) * 32;
            xr[i] = *reinterpret_cast<const u32x4 *>(src + 4 * i);
        } else {
            const int c = static_cast<int>(threadIdx.x) + kThreads * i;
            const bool whole = c < nchunks && 16 * static_cast<int64_t>(c) + 16 <= xbytes;
            xr[i] = *reinterpret_cast<const u32x4 *>(p.x + (whole ? 16 * static_cast<int64_t>(c) : 0));
        }
    }
    // the activation requests go out before any weight request: loads
    // complete in issue order, so a weight load scheduled among them would
    // make the staging wait for HBM
    __builtin_amdgcn_sched_barrier(0);
    int64_t row0;
    int nrows, kb0, kb1;
    const bool have = wave_span<LPR, WPR>(p, grp, wave, row0, nrows, kb0, kb1);
    const int g = lane / LPR;
    const int li = lane % LPR;
    u32x4 regs[CH];
    const int64_t sb0 = (row0 * p.nb + kb0) * kQ8Bytes;
    const int64_t sb1 = (row0 * p.nb + (WPR > 1 ? kb1 : static_cast<int64_t>(nrows) * p.nb)) * kQ8Bytes;
    u32x4 wlo[kPB], whi[kPB];
    uint16_t wd[kPB];
    if constexpr (PACKED) {
        // unconditional loads (see load_span): a block past the span re-reads
        // the span's last one, a row group past the last row reads the
        // wave's first row, an inactive wave reads block 0
        const int64_t row = !have ? 0 : row0 + (WPR > 1 || g >= nrows ? 0 : g);
        const int last = have ? kb1 - 1 : 0;
        const uint8_t * qrow = p.w + row * p.nb * 32;
        const uint16_t * drow = reinterpret_cast<const uint16_t *>(p.w + p.rows * p.nb * 32) + row * p.nb;
#pragma unroll
        for (int i = 0; i < kPB; ++i) {
            const int kb = !have ? 0 : std::min(kb0 + li + LPR * i, last);
            wlo[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + kb * 16));
            whi[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(qrow + (p.nb + kb) * 16));
            wd[i] = __builtin_nontemporal_load(drow + kb);
        }
    } else {
        load_span<CH>(p.w, p.w_bytes, sb0 & ~int64_t{15}, sb1, have, lane, regs);
    }

    // 2. activation blocks -> LDS (raw, through the stage area), then
    //    unpacked to aligned quant dwords and F32 scales; or, FUSED,
    //    quantized from F32 straight into that form; or columns copied to it
    if constexpr (XF == kXColumns) {
#pragma unroll
        for (int i = 0; i < kXChunks; ++i) {
            const int c = static_cast<int>(threadIdx.x) + kThreads * i;
            if (c >= nchunks) continue;
            if (16 * static_cast<int64_t>(c) + 16 <= xbytes) reinterpret_cast<u32x4 *>(smem)[c] = xr[i];
            else copy_tail_dwords(smem, p.x, xbytes, c);
        }
        for (int c = threadIdx.x + kThreads * kXChunks; c < nchunks; c += kThreads) {
            if (16 * static_cast<int64_t>(c) + 16 <= xbytes) {
                reinterpret_cast<u32x4 *>(smem)[c] = *reinterpret_cast<const u32x4 *>(p.x + 16 * static_cast<int64_t>(c));
            } else {
                copy_tail_dwords(smem, p.x, xbytes, c);
            }
        }
        lds_barrier();  // LDS only: the weight loads stay in flight
    } else if constexpr (PAIR) {
        uint32_t pk[4];
        const uint16_t d = quantize_q8_0_block_x2(xr, pk);
        if ((static_cast<int>(threadIdx.x) >> 1) < nvb) {
            reinterpret_cast<u32x4 *>(xq)[threadIdx.x] = u32x4{pk[0], pk[1], pk[2], pk[3]};
            if ((threadIdx.x & 1) == 0) dx[threadIdx.x >> 1] = h2f(d);
        }
        lds_barrier();  // LDS only: the weight loads stay in flight
    } else if constexpr (FUSED) {
        float xs[32];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            xs[4 * i] = __uint_as_float(xr[i].x);
            xs[4 * i + 1] = __uint_as_float(xr[i].y);
            xs[4 * i + 2] = __uint_as_float(xr[i].z);
            xs[4 * i + 3] = __uint_as_float(xr[i].w);
        }
        uint32_t q[8];
        const uint16_t d = quantize_q8_0_block(xs, q);
        if (static_cast<int>(threadIdx.x) < nvb) {
            dx[threadIdx.x] = h2f(d);
            u32x4 * dst = reinterpret_cast<u32x4 *>(xq + threadIdx.x * 8);
            dst[0] = u32x4{q[0], q[1], q[2], q[3]};
            dst[1] = u32x4{q[4], q[5], q[6], q[7]};
        }
        lds_barrier();  // LDS only: the weight loads stay in flight
    } else {
#pragma unroll
        for (int i = 0; i < kXChunks; ++i) {
            const int c = static_cast<int>(threadIdx.x) + kThreads * i;
            if (c >= nchunks) continue;
            reinterpret_cast<u32x4 *>(stages)[c] = 16 * static_cast<int64_t>(c) + 16 <= xbytes ? xr[i]
                                                                                             : load_x_chunk(p.x, xbytes, c);
        }
        for (int c = threadIdx.x + kThreads * kXChunks; c < nchunks; c += kThreads)
            reinterpret_cast<u32x4 *>(stages)[c] = load_x_chunk(p.x, xbytes, c);
        lds_barrier();  // LDS only: the weight loads stay in flight
        for (int t = threadIdx.x; t < nvb; t += kThreads) {
            uint32_t q[8];
            dx[t] = read_block(stages, t * kQ8Bytes, q);
            u32x4 * dst = reinterpret_cast<u32x4 *>(xq + t * 8);
            dst[0] = u32x4{q[0], q[1], q[2], q[3]};
            dst[1] = u32x4{q[4], q[5], q[6], q[7]};
        }
        lds_barrier();
    }

    // 3. the wave's blocks: lane li of row group g takes kb = kb0 + li + LPR * i
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0f;
    if constexpr (PACKED) {
        if (have && g < nrows) {
#pragma unroll
            for (int i = 0; i < kPB; ++i) {
                const int kb = kb0 + li + LPR * i;
                if (kb >= kb1) break;
                const uint32_t q[8] = {wlo[i].x, wlo[i].y, wlo[i].z, wlo[i].w, whi[i].x, whi[i].y, whi[i].z, whi[i].w};
                block_terms<NV>(q, h2f(wd[i]), xq, dx, p.nb, kb, p.n_vec, acc);
            }
        }
    } else {
        const int lead = static_cast<int>(sb0 & 15);
        store_span<CH>(stage, p.w, p.w_bytes, sb0 & ~int64_t{15}, sb1, have, lane, regs);
        wave_lds_fence();
        if (have && g < nrows) {
            const int row_base = WPR > 1 ? 0 : g * p.nb;  // LDS block index of (row g, kb0)
            for (int kb = kb0 + li; kb < kb1; kb += LPR) {
                uint32_t q[8];
                const float dw = read_block(stage, lead + (row_base + kb - kb0) * kQ8Bytes, q);
                block_terms<NV>(q, dw, xq, dx, p.nb, kb, p.n_vec, acc);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) {
        if (v >= p.n_vec) break;
        acc[v] = group_sum<LPR>(acc[v]);
    }
    if constexpr (WPR > 1) {
        // the row's parts meet in LDS, summed in wave order
        if (lane == 0) {
#pragma unroll
            for (int v = 0; v < NV; ++v) part[wave * kMaxVectors + v] = acc[v];
        }
        __syncthreads();
        if (wave % WPR == 0 && lane < p.n_vec && row0 < p.rows) {
            float s = part[wave * kMaxVectors + lane];
#pragma unroll
            for (int w = 1; w < WPR; ++w) s += part[(wave + w) * kMaxVectors + lane];
            p.y[lane * p.y_pitch + row0] = s;
        }
    } else if (have && g < nrows && li == 0) {
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            if (v >= p.n_vec) break;
            p.y[v * p.y_pitch + row0 + g] = acc[v];
        }
    }
}

template <int LPR, int WPR>
constexpr int rows_per_workgroup() {
    return WPR > 1 ? kWaves / WPR : kWaves * (64 / LPR);
}

// The instance for the activations' form (F32 values: two lanes per block up
// to 128 blocks; else columns for packed matrices, Q8_0 blocks otherwise)
// and the accumulator count.
template <int LPR, int WPR, int PB, int NV, int CH>
void launch_form(const mm_launch & ml, uint32_t blocks, size_t lds, hipStream_t st) {
    if (ml.xf != nullptr && ml.p.n_vec * ml.p.nb <= kThreads / 2)
        mul_mat_q8_0_kernel<LPR, WPR, kXF32Pair, PB, NV, CH><<<blocks, kThreads, lds, st>>>(ml);
    else if (ml.xf != nullptr) mul_mat_q8_0_kernel<LPR, WPR, kXF32, PB, NV, CH><<<blocks, kThreads, lds, st>>>(ml);
    else if constexpr (PB > 0) mul_mat_q8_0_kernel<LPR, WPR, kXColumns, PB, NV, CH><<<blocks, kThreads, lds, st>>>(ml);
    else mul_mat_q8_0_kernel<LPR, WPR, kXBlocks, PB, NV, CH><<<blocks, kThreads, lds, st>>>(ml);
}

template <int LPR, int WPR, int PB, int CH = 1>
int launch_pb(const mm_launch & ml, uint32_t blocks, size_t lds, hipStream_t st, const char * what) {
    if (ml.p.n_vec <= 2) launch_form<LPR, WPR, PB, 2, CH>(ml, blocks, lds, st);
    else launch_form<LPR, WPR, PB, kMaxVectors, CH>(ml, blocks, lds, st);
    return launch_status(what);
}

template <int LPR, int WPR>
int launch_mm(mm_launch ml, bool packed, hipStream_t st, const char * what) {
    constexpr int rows_per_block = rows_per_workgroup<LPR, WPR>();
    mm_params & p = ml.p;
    const int span_blocks = WPR > 1 ? (p.nb + WPR - 1) / WPR : (64 / LPR) * p.nb;
    p.stage_bytes = packed ? 0 : (span_blocks * kQ8Bytes + 32 + 15) & ~15;
    const int64_t nvb = static_cast<int64_t>(p.n_vec) * p.nb;
    // The raw activation blocks pass through the stage area before unpacking
    // (unpacking the last one reads 4 bytes past it), so it holds both; the
    // packed path's activations (columns, or F32) go to their place directly.
    const int64_t raw = packed ? 0 : (nvb * kQ8Bytes + 16 + 15) & ~int64_t{15};
    const int64_t stages = std::max<int64_t>(int64_t{kWaves} * p.stage_bytes, raw);
    const size_t lds = ((static_cast<size_t>(nvb) * 36 + kWaves * kMaxVectors * 4 + 15) & ~size_t{15}) +
                       static_cast<size_t>(stages);
    LEVO_REQUIRE(lds <= 64 * 1024, "%s: n_vec * K too large for the workgroup's LDS", what);
    int64_t groups = 0;
    for (int m = 0; m < ml.n_mats; ++m) {
        ml.first[m] = static_cast<int32_t>(groups);
        groups += ceil_div(ml.rows[m], rows_per_block);
    }
    for (int m = ml.n_mats; m <= kMaxMats; ++m) ml.first[m] = static_cast<int32_t>(groups);
    LEVO_REQUIRE(groups < (int64_t{1} << 31), "%s: too many rows", what);
    if (groups == 0) return LEVO_HIP_OK;
    const uint32_t blocks = static_cast<uint32_t>(groups);
    if (packed) {
        // blocks per lane: the span over LPR lanes, 1-4 at 16 lanes per row,
        // 3-4 for the longer rows (more than 64 blocks per 16 lanes)
        const int64_t per_lane = ceil_div(WPR > 1 ? (p.nb + WPR - 1) / WPR : p.nb, LPR);
        if constexpr (LPR == 16) {
            if (per_lane == 1) return launch_pb<LPR, WPR, 1>(ml, blocks, lds, st, what);
            if (per_lane == 2) return launch_pb<LPR, WPR, 2>(ml, blocks, lds, st, what);
        }
        if (per_lane == 3) return launch_pb<LPR, WPR, 3>(ml, blocks, lds, st, what);
        return launch_pb<LPR, WPR, 4>(ml, blocks, lds, st, what);
    }
    // Block layout: chunk loads per lane sized to the span where it is
    // smaller than the general instance's (every lane issues all of them):
    // 5 for half rows up to 294 blocks (ffn_down), 7 for four rows of up to
    // 52 blocks (K = 1536)
    const int64_t span_bytes = static_cast<int64_t>(span_blocks) * kQ8Bytes;
    if constexpr (WPR == 2) {
        if (span_bytes + 30 <= 5 * 64 * 16) return launch_pb<LPR, WPR, 0, 5>(ml, blocks, lds, st, what);
    }
    if constexpr (LPR == 16 && WPR == 1) {
        if (span_bytes + 30 <= 7 * 64 * 16) return launch_pb<LPR, WPR, 0, 7>(ml, blocks, lds, st, what);
    }
    return launch_pb<LPR, WPR, 0, kChunksPerLane>(ml, blocks, lds, st, what);
}

// The fewest lanes per row that hold the row's blocks in one wave's span.
// The geometry depends on K alone, so that a matrix gives the same bits alone
// or in a multi launch with any others (the lanes per row fix the summation
// order); 32 lanes per row would gain 0.2 us at 1536 x 1536 (4.0 -> 3.8 us)
// and lose at 8960 rows and more.
int launch_geometry(const mm_launch & ml, bool packed, hipStream_t st, const char * what) {
    const int nb = ml.p.nb;
    if (nb <= 64) return launch_mm<16, 1>(ml, packed, st, what);
    if (nb <= 128) return launch_mm<32, 1>(ml, packed, st, what);
    if (nb <= 256) return launch_mm<64, 1>(ml, packed, st, what);
    if (nb <= 512) return launch_mm<64, 2>(ml, packed, st, what);
    return launch_mm<64, 4>(ml, packed, st, what);
}

// levo_hip_quantize_q8_0_columns: thread t quantizes block t of the n_vec
// columns (column t / nb, block t % nb) with the block function of
// levo_hip_quantize_chunk; its quants go to byte 32 t, its scale, widened
// to F32, to the scale array after all quants.
__global__ __launch_bounds__(kThreads) void quantize_columns_kernel(const float * __restrict__ x, int64_t x_pitch,
                                                                    uint8_t * __restrict__ cols, int32_t nvb, int32_t nb) {
    const int t = static_cast<int>(blockIdx.x) * kThreads + static_cast<int>(threadIdx.x);
    if (t >= nvb) return;
    const u32x4 * src = reinterpret_cast<const u32x4 *>(x + (t / nb) * x_pitch + static_cast<int64_t>(t % nb) * 32);
    float xs[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const u32x4 v = src[i];
        xs[4 * i] = __uint_as_float(v.x);
        xs[4 * i + 1] = __uint_as_float(v.y);
        xs[4 * i + 2] = __uint_as_float(v.z);
        xs[4 * i + 3] = __uint_as_float(v.w);
    }
    uint32_t q[8];
    const uint16_t d = quantize_q8_0_block(xs, q);
    u32x4 * dst = reinterpret_cast<u32x4 *>(cols + static_cast<int64_t>(t) * 32);
    dst[0] = u32x4{q[0], q[1], q[2], q[3]};
    dst[1] = u32x4{q[4], q[5], q[6], q[7]};
    reinterpret_cast<float *>(cols + static_cast<int64_t>(nvb) * 32)[t] = h2f(d);
}

// levo_hip_repack_q8_0: thread t moves block t (17 aligned half-words at
// byte 34 t) to its row's two quant halves and the scale array.
__global__ __launch_bounds__(kThreads) void repack_q8_0_kernel(const uint8_t * __restrict__ blocks,
                                                               uint8_t * __restrict__ packed, int64_t rows, int32_t nb) {
    const int64_t b = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (b >= rows * nb) return;
    const uint16_t * src = reinterpret_cast<const uint16_t *>(blocks + b * kQ8Bytes);
    uint32_t h[17];
#pragma unroll
    for (int i = 0; i < 17; ++i) h[i] = src[i];
    const int64_t row = b / nb;
    const int64_t kb = b - row * nb;
    uint8_t * qrow = packed + row * nb * 32;
    *reinterpret_cast<u32x4 *>(qrow + kb * 16) =
        u32x4{h[1] | (h[2] << 16), h[3] | (h[4] << 16), h[5] | (h[6] << 16), h[7] | (h[8] << 16)};
    *reinterpret_cast<u32x4 *>(qrow + (nb + kb) * 16) =
        u32x4{h[9] | (h[10] << 16), h[11] | (h[12] << 16), h[13] | (h[14] << 16), h[15] | (h[16] << 16)};
    reinterpret_cast<uint16_t *>(packed + rows * nb * 32)[b] = static_cast<uint16_t>(h[0]);
}

// packed: the weights from levo_hip_repack_q8_0 and the activations as
// columns (levo_hip_quantize_q8_0_columns), else both as Q8_0 blocks.
int mul_mat_one(const void * weight, const void * x_blocks, float * y, int64_t y_pitch, int64_t rows, int64_t k,
                int64_t n_vec, bool packed, hipStream_t st, const char * what) {
    LEVO_REQUIRE(rows >= 0 && n_vec >= 0, "%s: negative size", what);
    if (rows == 0 || n_vec == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(k > 0 && k % 32 == 0, "%s: K must be a positive multiple of 32 (pad the rows)", what);
    LEVO_REQUIRE(k / 32 <= kMaxBlocksPerRow, "%s: K exceeds %d", what, kMaxBlocksPerRow * 32);
    LEVO_REQUIRE(n_vec <= kMaxVectors, "%s: at most %d activation columns", what, kMaxVectors);
    LEVO_REQUIRE(rows < (int64_t{1} << 31) / 4, "%s: too many rows", what);
    LEVO_REQUIRE(weight != nullptr && x_blocks != nullptr && y != nullptr, "%s: null tensor", what);
    LEVO_REQUIRE(aligned16(weight) && aligned16(x_blocks), "%s: block buffers must be 16-byte aligned", what);
    LEVO_REQUIRE(y_pitch >= rows, "%s: y pitch smaller than the row count", what);
    mm_launch ml{};
    ml.p.x = static_cast<const uint8_t *>(x_blocks);
    ml.p.nb = static_cast<int32_t>(k / 32);
    ml.p.n_vec = static_cast<int32_t>(n_vec);
    ml.n_mats = 1;
    ml.w[0] = static_cast<const uint8_t *>(weight);
    ml.y[0] = y;
    ml.rows[0] = rows;
    ml.y_pitch[0] = y_pitch;
    return launch_geometry(ml, packed, st, what);
}

int mul_mat_multi(const levo_hip_mat_q8_0 * mats, int32_t n_mats, const void * x_blocks, const float * x,
                  int64_t x_pitch, int64_t k, int64_t n_vec, bool packed, hipStream_t st, const char * what) {
    LEVO_REQUIRE(n_mats >= 1 && n_mats <= kMaxMats, "%s: 1 to %d matrices", what, kMaxMats);
    LEVO_REQUIRE(mats != nullptr, "%s: null matrix list", what);
    LEVO_REQUIRE(n_vec >= 0, "%s: negative size", what);
    LEVO_REQUIRE(k > 0 && k % 32 == 0, "%s: K must be a positive multiple of 32 (pad the rows)", what);
    LEVO_REQUIRE(k / 32 <= kMaxBlocksPerRow, "%s: K exceeds %d", what, kMaxBlocksPerRow * 32);
    LEVO_REQUIRE(n_vec <= kMaxVectors, "%s: at most %d activation columns", what, kMaxVectors);
    LEVO_REQUIRE((x_blocks == nullptr) != (x == nullptr), "%s: pass exactly one of x_blocks and x", what);
    if (x_blocks != nullptr) {
        LEVO_REQUIRE(aligned16(x_blocks), "%s: block buffers must be 16-byte aligned", what);
    } else {
        LEVO_REQUIRE(n_vec * (k / 32) <= kThreads,
                     "%s: F32 activations are quantized in the launch for n_vec * K / 32 <= %d blocks; "
                     "quantize larger ones with levo_hip_quantize_chunk", what, kThreads);
        LEVO_REQUIRE(aligned16(x) && x_pitch >= k && x_pitch % 4 == 0,
                     "%s: F32 activations need 16-byte aligned rows of at least K values", what);
    }
    mm_launch ml{};
    ml.p.x = static_cast<const uint8_t *>(x_blocks);
    ml.p.nb = static_cast<int32_t>(k / 32);
    ml.p.n_vec = static_cast<int32_t>(n_vec);
    ml.xf = x;
    ml.x_pitch = x_pitch;
    ml.n_mats = 0;
    for (int32_t i = 0; i < n_mats; ++i) {
        const levo_hip_mat_q8_0 & mt = mats[i];
        LEVO_REQUIRE(mt.rows >= 0, "%s: negative size", what);
        LEVO_REQUIRE(mt.rows < (int64_t{1} << 31) / 4, "%s: too many rows", what);
        if (mt.rows == 0) continue;
        LEVO_REQUIRE(mt.weight != nullptr && mt.y != nullptr, "%s: null tensor", what);
        LEVO_REQUIRE(aligned16(mt.weight), "%s: block buffers must be 16-byte aligned", what);
        LEVO_REQUIRE(mt.y_pitch >= mt.rows, "%s: y pitch smaller than the row count", what);
        ml.w[ml.n_mats] = static_cast<const uint8_t *>(mt.weight);
        ml.y[ml.n_mats] = mt.y;
        ml.rows[ml.n_mats] = mt.rows;
        ml.y_pitch[ml.n_mats] = mt.y_pitch;
        ++ml.n_mats;
    }
    if (ml.n_mats == 0 || n_vec == 0) return LEVO_HIP_OK;
    return launch_geometry(ml, packed, st, what);
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_mul_mat_q8_0(const void * weight, const void * x_blocks, float * y, int64_t y_pitch,
                                     int64_t rows, int64_t k, int64_t n_vec, levo_hip_stream_t stream) {
    return mul_mat_one(weight, x_blocks, y, y_pitch, rows, k, n_vec, false, as_hip(stream), "mul_mat_q8_0");
}

extern "C" int levo_hip_mul_mat_q8_0_multi(const levo_hip_mat_q8_0 * mats, int32_t n_mats, const void * x_blocks,
                                           const float * x, int64_t x_pitch, int64_t k, int64_t n_vec,
                                           levo_hip_stream_t stream) {
    return mul_mat_multi(mats, n_mats, x_blocks, x, x_pitch, k, n_vec, false, as_hip(stream), "mul_mat_q8_0_multi");
}

extern "C" int levo_hip_repack_q8_0(const void * blocks, void * packed, int64_t rows, int64_t k,
                                    levo_hip_stream_t stream) {
    const char * what = "repack_q8_0";
    LEVO_REQUIRE(rows >= 0, "%s: negative size", what);
    if (rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(k > 0 && k % 32 == 0, "%s: K must be a positive multiple of 32 (pad the rows)", what);
    LEVO_REQUIRE(k / 32 <= kMaxBlocksPerRow, "%s: K exceeds %d", what, kMaxBlocksPerRow * 32);
    LEVO_REQUIRE(rows * (k / 32) < (int64_t{1} << 31), "%s: too many blocks", what);
    LEVO_REQUIRE(blocks != nullptr && packed != nullptr, "%s: null tensor", what);
    LEVO_REQUIRE(aligned16(blocks) && aligned16(packed), "%s: buffers must be 16-byte aligned", what);
    const int64_t bytes = rows * (k / 32) * kQ8Bytes;
    const uint8_t * a = static_cast<const uint8_t *>(blocks);
    const uint8_t * b = static_cast<const uint8_t *>(packed);
    LEVO_REQUIRE(a + bytes <= b || b + bytes <= a, "%s: the packed matrix must not overlap the blocks", what);
    const int64_t n = rows * (k / 32);
    repack_q8_0_kernel<<<static_cast<uint32_t>(ceil_div(n, kThreads)), kThreads, 0, as_hip(stream)>>>(
        a, static_cast<uint8_t *>(packed), rows, static_cast<int32_t>(k / 32));
    return launch_status(what);
}

extern "C" int levo_hip_quantize_q8_0_columns(const float * x, int64_t x_pitch, void * columns, int64_t n_vec,
                                              int64_t k, levo_hip_stream_t stream) {
    const char * what = "quantize_q8_0_columns";
    LEVO_REQUIRE(n_vec >= 0, "%s: negative size", what);
    if (n_vec == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(k > 0 && k % 32 == 0, "%s: K must be a positive multiple of 32 (pad the rows)", what);
    LEVO_REQUIRE(k / 32 <= kMaxBlocksPerRow, "%s: K exceeds %d", what, kMaxBlocksPerRow * 32);
    LEVO_REQUIRE(n_vec <= kMaxVectors, "%s: at most %d activation columns", what, kMaxVectors);
    LEVO_REQUIRE(x != nullptr && columns != nullptr, "%s: null tensor", what);
    LEVO_REQUIRE(aligned16(x) && x_pitch >= k && x_pitch % 4 == 0,
                 "%s: F32 activations need 16-byte aligned rows of at least K values", what);
    LEVO_REQUIRE(aligned16(columns), "%s: the columns buffer must be 16-byte aligned", what);
    const int32_t nvb = static_cast<int32_t>(n_vec * (k / 32));
    quantize_columns_kernel<<<static_cast<uint32_t>(ceil_div(nvb, kThreads)), kThreads, 0, as_hip(stream)>>>(
        x, x_pitch, static_cast<uint8_t *>(columns), nvb, static_cast<int32_t>(k / 32));
    return launch_status(what);
}

extern "C" int levo_hip_mul_mat_q8_0_packed(const void * packed, const void * x_blocks, float * y, int64_t y_pitch,
                                            int64_t rows, int64_t k, int64_t n_vec, levo_hip_stream_t stream) {
    return mul_mat_one(packed, x_blocks, y, y_pitch, rows, k, n_vec, true, as_hip(stream), "mul_mat_q8_0_packed");
}

extern "C" int levo_hip_mul_mat_q8_0_packed_multi(const levo_hip_mat_q8_0 * mats, int32_t n_mats,
                                                  const void * x_blocks, const float * x, int64_t x_pitch, int64_t k,
                                                  int64_t n_vec, levo_hip_stream_t stream) {
    return mul_mat_multi(mats, n_mats, x_blocks, x, x_pitch, k, n_vec, true, as_hip(stream),
                         "mul_mat_q8_0_packed_multi");
}
