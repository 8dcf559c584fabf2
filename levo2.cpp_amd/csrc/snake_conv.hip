// Conv1d (stride 1) with SnakeBeta applied to its input and the bias and a
// residual add applied to its output, as one implicit GEMM on the F32 matrix
// cores. It is the Oobleck VAE decoder's residual unit written as two calls
// (src/levo-vae.cpp:91-100):
//   h = conv_1d_f32(snake(x, pre), W0, b0, pad 3d, dilation d)
//   y = x + conv_1d_f32(snake(h, post), W1, b1, 0, 1)
// and also its input / output convolutions (:219-221, :260-262). conv_1d_f32
// is ggml_im2col + ggml_mul_mat + the bias add (src/levo-audio-ops.cpp:56-87);
// here the im2col matrix is never formed and the activated input is never
// written to HBM:
//   y[co][t] = (sum_{ci,k} W[co][ci][k] * s(x)[ci][t + k * dil - pad]) + b[co]
//              (+ r[co][t])
// with s the SnakeBeta of snake_math.hpp (or the identity) and zero outside
// [0, T_in), the same arithmetic as the standalone SnakeBeta kernel. The sum
// is accumulated by the F32 MFMA in another order than ggml's dot, so y
// agrees with the reference to F32 rounding.
//
// Workgroup tile: 128 output channels x 128 samples, 4 waves of 64 x 64, each
// 4 x 4 tiles of v_mfma_f32_16x16x4f32. K runs over chunks of CI input
// channels x KW taps: the weight chunk is staged in LDS k-major with the rows
// permuted so that a lane's four A fragments are one 16-byte read; the input
// chunk (CI rows of 128 + (KW - 1) * dil samples, the halo included) is staged
// with SnakeBeta applied once per element, from per-channel parameters the
// workgroup computes up front.
#include "common.hpp"
#include "snake_math.hpp"

#include <algorithm>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kMT = 128;  // output channels per workgroup
constexpr int kNT = 128;  // output samples per workgroup
constexpr int kMaxSnakeChannels = 2048;

typedef float f32x4v __attribute__((ext_vector_type(4)));

template <int KW>
struct conv_chunk {
    static constexpr int CI = KW == 1 ? 32 : KW == 2 ? 16 : 8;  // input channels per K chunk
    static constexpr int KC = CI * KW;                          // K values per chunk (a multiple of 4)
};

struct conv_params {
    const float * x;
    int64_t x_pitch;
    int64_t t_in;
    const void * alpha_log;
    const void * beta_log;
    int32_t param_f16;
    int32_t snake;
    const float * w;          // [c_out][c_in][KW]
    const float * bias;       // [c_out] or null
    const float * residual;   // [c_out][r_pitch] or null
    int64_t r_pitch;
    float * y;
    int64_t y_pitch;
    int64_t t_out;
    int32_t c_in, c_out;
    int32_t pad, dil;
    int32_t b_width;          // staged samples per input row: kNT + (KW - 1) * dil, rounded up to 4
    int32_t w_vec;            // weight rows 16-byte aligned with KW * c_in % 4 == 0
    int32_t y_vec;            // y (and residual) rows 16-byte aligned: float4 epilogue
    // Output placement: column q of phase z = blockIdx.z goes to sample
    // q * o_stride + o_base + z of y (kept when in [0, y_len)); the phase's
    // weights start w_phase floats after p.w. A plain convolution has one
    // phase, o_stride 1, o_base 0, y_len t_out.
    int32_t o_stride;
    int32_t o_base;
    int64_t y_len;
    int64_t w_phase;
    int32_t scatter;          // transposed convolution: the strided epilogue
    // SnakeBeta parameters in LDS: 0 = all c_in channels, computed up front;
    // 1 = two slots of CI channels, each chunk's computed one chunk ahead (for
    // wide inputs, where the full table would cost a workgroup per CU)
    int32_t param_ring;
    int32_t b_magic;          // ceil(2^24 / b_width): row of a flat B index by multiply
    // Workgroup order: 0 = grid (time tiles, channel tiles, phases); 1 = a 1-D
    // grid that gives each XCD a run of consecutive tiles, every phase of a
    // tile back to back
    int32_t xcd_order;
    int32_t tiles_x, tiles, phases;
    // Split K: the grid's phase axis z covers n_phase stride phases times
    // `splits` splits, phase z % n_phase and split z / n_phase. Split j sums
    // the input channels of chunks [j n / splits, (j + 1) n / splits) of the
    // n chunks and writes that partial sum (columns q of the phase, without
    // bias or residual) to part + z * part_slice, rows part_pitch floats
    // apart, 16-byte aligned; a combine kernel then adds the partials in
    // split order and applies the epilogue.
    int32_t n_phase;
    int32_t splits;
    // SnakeBeta applied to the output after the bias and residual (null: none;
    // same parameter type as alpha_log): the decoder's residual units store
    // snake_post(conv_0(...)), the input of their k = 1 conv, once per sample.
    const void * post_alpha_log;
    const void * post_beta_log;
    float * part;
    int64_t part_slice;
    int64_t part_pitch;
};

// Input channels [begin, end) of split z (all of them without a split).
template <int CI>
__device__ __forceinline__ void split_range(const conv_params & p, int z, int & begin, int & end) {
    if (p.splits <= 1) {
        begin = 0;
        end = p.c_in;
        return;
    }
    const int n = (p.c_in + CI - 1) / CI;
    begin = CI * (z * n / p.splits);
    end = min(p.c_in, CI * ((z + 1) * n / p.splits));
}

// Where split z's partial sum goes: the epilogue's plain path into the
// partial slice, with no bias and no residual.
__device__ __forceinline__ conv_params split_target(const conv_params & p, int z) {
    conv_params e = p;
    e.y = p.part + static_cast<int64_t>(z) * p.part_slice;
    e.y_pitch = p.part_pitch;
    e.bias = nullptr;
    e.residual = nullptr;
    e.post_alpha_log = nullptr;
    e.y_vec = 1;
    e.scatter = 0;
    return e;
}

// The time tile x, channel tile y and phase z of this workgroup. With
// xcd_order the grid is 1-D: the hardware deals workgroups to the 8 XCDs
// round-robin by linear id, and XCD j takes the j-th run of ceil(tiles / 8)
// consecutive tiles (tile = y * tiles_x + x, so a run is one channel tile's
// time tiles, or a part of them), each tile's phases back to back.
// - Every phase of a tile runs on one XCD, right after the others. The
//   phases of a transposed convolution write interleaved samples of the same
//   output lines, which then meet in that XCD's L2 instead of going back to
//   memory as partial lines; their shared input tile is read from there too.
// - A channel tile's weights (every phase's) are read by the XCDs its run
//   covers, one or two, and by the others not at all, where the deal of
//   consecutive tiles to the 8 XCDs had every XCD read all of them; and the
//   k = 7 halo of a time tile is mostly read by the XCD that read its
//   neighbours' inputs.
// Workgroups past the last tile (the short last run) are not live.
struct tile_id {
    int x, y, z;
    bool live;
};

__device__ __forceinline__ tile_id conv_tile(const conv_params & p) {
    if (!p.xcd_order) return {static_cast<int>(blockIdx.x), static_cast<int>(blockIdx.y), static_cast<int>(blockIdx.z), true};
    const int lin = static_cast<int>(blockIdx.x);
    const int k = lin >> 3;              // this workgroup's place in its XCD's run
    const int run = (p.tiles + 7) >> 3;  // tiles per XCD
    const int tile = (lin & 7) * run + k / p.phases;
    return {tile % p.tiles_x, tile / p.tiles_x, k % p.phases, tile < p.tiles};
}

// The k = 1 half of a residual unit (src/levo-vae.cpp:96-100) fused into the
// k = 7 launch, for c = kMT channels: one workgroup holds every channel of
// its time tile.
struct fuse_params {
    const float * w1;          // [c][c] k = 1 weights, 16-byte aligned
    const float * bias1;       // [c] or null
    const void * alpha1_log;   // post SnakeBeta [c] (type of conv_params::param_f16)
    const void * beta1_log;
    float * y;                 // [c][y_pitch]: the unit's output, not its input
    int64_t y_pitch;
    int32_t y_vec;             // y and the input rows 16-byte aligned
};

// LDS float index of weight (kk, r) in the A chunk: rows r = 64 h + 16 i + m
// are stored as [kk][h][m][i] so lane m of a wave on row half h reads
// its four fragments i = 0..3 with one ds_read_b128. Rows of kk are kAStride
// floats apart, which puts the four lane groups (four kk) of one read on
// different banks.
constexpr int kAStride = kMT + 4;

__device__ __forceinline__ int a_index(int kk, int r) {
    const int h = r >> 6;
    const int i = (r >> 4) & 3;
    const int m = r & 15;
    return kk * kAStride + h * 64 + m * 4 + i;
}

// Register slots of one K chunk, loaded while the previous chunk's MFMAs run.
// A: NA float4s per thread, slot u = element e = tid + 256 u of the
// [q][r] = [KC / 4][kMT] chunk (row r = e % kMT, weights 4q .. 4q + 3).
// B: NB input samples per thread: for KW = 1 (128-sample rows) slot s is row
// 2 s + tid / 128, sample tid % 128; otherwise row s % CI, sample
// tid + 256 (s / CI) (b_width <= 512). Threads past a row's end idle; the
// waves that stage less reach their MFMAs first, which measured faster than
// spreading the samples evenly.
template <int KW>
struct conv_slots {
    static constexpr int CI = conv_chunk<KW>::CI;
    static constexpr int KC = conv_chunk<KW>::KC;
    static constexpr int NA = KC / 4 * kMT / kThreads;
    static constexpr int NB = KW == 1 ? CI / 2 : KW == 2 ? CI : 2 * CI;
};

template <int KW>
__device__ __forceinline__ void b_slot(int s, int tid, int & c, int & j) {
    c = KW == 1 ? 2 * s + (tid >> 7) : s % conv_chunk<KW>::CI;
    j = KW == 1 ? (tid & 127) : tid + kThreads * (s / conv_chunk<KW>::CI);
}

// The weight part of a K chunk: NA float4s per thread (see conv_slots).
template <int KW>
__device__ __forceinline__ void load_chunk_a(const conv_params & p, int ci0, int co0, int tid,
                                             f32x4v (&ra)[conv_slots<KW>::NA]) {
    constexpr int CI = conv_slots<KW>::CI;
    const int64_t w_row = static_cast<int64_t>(p.c_in) * KW;
    const bool a_inside = p.w_vec && co0 + kMT <= p.c_out && ci0 + CI <= p.c_in;
#pragma unroll
    for (int u = 0; u < conv_slots<KW>::NA; ++u) {
        const int e = tid + kThreads * u;
        const int r = e % kMT;
        const int kk = 4 * (e / kMT);
        const int co = co0 + r;
        const float * src = p.w + co * w_row + static_cast<int64_t>(ci0) * KW + kk;
        f32x4v v = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
        if (a_inside) {
            v = *reinterpret_cast<const f32x4v *>(src);
        } else if (co < p.c_out) {
            if (p.w_vec && ci0 + (kk + 3) / KW < p.c_in) {
                v = *reinterpret_cast<const f32x4v *>(src);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (ci0 + (kk + q) / KW < p.c_in) v[q] = src[q];
                }
            }
        }
        ra[u] = v;
    }
}

template <int KW>
__device__ __forceinline__ void load_chunk(const conv_params & p, int ci0, int co0, int64_t t0, int tid,
                                           f32x4v (&ra)[conv_slots<KW>::NA], float (&rb)[conv_slots<KW>::NB]) {
    constexpr int CI = conv_slots<KW>::CI;
    load_chunk_a<KW>(p, ci0, co0, tid, ra);
    const int64_t tb = t0 - p.pad;
    const bool b_inside = tb >= 0 && tb + p.b_width <= p.t_in && ci0 + CI <= p.c_in;
    const float * xb = p.x + static_cast<int64_t>(ci0) * p.x_pitch + tb;
#pragma unroll
    for (int s = 0; s < conv_slots<KW>::NB; ++s) {
        int c, j;
        b_slot<KW>(s, tid, c, j);
        float v = 0.0f;
        if (j < p.b_width) {
            if (b_inside) {
                v = xb[c * p.x_pitch + j];
            } else if (ci0 + c < p.c_in && tb + j >= 0 && tb + j < p.t_in) {
                v = xb[c * p.x_pitch + j];
            }
        }
        rb[s] = v;
    }
}

// Weight slot u of a thread into the A chunk's permuted layout.
template <int KW>
__device__ __forceinline__ void store_a_slot(float * As, int tid, int u, const f32x4v & v) {
    const int e = tid + kThreads * u;
    const int r = e % kMT;
    const int kk = 4 * (e / kMT);
#pragma unroll
    for (int q = 0; q < 4; ++q) As[a_index(kk + q, r)] = v[q];
}

// spc: the SnakeBeta parameters of this chunk's channels ci0 .. ci0 + CI - 1.
template <int KW>
__device__ __forceinline__ void store_chunk(const conv_params & p, int ci0, int tid, float * As, float * Bs,
                                            const snake_param * spc, const f32x4v (&ra)[conv_slots<KW>::NA],
                                            const float (&rb)[conv_slots<KW>::NB]) {
#pragma unroll
    for (int u = 0; u < conv_slots<KW>::NA; ++u) {
        const int e = tid + kThreads * u;
        const int r = e % kMT;
        const int kk = 4 * (e / kMT);
#pragma unroll
        for (int q = 0; q < 4; ++q) As[a_index(kk + q, r)] = ra[u][q];
    }
#pragma unroll
    for (int s = 0; s < conv_slots<KW>::NB; ++s) {
        int c, j;
        b_slot<KW>(s, tid, c, j);
        if (j < p.b_width) {
            float v = rb[s];
            // zero padding stays zero: s(0) = 0 + sin^2(0) / beta = 0 exactly
            if (p.snake && ci0 + c < p.c_in) v = snake(v, spc[c]);
            Bs[c * p.b_width + j] = v;
        }
    }
}

// LDS floats of one A buffer.
template <int KW>
__host__ __device__ constexpr int a_floats() {
    return conv_chunk<KW>::KC * kAStride;
}

constexpr int kOutStride = kNT + 4;  // floats per row of the staged output tile

// A fragments (rows 16 i + m of the wave's row half, i = 0..3) and B
// fragments (columns 16 j + m of its column half) of K step ks for lane
// group g: K index kk = 4 ks + g is input channel kk / KW, tap kk % KW.
template <int KW>
__device__ __forceinline__ void read_operands(const float * As, const float * Bs, const conv_params & p, int ks,
                                              int g, int h, int vh, int m, f32x4v & a, float (&b)[4]) {
    const int kk = 4 * ks + g;
    const int c = kk / KW;
    const int k = kk - c * KW;
    a = *reinterpret_cast<const f32x4v *>(As + kk * kAStride + h * 64 + m * 4);
    const float * brow = Bs + c * p.b_width + vh * 64 + m + k * p.dil;
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = brow[16 * j];
}

// Raw alpha_log / beta_log of channel c (zero past c_in).
__device__ __forceinline__ void load_snake_logs(const conv_params & p, int c, float & al, float & bl) {
    al = 0.0f;
    bl = 0.0f;
    if (c < p.c_in) {
        al = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.alpha_log)[c]) : static_cast<const float *>(p.alpha_log)[c];
        bl = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.beta_log)[c]) : static_cast<const float *>(p.beta_log)[c];
    }
}

// The post-output SnakeBeta parameters of output channel co.
__device__ __forceinline__ snake_param post_param(const conv_params & p, int co) {
    const float al = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.post_alpha_log)[co])
                                 : static_cast<const float *>(p.post_alpha_log)[co];
    const float bl = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.post_beta_log)[co])
                                 : static_cast<const float *>(p.post_beta_log)[co];
    return make_snake_param(al, bl);
}

// The output tile goes through LDS (the A / B buffers, free after the
// kernel's last barrier) so that bias, residual and y move as whole rows.
// D[row][col] of a 16 x 16 tile is in lane col + 16 * (row / 4), item row % 4.
template <bool SCATTER>
__device__ __forceinline__ void conv_epilogue(const conv_params & p, float * lds, const f32x4v (&acc)[4][4], int tid,
                                              int h, int vh, int g, int m, int64_t t0, int co0, int phase) {
    float * out = lds;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int u = 0; u < 4; ++u)
                out[(h * 64 + 16 * i + 4 * g + u) * kOutStride + vh * 64 + 16 * j + m] = acc[i][j][u];
    __syncthreads();
    if (SCATTER && p.scatter) {
        // transposed convolution: phase z's columns land every o_stride samples
        const int64_t base = p.o_base + static_cast<int64_t>(phase);
        for (int e = tid; e < kMT * kNT; e += kThreads) {
            const int r = e / kNT;
            const int c = e % kNT;
            const int co = co0 + r;
            if (co >= p.c_out) break;  // rows only grow with e
            const int64_t q = t0 + c;
            const int64_t t = q * p.o_stride + base;
            if (q >= p.t_out || t < 0 || t >= p.y_len) continue;
            float v = out[r * kOutStride + c];
            if (p.bias) v = v + p.bias[co];
            p.y[co * p.y_pitch + t] = v;
        }
        return;
    }
    const bool vec = p.y_vec && t0 + kNT <= p.t_out;
    constexpr int kOutIters = kMT * (kNT / 4) / kThreads;  // float4s of the tile per thread
    if (vec && co0 + kMT <= p.c_out) {
        // Whole tile inside y: the thread's residual float4s are loaded
        // before any store (y may be the residual, so the loads cannot move
        // past the stores on their own), then each row is finished.
        f32x4v res[kOutIters];
        if (p.residual) {
#pragma unroll
            for (int it = 0; it < kOutIters; ++it) {
                const int e = tid + kThreads * it;
                const int r = e / (kNT / 4);
                const int c4 = 4 * (e % (kNT / 4));
                res[it] = *reinterpret_cast<const f32x4v *>(p.residual + (co0 + r) * p.r_pitch + t0 + c4);
            }
        }
#pragma unroll
        for (int it = 0; it < kOutIters; ++it) {
            const int e = tid + kThreads * it;
            const int r = e / (kNT / 4);
            const int c4 = 4 * (e % (kNT / 4));
            const int co = co0 + r;
            f32x4v v = *reinterpret_cast<const f32x4v *>(out + r * kOutStride + c4);
            if (p.bias) v = v + p.bias[co];
            if (p.residual) v = res[it] + v;
            if (p.post_alpha_log) {
                const snake_param q = post_param(p, co);
#pragma unroll
                for (int u = 0; u < 4; ++u) v[u] = snake(v[u], q);
            }
            *reinterpret_cast<f32x4v *>(p.y + co * p.y_pitch + t0 + c4) = v;
        }
        return;
    }
    for (int e = tid; e < kMT * (kNT / 4); e += kThreads) {
        const int r = e / (kNT / 4);
        const int c4 = 4 * (e % (kNT / 4));
        const int co = co0 + r;
        if (co >= p.c_out) break;  // rows only grow with e
        const float bv = p.bias ? p.bias[co] : 0.0f;
        const f32x4v o = *reinterpret_cast<const f32x4v *>(out + r * kOutStride + c4);
        const int64_t t = t0 + c4;
        snake_param sq{};
        if (p.post_alpha_log) sq = post_param(p, co);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (t + q >= p.t_out) break;
            float v = o[q];
            if (p.bias) v = v + bv;
            if (p.residual) v = p.residual[co * p.r_pitch + t + q] + v;
            if (p.post_alpha_log) v = snake(v, sq);
            p.y[co * p.y_pitch + t + q] = v;
        }
    }
}

template <int KW, bool RING>
__global__ __launch_bounds__(kThreads) void snake_conv1d_kernel(const conv_params p0) {
    const tile_id tl = conv_tile(p0);
    if (!tl.live) return;
    conv_params p = p0;
    const int n_phase = p.n_phase > 0 ? p.n_phase : 1;
    const int phase = tl.z % n_phase;
    const int split = tl.z / n_phase;
    p.w += static_cast<int64_t>(phase) * p.w_phase;  // this phase's weights
    constexpr int CI = conv_chunk<KW>::CI;
    constexpr int KC = conv_chunk<KW>::KC;
    extern __shared__ __attribute__((aligned(16))) float lds[];
    // two buffers of [A: KC x kAStride][B: CI x b_width], then the SnakeBeta
    // parameters: [c_in], or with param_ring [2][CI] (chunk i's in slot i % 2,
    // computed one chunk ahead of its staging); the output tile reuses the
    // buffers at the end
    const int buf_floats = a_floats<KW>() + CI * p.b_width;
    snake_param * sp = reinterpret_cast<snake_param *>(lds + 2 * buf_floats);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = wave >> 1;      // row half of the tile
    const int vh = wave & 1;      // column half
    const int m = lane & 15;
    const int g = lane >> 4;
    const int64_t t0 = static_cast<int64_t>(tl.x) * kNT;
    const int co0 = tl.y * kMT;

    // input channels of this workgroup (a split's share, or all); the
    // parameter table is indexed from ci_begin
    int ci_begin, ci_end;
    split_range<CI>(p, split, ci_begin, ci_end);

    f32x4v ra[conv_slots<KW>::NA];
    float rb[conv_slots<KW>::NB];
    load_chunk<KW>(p, ci_begin, co0, t0, tid, ra, rb);

    if (p.snake) {
        const int n = RING ? 2 * CI : ci_end - ci_begin;  // ring: the first two chunks
        for (int c = tid; c < n; c += kThreads) {
            float al, bl;
            load_snake_logs(p, ci_begin + c, al, bl);
            sp[c] = make_snake_param(al, bl);
        }
        __syncthreads();
    }
    store_chunk<KW>(p, ci_begin, tid, lds, lds + a_floats<KW>(), sp, ra, rb);
    __syncthreads();

    f32x4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};

    int buf = 0;
    for (int ci0 = ci_begin; ci0 < ci_end; ci0 += CI) {
        const bool more = ci0 + CI < ci_end;
        if (more) load_chunk<KW>(p, ci0 + CI, co0, t0, tid, ra, rb);  // in flight during the MFMAs
        // parameters of the chunk after next, computed in this chunk's store phase
        const bool params = RING && p.snake && ci0 + 2 * CI < ci_end && tid < CI;
        float al = 0.0f, bl = 0.0f;
        if (params) load_snake_logs(p, ci0 + 2 * CI + tid, al, bl);
        const float * As = lds + buf * buf_floats;
        const float * Bs = As + a_floats<KW>();
        // Operands of step ks + 1 are read while step ks's 16 MFMAs issue.
        f32x4v a;
        float b[4];
        read_operands<KW>(As, Bs, p, 0, g, h, vh, m, a, b);
#pragma unroll 2
        for (int ks = 0; ks < KC / 4; ++ks) {
            f32x4v an = a;
            float bn[4] = {b[0], b[1], b[2], b[3]};
            if (ks + 1 < KC / 4) read_operands<KW>(As, Bs, p, ks + 1, g, h, vh, m, an, bn);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
            a = an;
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bn[j];
        }
        if (more) {
            // the other buffer was last read before the previous barrier
            float * An = lds + (buf ^ 1) * buf_floats;
            store_chunk<KW>(p, ci0 + CI, tid, An, An + a_floats<KW>(),
                            sp + (RING ? (buf ^ 1) * CI : ci0 + CI - ci_begin), ra, rb);
        }
        // slot buf held this chunk's parameters, last read before the previous barrier
        if (RING && params) sp[buf * CI + tid] = make_snake_param(al, bl);
        __syncthreads();
        buf ^= 1;
    }

    conv_epilogue<true>(p.splits > 1 ? split_target(p, tl.z) : p, lds, acc, tid, h, vh, g, m, t0, co0, phase);
}

// ---- narrow output (c_out <= 4): the decoder's 128 -> 2 output conv -------
//
// A 128-row matrix-core tile would compute 2 useful rows, so narrow outputs
// take a VALU kernel instead: a workgroup owns kNarrowT output samples (thread
// tid the samples tid + 256 j, j < 4) and walks the input channels in chunks
// of kNarrowCI. A chunk's raw input rows (halo included) and weights are
// loaded into registers while the previous chunk is summed, then SnakeBeta is
// applied once per element on the way into LDS; the weights sit in LDS
// (zero past c_out) and are read at wave-uniform addresses. Every output
// channel is summed with FMAs over (ci, k) in ascending order.
constexpr int kNarrowT = 1024;
constexpr int kNarrowCI = 8;
constexpr int kNarrowJ = kNarrowT / kThreads;
constexpr int kNarrowMaxSpan = 512;                                   // (kernel - 1) * dilation
constexpr int kNarrowRowLoads = (kNarrowT + kNarrowMaxSpan + kThreads - 1) / kThreads;  // per row and thread

template <int KW, int NCO>
struct narrow_regs {
    float x[kNarrowCI][kNarrowRowLoads];
    float w;  // weight tid of the chunk's [NCO][kNarrowCI][KW] (tid < NCO * kNarrowCI * KW)
};

template <int KW, int NCO>
__device__ __forceinline__ void narrow_load(const conv_params & p, int ci0, int64_t tb, bool inside, int tid,
                                            narrow_regs<KW, NCO> & r) {
#pragma unroll
    for (int c = 0; c < kNarrowCI; ++c) {
        const bool row = ci0 + c < p.c_in;
        const float * xr = p.x + static_cast<int64_t>(ci0 + c) * p.x_pitch + tb;
#pragma unroll
        for (int i = 0; i < kNarrowRowLoads; ++i) {
            const int j = tid + kThreads * i;
            float v = 0.0f;
            if (row && j < p.b_width && (inside || (tb + j >= 0 && tb + j < p.t_in))) v = xr[j];
            r.x[c][i] = v;
        }
    }
    r.w = 0.0f;
    if (tid < NCO * kNarrowCI * KW) {
        const int co = tid / (kNarrowCI * KW);
        const int rem = tid - co * (kNarrowCI * KW);  // c * KW + k
        const int c = rem / KW;
        if (co < p.c_out && ci0 + c < p.c_in) r.w = p.w[(static_cast<int64_t>(co) * p.c_in + ci0) * KW + rem];
    }
}

template <int KW, int NCO>
__global__ __launch_bounds__(kThreads) void snake_conv_narrow_kernel(const conv_params p) {
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int width = p.b_width;                                     // kNarrowT + (KW - 1) * dil, rounded to 4
    float * xs = lds;                                                // [kNarrowCI][width]
    float * ws = xs + kNarrowCI * width;                             // [NCO][kNarrowCI][KW]
    snake_param * sp = reinterpret_cast<snake_param *>(ws + NCO * kNarrowCI * KW);  // [c_in] when p.snake
    const int tid = threadIdx.x;
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kNarrowT;
    const int64_t tb = t0 - p.pad;
    const bool inside = tb >= 0 && tb + width <= p.t_in;
    narrow_regs<KW, NCO> r;
    narrow_load<KW, NCO>(p, 0, tb, inside, tid, r);
    if (p.snake) {
        for (int c = tid; c < p.c_in; c += kThreads) {
            const float al = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.alpha_log)[c])
                                         : static_cast<const float *>(p.alpha_log)[c];
            const float bl = p.param_f16 ? h2f(static_cast<const uint16_t *>(p.beta_log)[c])
                                         : static_cast<const float *>(p.beta_log)[c];
            sp[c] = make_snake_param(al, bl);
        }
    }
    float acc[NCO][kNarrowJ];
#pragma unroll
    for (int co = 0; co < NCO; ++co)
#pragma unroll
        for (int j = 0; j < kNarrowJ; ++j) acc[co][j] = 0.0f;
    for (int ci0 = 0; ci0 < p.c_in; ci0 += kNarrowCI) {
        __syncthreads();  // the previous chunk's reads are done (and sp is ready)
#pragma unroll
        for (int c = 0; c < kNarrowCI; ++c) {
#pragma unroll
            for (int i = 0; i < kNarrowRowLoads; ++i) {
                const int j = tid + kThreads * i;
                if (j < width) {
                    float v = r.x[c][i];
                    // zero padding stays zero: s(0) = 0 + sin^2(0) / beta = 0 exactly
                    if (p.snake && ci0 + c < p.c_in) v = snake(v, sp[ci0 + c]);
                    xs[c * width + j] = v;
                }
            }
        }
        if (tid < NCO * kNarrowCI * KW) ws[tid] = r.w;
        __syncthreads();
        if (ci0 + kNarrowCI < p.c_in) narrow_load<KW, NCO>(p, ci0 + kNarrowCI, tb, inside, tid, r);  // in flight
        const int nc = min(kNarrowCI, p.c_in - ci0);
        for (int c = 0; c < nc; ++c) {
            const float * row = xs + c * width + tid;
#pragma unroll
            for (int k = 0; k < KW; ++k) {
                float xv[kNarrowJ];
#pragma unroll
                for (int j = 0; j < kNarrowJ; ++j) xv[j] = row[kThreads * j + k * p.dil];
#pragma unroll
                for (int co = 0; co < NCO; ++co) {
                    const float w = ws[(co * kNarrowCI + c) * KW + k];
#pragma unroll
                    for (int j = 0; j < kNarrowJ; ++j) acc[co][j] = __builtin_fmaf(w, xv[j], acc[co][j]);
                }
            }
        }
    }
#pragma unroll
    for (int co = 0; co < NCO; ++co) {
        if (co >= p.c_out) break;
        const float bv = p.bias ? p.bias[co] : 0.0f;
#pragma unroll
        for (int j = 0; j < kNarrowJ; ++j) {
            const int64_t t = t0 + tid + kThreads * j;
            if (t >= p.t_out) break;
            float v = acc[co][j];
            if (p.bias) v = v + bv;
            if (p.residual) v = p.residual[co * p.r_pitch + t] + v;
            p.y[co * p.y_pitch + t] = v;
        }
    }
}

template <int KW>
int launch_narrow(conv_params p, hipStream_t st, const char * what) {
    p.b_width = (kNarrowT + (KW - 1) * p.dil + 3) & ~3;
    const int nco = p.c_out <= 2 ? 2 : 4;
    const size_t lds = (static_cast<size_t>(kNarrowCI) * p.b_width + nco * kNarrowCI * KW) * sizeof(float) +
                       (p.snake ? static_cast<size_t>(p.c_in) * sizeof(snake_param) : 0);
    LEVO_REQUIRE(p.b_width <= kThreads * kNarrowRowLoads, "snake_conv1d: dilation too large");
    LEVO_REQUIRE(lds <= 64 * 1024, "snake_conv1d: dilation or channel count too large for LDS");
    const dim3 grid(static_cast<uint32_t>(ceil_div(p.t_out, kNarrowT)));
    if (nco == 2) {
        snake_conv_narrow_kernel<KW, 2><<<grid, kThreads, lds, st>>>(p);
    } else {
        snake_conv_narrow_kernel<KW, 4><<<grid, kThreads, lds, st>>>(p);
    }
    return launch_status(what);
}

// ---- the next chunk's staging interleaved into the MFMAs (k = 2, 7) -------
//
// The same tile, chunks and arithmetic as snake_conv1d_kernel<KW, false>, but
// the staging of chunk n + 1 is spread over the second half of chunk n's MFMA
// K steps instead of following them: per K step a share of the weight slots
// and of the input elements, with scheduling barriers that issue each of the
// step's 16 MFMAs between VALU instructions, so a single wave keeps the matrix
// pipe busy while it stages. The input elements are dealt evenly over the 256
// threads by the flat index e = tid + 256 s of the chunk's [CI][b_width]
// rows, which is also the element's LDS offset (the B region is padded to
// 256 * NB floats, so every store is unconditional); at k = 2, e / b_width is
// a multiply by b_magic = ceil(2^24 / b_width), exact for e < 4096 and
// b_width in [128, 512]. The SnakeBeta in the interleaved part is the
// reduced-argument form only; a thread with an argument beyond its range (or
// NaN / inf) rewrites its elements with the full form before the barrier.
// Outputs are bit-identical to snake_conv1d_kernel<KW, false>. The parameter
// table follows the two buffers and may overlap the output tile of the
// epilogue, which starts after the last barrier.
template <int KW>
struct il_shape {
    static constexpr int CI = conv_chunk<KW>::CI;
    static constexpr int KS = conv_chunk<KW>::KC / 4;  // K steps per chunk
    static constexpr int P = KS / 2;                    // steps that stage
    static constexpr int NA = conv_slots<KW>::NA;
    static constexpr int APP = (NA + P - 1) / P;        // weight slots per staging step
    // B slots per thread: the largest chunk ([CI][b_width] over 256 threads)
    static constexpr int kMaxNB = KW == 2 ? 9 : 6;
    // per MFMA of a staging step: VALU instructions, and an LDS store every
    // kDsEvery MFMAs
    static constexpr int kValu = KW == 7 ? 2 : 4;
    static constexpr int kDsEvery = KW == 7 ? 3 : 2;
};

__device__ __forceinline__ float snake_reduced(float x, const snake_param & q, bool & slow) {
    const float m = x * q.alpha;
    slow |= !(__builtin_fabsf(m) <= kSinSqFastMax);
    return x + div_by(sin_sq_reduced(m), q.beta, q.rbeta);
}

__device__ __forceinline__ int b_row(int e, int b_magic) {
    return static_cast<int>((static_cast<uint32_t>(e) * static_cast<uint32_t>(b_magic)) >> 24);
}

// After the k = 7 loop of a fused residual unit: h = acc + bias0 goes through
// the post SnakeBeta into LDS in the output tile's layout, H[channel][sample],
// the B operand of the k = 1 conv; the k = 1 weights come straight from
// global memory (64 KB, shared by every workgroup through L2). K runs in a
// permuted order, the same for both operands: at step 4q + r lane group g
// takes channel 16q + 4g + r, so a lane's weights of one row for steps
// 4q .. 4q + 3 are one float4. The result + bias1 + the unit input goes to y
// through the shared epilogue.
__device__ __forceinline__ void residual_tail(const conv_params & p, const fuse_params & f, float * lds,
                                              f32x4v (&acc)[4][4], int tid, int h, int vh, int g, int m,
                                              int64_t t0) {
    float * H = lds;
    snake_param * sp1 = reinterpret_cast<snake_param *>(lds + kMT * kOutStride);
    for (int c = tid; c < kMT; c += kThreads) {
        const float al = p.param_f16 ? h2f(static_cast<const uint16_t *>(f.alpha1_log)[c])
                                     : static_cast<const float *>(f.alpha1_log)[c];
        const float bl = p.param_f16 ? h2f(static_cast<const uint16_t *>(f.beta1_log)[c])
                                     : static_cast<const float *>(f.beta1_log)[c];
        sp1[c] = make_snake_param(al, bl);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int row = h * 64 + 16 * i + 4 * g + u;
            const float bv = p.bias ? p.bias[row] : 0.0f;
            const snake_param q = sp1[row];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float v = acc[i][j][u];
                if (p.bias) v = v + bv;  // the conv's bias add, then SnakeBeta
                H[row * kOutStride + vh * 64 + 16 * j + m] = snake(v, q);
            }
        }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
    const float * wrow = f.w1 + (h * 64 + m) * kMT + 4 * g;  // row h*64 + 16 i + m at + 16 i kMT
    f32x4v wa[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) wa[i] = *reinterpret_cast<const f32x4v *>(wrow + 16 * i * kMT);
#pragma unroll
    for (int q = 0; q < kMT / 16; ++q) {
        f32x4v wn[4];
        if (q + 1 < kMT / 16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) wn[i] = *reinterpret_cast<const f32x4v *>(wrow + 16 * i * kMT + 16 * (q + 1));
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float * brow = H + (16 * q + 4 * g + r) * kOutStride + vh * 64 + m;
            float b[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = brow[16 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[i][r], b[j], acc[i][j], 0, 0, 0);
        }
        if (q + 1 < kMT / 16) {
#pragma unroll
            for (int i = 0; i < 4; ++i) wa[i] = wn[i];
        }
    }
    __syncthreads();  // every wave is done with H before the epilogue reuses the LDS
    conv_params e = p;
    e.bias = f.bias1;
    e.residual = p.x;  // the unit input: y = x + conv(snake(h))
    e.r_pitch = p.x_pitch;
    e.y = f.y;
    e.y_pitch = f.y_pitch;
    e.y_vec = f.y_vec;
    conv_epilogue<false>(e, lds, acc, tid, h, vh, g, m, t0, 0, 0);
}

template <int KW, int NB, bool FUSE>
__global__ __launch_bounds__(kThreads, 2) void snake_conv1d_il(const conv_params p0, const fuse_params f) {
    using S = il_shape<KW>;
    constexpr int CI = S::CI;
    constexpr int NA = S::NA;
    constexpr int BPP = (NB + S::P - 1) / S::P;  // input elements per staging step
    conv_params p = p0;
    const tile_id tl = conv_tile(p0);
    if (!tl.live) return;
    const int n_phase = p.n_phase > 0 ? p.n_phase : 1;
    const int phase = tl.z % n_phase;
    const int split = tl.z / n_phase;
    if (KW == 2) p.w += static_cast<int64_t>(phase) * p.w_phase;  // this phase's weights (one phase otherwise)
    extern __shared__ __attribute__((aligned(16))) float lds[];
    const int buf_floats = a_floats<KW>() + kThreads * NB;
    snake_param * sp = reinterpret_cast<snake_param *>(lds + 2 * buf_floats);  // [c_in] when p.snake
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = wave >> 1;
    const int vh = wave & 1;
    const int m = lane & 15;
    const int g = lane >> 4;
    const int64_t t0 = static_cast<int64_t>(tl.x) * kNT;
    const int co0 = tl.y * kMT;
    const int bw = p.b_width;
    const int n_b = CI * bw;
    // input channels of this workgroup (a split's share, or all); the
    // parameter table is indexed from ci_begin
    int ci_begin, ci_end;
    split_range<CI>(p, split, ci_begin, ci_end);
    // k = 7 divides (faster there, measured); k = 2 multiplies by b_magic
    auto row_of = [&](int e) { return KW == 7 ? e / bw : b_row(e, p.b_magic); };
    const int64_t tb = t0 - p.pad;

    f32x4v ra[NA];
    float rb[NB];
    const int64_t w_row = static_cast<int64_t>(p.c_in) * KW;
    auto load_a = [&](int ci0) {  // weight rows are 16-byte aligned (w_vec)
#pragma unroll
        for (int u = 0; u < NA; ++u) {
            const int e = tid + kThreads * u;
            const int r = e % kMT;
            const int kk = 4 * (e / kMT);
            const int co = co0 + r;
            f32x4v v = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
            if (co < p.c_out && ci0 + (kk + 3) / KW < p.c_in)
                v = *reinterpret_cast<const f32x4v *>(p.w + co * w_row + static_cast<int64_t>(ci0) * KW + kk);
            ra[u] = v;
        }
    };
    auto load_b = [&](int ci0) {
#pragma unroll
        for (int sl = 0; sl < NB; ++sl) {
            const int e = tid + kThreads * sl;
            const int c = row_of(e);
            const int64_t t = tb + (e - c * bw);
            float v = 0.0f;
            if (e < n_b && ci0 + c < p.c_in && t >= 0 && t < p.t_in) v = p.x[static_cast<int64_t>(ci0 + c) * p.x_pitch + t];
            rb[sl] = v;
        }
    };
    load_a(ci_begin);
    load_b(ci_begin);
    if (p.snake) {
        for (int c = tid; c < ci_end - ci_begin; c += kThreads) {
            float al, bl;
            load_snake_logs(p, ci_begin + c, al, bl);
            sp[c] = make_snake_param(al, bl);
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < NA; ++u) store_a_slot<KW>(lds, tid, u, ra[u]);
#pragma unroll
    for (int sl = 0; sl < NB; ++sl) {
        const int e = tid + kThreads * sl;
        const int c = row_of(e);
        float v = rb[sl];
        if (p.snake && e < n_b && ci_begin + c < p.c_in) v = snake(v, sp[c]);
        lds[a_floats<KW>() + e] = v;
    }
    __syncthreads();

    f32x4v acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};

    int buf = 0;
    const int cmax = ci_end - 1;
    for (int ci0 = ci_begin; ci0 < ci_end; ci0 += CI) {
        const bool more = ci0 + CI < ci_end;
        // the next chunk's loads (past the last chunk they are guarded to zeros)
        load_a(ci0 + CI);
        load_b(ci0 + CI);
        const float * As = lds + buf * buf_floats;
        const float * Bs = As + a_floats<KW>();
        f32x4v a;
        float b[4];
        read_operands<KW>(As, Bs, p, 0, g, h, vh, m, a, b);
#pragma unroll
        for (int ks = 0; ks < S::KS - S::P; ++ks) {
            f32x4v an = a;
            float bn[4] = {b[0], b[1], b[2], b[3]};
            read_operands<KW>(As, Bs, p, ks + 1, g, h, vh, m, an, bn);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
            a = an;
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bn[j];
        }
        // second half: each K step also stages its share of the next chunk
        // into the other buffer (last read before the previous barrier);
        // after the last chunk they go unused
        float * An = lds + (buf ^ 1) * buf_floats;
        float * Bn = An + a_floats<KW>();
        bool slow = false;
#pragma unroll
        for (int ks = S::KS - S::P; ks < S::KS; ++ks) {
            const int piece = ks - (S::KS - S::P);
            f32x4v an = a;
            float bn[4] = {b[0], b[1], b[2], b[3]};
            if (ks + 1 < S::KS) read_operands<KW>(As, Bs, p, ks + 1, g, h, vh, m, an, bn);
#pragma unroll
            for (int i = 0; i < S::APP; ++i) {
                const int u = piece * S::APP + i;
                if (u < NA) store_a_slot<KW>(An, tid, u, ra[u]);
            }
#pragma unroll
            for (int i = 0; i < BPP; ++i) {
                const int sl = piece * BPP + i;
                if (sl < NB) {
                    const int e = tid + kThreads * sl;
                    const float v = rb[sl];
                    // without SnakeBeta the value is computed from table
                    // entry 0 (allocated, not filled) and discarded
                    const snake_param q = sp[p.snake ? min(ci0 + CI + row_of(e), cmax) - ci_begin : 0];
                    const float sv = snake_reduced(v, q, slow);
                    Bn[e] = p.snake ? sv : v;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
            // the operand reads first, then each MFMA followed by VALU
            // instructions, with an LDS store after every few
            __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
            for (int q2 = 0; q2 < 16; ++q2) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, S::kValu, 0);
                if (q2 % S::kDsEvery == 0) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
            }
            a = an;
#pragma unroll
            for (int j = 0; j < 4; ++j) b[j] = bn[j];
        }
        if (slow && p.snake && more) {  // rare: arguments beyond the reduced sine's range
#pragma unroll
            for (int sl = 0; sl < NB; ++sl) {
                const int e = tid + kThreads * sl;
                const int c = row_of(e);
                if (e < n_b && ci0 + CI + c < p.c_in) Bn[e] = snake(rb[sl], sp[ci0 + CI + c - ci_begin]);
            }
        }
        __syncthreads();
        buf ^= 1;
    }
    if constexpr (FUSE) {
        residual_tail(p, f, lds, acc, tid, h, vh, g, m, t0);
    } else {
        conv_epilogue<KW == 2>(p.splits > 1 ? split_target(p, tl.z) : p, lds, acc, tid, h, vh, g, m, t0, co0,
                               phase);
    }
}

// y = ((part_0 + part_1) + ...) + bias (+ residual), then the post SnakeBeta
// if any, per float4 of a row: the split launch's partial sums in split
// order, then the unsplit epilogue's steps. Rows of the partials are padded to a multiple of 4
// floats; the padding is summed and dropped.
__global__ __launch_bounds__(kThreads) void split_combine_kernel(const conv_params p) {
    const int64_t groups = (p.t_out + 3) / 4;  // float4 groups per row
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= groups * p.c_out) return;
    const int co = static_cast<int>(e / groups);
    const int64_t t = 4 * (e - co * groups);
    const float * src = p.part + co * p.part_pitch + t;
    f32x4v v = *reinterpret_cast<const f32x4v *>(src);
    for (int z = 1; z < p.splits; ++z) v = v + *reinterpret_cast<const f32x4v *>(src + z * p.part_slice);
    if (p.bias) v = v + p.bias[co];
    snake_param sq{};
    if (p.post_alpha_log) sq = post_param(p, co);
    if (p.y_vec && t + 4 <= p.t_out) {
        if (p.residual) v = *reinterpret_cast<const f32x4v *>(p.residual + co * p.r_pitch + t) + v;
        if (p.post_alpha_log) {
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = snake(v[u], sq);
        }
        *reinterpret_cast<f32x4v *>(p.y + co * p.y_pitch + t) = v;
        return;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (t + q >= p.t_out) break;
        float o = v[q];
        if (p.residual) o = p.residual[co * p.r_pitch + t + q] + o;
        if (p.post_alpha_log) o = snake(o, sq);
        p.y[co * p.y_pitch + t + q] = o;
    }
}

// The transposed convolution's combine, per output sample t of y (coalesced
// writes): t + padding = q * o_stride + r is column q of phase r, whose
// partial sums are added in split order, then the bias, as the scatter
// epilogue adds it. Every t in [0, y_len) is one (q, r) with q <= t_in.
__global__ __launch_bounds__(kThreads) void split_combine_scatter_kernel(const conv_params p) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= p.y_len * p.c_out) return;
    const int co = static_cast<int>(e / p.y_len);
    const int64_t t = e - co * p.y_len;
    const int64_t u = t - p.o_base;  // o_base = -padding <= 0
    const int64_t q = u / p.o_stride;
    const int r = static_cast<int>(u - q * p.o_stride);
    const float * src = p.part + r * p.part_slice + co * p.part_pitch + q;
    float v = src[0];
    for (int j = 1; j < p.splits; ++j) v = v + src[static_cast<int64_t>(j) * p.n_phase * p.part_slice];
    if (p.bias) v = v + p.bias[co];
    p.y[co * p.y_pitch + t] = v;
}

// The launch grid: the XCD-ordered 1-D grid for more than 8 workgroups.
inline dim3 conv_grid(conv_params & p, int phases) {
    const int64_t tx = ceil_div(p.t_out, kNT);
    const int64_t ty = ceil_div(p.c_out, kMT);
    p.xcd_order = tx * ty * phases > 8 && ceil_div(tx * ty, 8) * 8 * phases < INT32_MAX;
    p.tiles_x = static_cast<int32_t>(tx);
    p.tiles = static_cast<int32_t>(tx * ty);
    p.phases = phases;
    if (p.xcd_order) return dim3(static_cast<uint32_t>(ceil_div(tx * ty, 8) * 8 * phases));
    return dim3(static_cast<uint32_t>(tx), static_cast<uint32_t>(ty), static_cast<uint32_t>(phases));
}

// Launches the interleaved kernel when its LDS fits; returns -1 when not.
template <int KW, int NB>
int launch_il(conv_params p, int phases, size_t table, hipStream_t st, const char * what) {
    const size_t bufs = 2 * static_cast<size_t>(a_floats<KW>() + kThreads * NB) * sizeof(float);
    // a table entry even without SnakeBeta: the kernel reads entry 0 then
    const size_t lds = std::max(bufs + (p.snake ? table : sizeof(snake_param)),
                                static_cast<size_t>(kMT) * kOutStride * sizeof(float));
    if (lds > 152 * 1024) return -1;
    p.param_ring = 0;
    p.b_magic = static_cast<int32_t>(((1 << 24) + p.b_width - 1) / p.b_width);
    const void * f = reinterpret_cast<const void *>(&snake_conv1d_il<KW, NB, false>);
    if (const int rc = allow_dynamic_lds(f, 152 * 1024, what); rc != LEVO_HIP_OK) return rc;
    const dim3 grid = conv_grid(p, phases);
    snake_conv1d_il<KW, NB, false><<<grid, kThreads, lds, st>>>(p, fuse_params{});
    return launch_status(what);
}

int launch_split_combine(const conv_params & p, hipStream_t st, const char * what) {
    if (p.scatter) {
        const int64_t n = p.y_len * p.c_out;
        split_combine_scatter_kernel<<<dim3(static_cast<uint32_t>(ceil_div(n, kThreads))), kThreads, 0, st>>>(p);
    } else {
        const int64_t groups = ceil_div(p.t_out, 4) * p.c_out;
        split_combine_kernel<<<dim3(static_cast<uint32_t>(ceil_div(groups, kThreads))), kThreads, 0, st>>>(p);
    }
    return launch_status(what);
}

// One convolution launch (with p.splits > 1: the split launch, then the
// combine).
template <int KW>
int launch_conv(conv_params p, int phases, hipStream_t st, const char * what) {
    if (!p.scatter && p.c_out <= 4 && (KW - 1) * p.dil <= kNarrowMaxSpan) return launch_narrow<KW>(p, st, what);
    constexpr int CI = conv_chunk<KW>::CI;
    const int splits = p.splits > 1 ? p.splits : 1;
    const int gphases = phases * splits;  // the grid's phase axis: phases times splits
    p.n_phase = phases;
    p.b_width = (kNT + (KW - 1) * p.dil + 3) & ~3;
    // each thread stages at most two samples of an input row (one for KW = 2)
    LEVO_REQUIRE(KW == 1 || p.b_width <= (KW == 2 ? 1 : 2) * kThreads, "snake_conv1d: dilation too large");
    p.w_vec = aligned16(p.w) && (static_cast<int64_t>(p.c_in) * KW) % 4 == 0 && p.w_phase % 4 == 0;
    p.y_vec = !p.scatter && aligned16(p.y) && p.y_pitch % 4 == 0 &&
              (p.residual == nullptr || (aligned16(p.residual) && p.r_pitch % 4 == 0));
    const size_t buf = static_cast<size_t>(a_floats<KW>() + CI * p.b_width);
    const size_t tiles = std::max(2 * buf, static_cast<size_t>(kMT) * kOutStride) * sizeof(float);
    const int64_t wgs = ceil_div(p.t_out, kNT) * ceil_div(p.c_out, kMT) * gphases;
    // parameter table: the channels of one workgroup (a split's largest share)
    const int64_t table_channels = splits > 1 ? CI * ceil_div(ceil_div(p.c_in, CI), splits) : p.c_in;
    const size_t table = static_cast<size_t>(table_channels) * sizeof(snake_param);
    // the full parameter table unless it alone keeps a second workgroup off
    // a CU (160 KB of LDS) in a grid that has more than one per CU
    p.param_ring = splits == 1 && p.snake && 2 * (tiles + table) > 160 * 1024 &&
                   2 * (tiles + 2 * CI * sizeof(snake_param)) <= 160 * 1024 && wgs > 256;
    const size_t lds = tiles + (p.snake ? (p.param_ring ? 2 * CI * sizeof(snake_param) : table) : 0);
    LEVO_REQUIRE(lds <= 152 * 1024, "snake_conv1d: dilation or channel count too large for LDS");
    const auto finish = [&](int rc) { return rc == LEVO_HIP_OK && splits > 1 ? launch_split_combine(p, st, what) : rc; };
    if constexpr (KW == 2 || KW == 7) {
        // With the full parameter table even where the other kernel would
        // take the ring: one workgroup per CU of this kernel outruns two of
        // that one (measured at 1024 channels, k = 7). Measured per layer:
        // at k = 7 every decoder layer gains; at k = 2 (the upsamplers) from
        // 512 input channels (16 K steps per chunk pair and up), below that
        // the plain kernel's higher occupancy wins; at k = 1 (four chunks a
        // tile) the plain kernel wins everywhere.
        const int64_t nb = ceil_div(static_cast<int64_t>(CI) * p.b_width, kThreads);
        if (p.w_vec && p.b_width >= kNT && nb <= il_shape<KW>::kMaxNB && (KW == 7 || p.c_in >= 512)) {
            int rc = -1;
            if (KW == 7 && nb <= 5) rc = launch_il<KW, KW == 7 ? 5 : il_shape<KW>::kMaxNB>(p, gphases, table, st, what);
            if (rc < 0) rc = launch_il<KW, il_shape<KW>::kMaxNB>(p, gphases, table, st, what);
            if (rc >= 0) return finish(rc);
        }
    }
    const dim3 grid = conv_grid(p, gphases);
    const void * kernel = p.param_ring ? reinterpret_cast<const void *>(&snake_conv1d_kernel<KW, true>)
                                       : reinterpret_cast<const void *>(&snake_conv1d_kernel<KW, false>);
    if (const int rc = allow_dynamic_lds(kernel, 152 * 1024, what); rc != LEVO_HIP_OK) return rc;
    if (p.param_ring) {
        snake_conv1d_kernel<KW, true><<<grid, kThreads, lds, st>>>(p);
    } else {
        snake_conv1d_kernel<KW, false><<<grid, kThreads, lds, st>>>(p);
    }
    return finish(launch_status(what));
}

}  // namespace

int launch_residual_unit_fused(const float * x, int64_t c, int64_t t, const void * pre_alpha_log,
                               const void * pre_beta_log, const float * w0, const float * b0,
                               const void * post_alpha_log, const void * post_beta_log, const float * w1,
                               const float * b1, int64_t dilation, levo_hip_type param_type, float * y,
                               hipStream_t st) {
    if (c != kMT || dilation < 1 || !aligned16(w0) || !aligned16(w1) || pre_alpha_log == nullptr ||
        pre_beta_log == nullptr || post_alpha_log == nullptr || post_beta_log == nullptr)
        return kNotFused;
    conv_params p{};
    p.x = x;
    p.x_pitch = t;
    p.t_in = t;
    p.alpha_log = pre_alpha_log;
    p.beta_log = pre_beta_log;
    p.param_f16 = param_type == LEVO_HIP_TYPE_F16;
    p.snake = 1;
    p.w = w0;
    p.bias = b0;
    p.y_pitch = t;
    p.t_out = t;  // k 7 at padding 3d keeps the length
    p.c_in = kMT;
    p.c_out = kMT;
    p.pad = static_cast<int32_t>(3 * dilation);
    p.dil = static_cast<int32_t>(dilation);
    p.b_width = (kNT + 6 * p.dil + 3) & ~3;
    p.w_vec = 1;  // 16-byte aligned, c * 7 % 4 == 0
    p.o_stride = 1;
    p.y_len = t;
    const int64_t nb = ceil_div(static_cast<int64_t>(conv_chunk<7>::CI) * p.b_width, kThreads);
    if (nb > il_shape<7>::kMaxNB) return kNotFused;
    const int slots = nb <= 5 ? 5 : il_shape<7>::kMaxNB;
    const size_t bufs = 2 * static_cast<size_t>(a_floats<7>() + kThreads * slots) * sizeof(float);
    const size_t lds = std::max(bufs + kMT * sizeof(snake_param),
                                static_cast<size_t>(kMT) * kOutStride * sizeof(float) + kMT * sizeof(snake_param));
    if (lds > 152 * 1024) return kNotFused;
    fuse_params f{};
    f.w1 = w1;
    f.bias1 = b1;
    f.alpha1_log = post_alpha_log;
    f.beta1_log = post_beta_log;
    f.y = y;
    f.y_pitch = t;
    f.y_vec = aligned16(y) && aligned16(x) && t % 4 == 0;
    const char * what = "levo_hip_vae_residual_unit";
    const dim3 grid = conv_grid(p, 1);
    const void * fn = slots == 5 ? reinterpret_cast<const void *>(&snake_conv1d_il<7, 5, true>)
                                 : reinterpret_cast<const void *>(&snake_conv1d_il<7, il_shape<7>::kMaxNB, true>);
    if (const int rc = allow_dynamic_lds(fn, 152 * 1024, what); rc != LEVO_HIP_OK) return rc;
    if (slots == 5) {
        snake_conv1d_il<7, 5, true><<<grid, kThreads, lds, st>>>(p, f);
    } else {
        snake_conv1d_il<7, il_shape<7>::kMaxNB, true><<<grid, kThreads, lds, st>>>(p, f);
    }
    return launch_status(what);
}

}  // namespace levo_hip

using namespace levo_hip;

namespace levo_hip {
namespace {

constexpr int kMaxSplits = 4;

int64_t split_pitch(int64_t t_out) { return (t_out + 3) / 4 * 4; }

bool ranges_overlap(const void * a, int64_t a_bytes, const void * b, int64_t b_bytes) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + static_cast<uintptr_t>(b_bytes) && pb < pa + static_cast<uintptr_t>(a_bytes);
}

// LDS bytes of the launch launch_conv<KW> makes (interleaved or plain
// kernel) with a SnakeBeta table of table_ch channels.
template <int KW>
int64_t conv_lds_bytes(int64_t c_in, int64_t table_ch, int64_t dil, bool snake, bool w_vec) {
    constexpr int CI = conv_chunk<KW>::CI;
    const int64_t b_width = (kNT + (KW - 1) * dil + 3) & ~int64_t{3};
    const int64_t entry = static_cast<int64_t>(sizeof(snake_param));
    const int64_t out_tile = int64_t{kMT} * kOutStride * static_cast<int64_t>(sizeof(float));
    if constexpr (KW == 2 || KW == 7) {
        const int64_t nb = ceil_div(CI * b_width, kThreads);
        if (w_vec && b_width >= kNT && nb <= il_shape<KW>::kMaxNB && (KW == 7 || c_in >= 512)) {
            const int64_t slots = KW == 7 && nb <= 5 ? 5 : il_shape<KW>::kMaxNB;
            const int64_t bufs = 2 * (a_floats<KW>() + kThreads * slots) * static_cast<int64_t>(sizeof(float));
            return std::max(bufs + (snake ? table_ch * entry : entry), out_tile);
        }
    }
    const int64_t buf = (a_floats<KW>() + CI * b_width) * static_cast<int64_t>(sizeof(float));
    return std::max(2 * buf, out_tile) + (snake ? table_ch * entry : 0);
}

// Splits of a launch of `wgs` workgroups (tiles times stride phases) over
// `chunks` K chunks of CI channels. A grid with fewer workgroups than CUs
// splits up to kMaxSplits ways (two workgroups per CU). A larger grid splits
// in two when that evens its last round: with w workgroups per CU (two when
// the launch's LDS fits twice in a CU, one otherwise; a split halves the
// SnakeBeta table) the launch takes ceil(wgs / (w CUs)) rounds of whole
// tiles, or ceil(2 wgs / (w' CUs)) rounds of half tiles; two splits are taken
// when they need at most 0.8 of the time (632 workgroups of stage 1 at
// 1000 frames: 2 rounds of whole tiles against 3 of halves).
template <int KW>
int64_t pick_splits(int64_t wgs, int64_t chunks, int64_t c_in, int64_t dil, bool snake, bool w_vec) {
    const int cus = device_cu_count();
    if (cus <= 0) return 1;
    if (wgs < cus) return std::min<int64_t>(kMaxSplits, 2 * cus / wgs);
    constexpr int CI = conv_chunk<KW>::CI;
    const int64_t per_cu_1 = conv_lds_bytes<KW>(c_in, c_in, dil, snake, w_vec) <= 80 * 1024 ? 2 : 1;
    const int64_t half = CI * ceil_div(chunks, 2);
    const int64_t per_cu_2 = conv_lds_bytes<KW>(c_in, half, dil, snake, w_vec) <= 80 * 1024 ? 2 : 1;
    const int64_t rounds_1 = ceil_div(wgs, per_cu_1 * cus);
    const int64_t rounds_2 = ceil_div(2 * wgs, per_cu_2 * cus);  // of half tiles
    return rounds_2 * 5 <= rounds_1 * 8 ? 2 : 1;                 // rounds_2 / 2 <= 0.8 rounds_1
}

// levo_hip_snake_conv1d, and with a workspace the split-K form when the grid
// would leave compute units idle: up to two workgroups per CU (at most
// kMaxSplits splits), each split at least two K chunks, as many partial
// slices as the workspace holds.
int conv1d_entry(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in, const void * alpha_log,
                 const void * beta_log, levo_hip_type param_type, const float * weight, int64_t c_out,
                 int64_t kernel, const float * bias, int64_t padding, int64_t dilation, const float * residual,
                 int64_t residual_stride, float * y, int64_t y_stride, float * ws, int64_t ws_floats,
                 const void * post_alpha_log, const void * post_beta_log, hipStream_t st, const char * what) {
    LEVO_REQUIRE(c_in > 0 && c_out > 0 && t_in > 0, "LeVo audio graph: incompatible Conv1d weight/input shapes");
    LEVO_REQUIRE(padding >= 0 && dilation > 0, "LeVo audio graph: invalid Conv1d stride, padding, or dilation");
    LEVO_REQUIRE(kernel == 1 || kernel == 3 || kernel == 5 || kernel == 7, "snake_conv1d: kernel size must be 1, 3, 5 or 7");
    LEVO_REQUIRE(c_in <= (1 << 20) && c_out <= (1 << 20) && t_in < (int64_t{1} << 40) && padding < (1 << 20) &&
                     dilation < (1 << 16),
                 "snake_conv1d: dimensions too large");
    const int64_t t_out = t_in + 2 * padding - dilation * (kernel - 1);
    LEVO_REQUIRE(t_out > 0, "snake_conv1d: the kernel is wider than the padded input");
    LEVO_REQUIRE(ceil_div(t_out, kNT) < (int64_t{1} << 31) && ceil_div(c_out, kMT) < 65536, "snake_conv1d: grid too large");
    LEVO_REQUIRE(x != nullptr && weight != nullptr && y != nullptr, "snake_conv1d: null tensor");
    LEVO_REQUIRE(x_stride >= t_in && y_stride >= t_out && (residual == nullptr || residual_stride >= t_out),
                 "snake_conv1d: row stride smaller than the row");
    const bool snake = alpha_log != nullptr || beta_log != nullptr;
    LEVO_REQUIRE(!snake || (alpha_log != nullptr && beta_log != nullptr),
                 "snake_conv1d: SnakeBeta needs both alpha_log and beta_log");
    LEVO_REQUIRE(!snake || param_type == LEVO_HIP_TYPE_F32 || param_type == LEVO_HIP_TYPE_F16,
                 "LeVo audio graph: SnakeBeta alpha_log must be F32 or F16");
    LEVO_REQUIRE(!snake || c_in <= kMaxSnakeChannels, "snake_conv1d: at most %d input channels with SnakeBeta",
                 kMaxSnakeChannels);
    conv_params p{};
    p.x = x;
    p.x_pitch = x_stride;
    p.t_in = t_in;
    p.alpha_log = alpha_log;
    p.beta_log = beta_log;
    p.param_f16 = param_type == LEVO_HIP_TYPE_F16;
    p.snake = snake;
    p.w = weight;
    p.bias = bias;
    p.residual = residual;
    p.r_pitch = residual_stride;
    p.y = y;
    p.y_pitch = y_stride;
    p.t_out = t_out;
    p.c_in = static_cast<int32_t>(c_in);
    p.c_out = static_cast<int32_t>(c_out);
    p.pad = static_cast<int32_t>(padding);
    p.dil = static_cast<int32_t>(dilation);
    p.b_width = 0;
    p.w_vec = 0;
    p.y_vec = 0;
    p.o_stride = 1;
    p.o_base = 0;
    p.y_len = t_out;
    p.w_phase = 0;
    p.scatter = 0;
    p.param_ring = 0;
    p.splits = 1;
    p.post_alpha_log = post_alpha_log;
    p.post_beta_log = post_beta_log;
    LEVO_REQUIRE(post_alpha_log == nullptr || (post_beta_log != nullptr && c_out > 4),
                 "snake_conv1d: post SnakeBeta needs both parameters and more than 4 outputs");
    LEVO_REQUIRE(post_alpha_log == nullptr || param_type == LEVO_HIP_TYPE_F32 || param_type == LEVO_HIP_TYPE_F16,
                 "LeVo audio graph: SnakeBeta alpha_log must be F32 or F16");
    if (ws != nullptr && c_out > 4) {
        LEVO_REQUIRE(aligned16(ws) && ws_floats >= 0, "snake_conv1d: workspace must be 16-byte aligned");
        const int64_t tiles = ceil_div(t_out, kNT) * ceil_div(c_out, kMT);
        const int64_t chunks = ceil_div(c_in, kernel == 1 ? conv_chunk<1>::CI : conv_chunk<7>::CI);
        const int64_t pitch = split_pitch(t_out);
        const bool w_vec = aligned16(weight) && (c_in * kernel) % 4 == 0;
        int64_t splits;
        switch (kernel) {
            case 1: splits = pick_splits<1>(tiles, chunks, c_in, dilation, snake, w_vec); break;
            case 3: splits = pick_splits<3>(tiles, chunks, c_in, dilation, snake, w_vec); break;
            case 5: splits = pick_splits<5>(tiles, chunks, c_in, dilation, snake, w_vec); break;
            default: splits = pick_splits<7>(tiles, chunks, c_in, dilation, snake, w_vec); break;
        }
        while (splits > 1 && (chunks / splits < 2 || splits * c_out * pitch > ws_floats)) --splits;
        if (splits > 1) {
            const int64_t bytes = splits * c_out * pitch * static_cast<int64_t>(sizeof(float));
            const int64_t elt = static_cast<int64_t>(sizeof(float));
            LEVO_REQUIRE(!ranges_overlap(ws, bytes, y, c_out * y_stride * elt) &&
                             !ranges_overlap(ws, bytes, x, c_in * x_stride * elt) &&
                             (residual == nullptr || !ranges_overlap(ws, bytes, residual, c_out * residual_stride * elt)),
                         "snake_conv1d: workspace overlaps a tensor");
            p.splits = static_cast<int32_t>(splits);
            p.part = ws;
            p.part_slice = c_out * pitch;
            p.part_pitch = pitch;
        }
    }
    switch (kernel) {
        case 1: return launch_conv<1>(p, 1, st, what);
        case 3: return launch_conv<3>(p, 1, st, what);
        case 5: return launch_conv<5>(p, 1, st, what);
        default: return launch_conv<7>(p, 1, st, what);
    }
}

}  // namespace
}  // namespace levo_hip

extern "C" int levo_hip_snake_conv1d(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                     const void * alpha_log, const void * beta_log, levo_hip_type param_type,
                                     const float * weight, int64_t c_out, int64_t kernel, const float * bias,
                                     int64_t padding, int64_t dilation, const float * residual,
                                     int64_t residual_stride, float * y, int64_t y_stride,
                                     levo_hip_stream_t stream) {
    return conv1d_entry(x, x_stride, c_in, t_in, alpha_log, beta_log, param_type, weight, c_out, kernel, bias,
                        padding, dilation, residual, residual_stride, y, y_stride, nullptr, 0, nullptr, nullptr,
                        as_hip(stream), "levo_hip_snake_conv1d");
}

namespace levo_hip {

int snake_conv1d_post(const float * x, int64_t c_in, int64_t t, const void * alpha_log, const void * beta_log,
                      levo_hip_type param_type, const float * weight, int64_t c_out, int64_t kernel,
                      const float * bias, int64_t padding, int64_t dilation, float * y, const void * post_alpha_log,
                      const void * post_beta_log, float * ws, int64_t ws_floats, hipStream_t st) {
    return conv1d_entry(x, t, c_in, t, alpha_log, beta_log, param_type, weight, c_out, kernel, bias, padding,
                        dilation, nullptr, 0, y, t, ws, ws_floats, post_alpha_log, post_beta_log, st,
                        "levo_hip_vae_decode");
}

}  // namespace levo_hip

extern "C" int64_t levo_hip_snake_conv1d_split_workspace_floats(int64_t c_out, int64_t t_out) {
    if (c_out <= 0 || t_out <= 0 || c_out > (1 << 20) || t_out >= (int64_t{1} << 40)) return -1;
    return kMaxSplits * c_out * split_pitch(t_out);
}

extern "C" int levo_hip_snake_conv1d_split(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                           const void * alpha_log, const void * beta_log,
                                           levo_hip_type param_type, const float * weight, int64_t c_out,
                                           int64_t kernel, const float * bias, int64_t padding, int64_t dilation,
                                           const float * residual, int64_t residual_stride, float * y,
                                           int64_t y_stride, float * workspace, int64_t workspace_floats,
                                           levo_hip_stream_t stream) {
    return conv1d_entry(x, x_stride, c_in, t_in, alpha_log, beta_log, param_type, weight, c_out, kernel, bias,
                        padding, dilation, residual, residual_stride, y, y_stride, workspace, workspace_floats,
                        nullptr, nullptr, as_hip(stream), "levo_hip_snake_conv1d_split");
}

namespace levo_hip {
namespace {

// packed[r][co][ci][0] = w[ci][co][r + stride], packed[r][co][ci][1] = w[ci][co][r]:
// phase r of the transposed convolution as a 2-tap convolution over
// x[q - 1], x[q].
__global__ __launch_bounds__(kThreads) void pack_transpose_kernel(const float * __restrict__ w, float * packed,
                                                                  int64_t c_in, int64_t c_out, int32_t stride) {
    const int64_t n = static_cast<int64_t>(stride) * c_out * c_in;
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= n) return;
    const int64_t ci = e % c_in;
    const int64_t co = (e / c_in) % c_out;
    const int64_t r = e / (c_in * c_out);
    const int64_t k = 2 * static_cast<int64_t>(stride);
    const float * src = w + (ci * c_out + co) * k;
    packed[2 * e] = src[r + stride];
    packed[2 * e + 1] = src[r];
}

}  // namespace
}  // namespace levo_hip

extern "C" int levo_hip_conv_transpose1d_pack_weights(const float * weight, float * packed, int64_t c_in,
                                                      int64_t c_out, int64_t stride, levo_hip_stream_t stream) {
    LEVO_REQUIRE(c_in > 0 && c_out > 0 && stride > 0, "LeVo audio graph: incompatible ConvTranspose1d weight/input shapes");
    LEVO_REQUIRE(c_in <= (1 << 20) && c_out <= (1 << 20) && stride <= 64, "conv_transpose1d: dimensions too large");
    LEVO_REQUIRE(weight != nullptr && packed != nullptr, "conv_transpose1d: null tensor");
    const int64_t n = stride * c_out * c_in;
    pack_transpose_kernel<<<static_cast<uint32_t>(ceil_div(n, kThreads)), kThreads, 0, as_hip(stream)>>>(
            weight, packed, c_in, c_out, static_cast<int32_t>(stride));
    return launch_status("levo_hip_conv_transpose1d_pack_weights");
}

namespace levo_hip {
namespace {

int conv_transpose_entry(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in, const void * alpha_log,
                         const void * beta_log, levo_hip_type param_type, const float * packed_weight,
                         int64_t c_out, int64_t stride, const float * bias, int64_t padding, float * y,
                         int64_t y_stride, float * ws, int64_t ws_floats, hipStream_t st, const char * what) {
    LEVO_REQUIRE(c_in > 0 && c_out > 0 && t_in > 0, "LeVo audio graph: incompatible ConvTranspose1d weight/input shapes");
    LEVO_REQUIRE(stride > 0 && padding >= 0, "LeVo audio graph: invalid ConvTranspose1d stride or padding");
    LEVO_REQUIRE(stride <= 64 && c_in <= (1 << 20) && c_out <= (1 << 20) && t_in < (int64_t{1} << 36),
                 "conv_transpose1d: dimensions too large");
    const int64_t y_len = (t_in + 1) * stride - 2 * padding;
    LEVO_REQUIRE(y_len > 0, "LeVo audio graph: ConvTranspose1d padding removes the entire output");
    LEVO_REQUIRE(x != nullptr && packed_weight != nullptr && y != nullptr, "conv_transpose1d: null tensor");
    LEVO_REQUIRE(x_stride >= t_in && y_stride >= y_len, "conv_transpose1d: row stride smaller than the row");
    const bool snake = alpha_log != nullptr || beta_log != nullptr;
    LEVO_REQUIRE(!snake || (alpha_log != nullptr && beta_log != nullptr),
                 "snake_conv1d: SnakeBeta needs both alpha_log and beta_log");
    LEVO_REQUIRE(!snake || param_type == LEVO_HIP_TYPE_F32 || param_type == LEVO_HIP_TYPE_F16,
                 "LeVo audio graph: SnakeBeta alpha_log must be F32 or F16");
    LEVO_REQUIRE(!snake || c_in <= kMaxSnakeChannels, "snake_conv1d: at most %d input channels with SnakeBeta",
                 kMaxSnakeChannels);
    LEVO_REQUIRE(ceil_div(t_in + 1, kNT) < (int64_t{1} << 31) && ceil_div(c_out, kMT) < 65536,
                 "conv_transpose1d: grid too large");
    conv_params p{};
    p.x = x;
    p.x_pitch = x_stride;
    p.t_in = t_in;
    p.alpha_log = alpha_log;
    p.beta_log = beta_log;
    p.param_f16 = param_type == LEVO_HIP_TYPE_F16;
    p.snake = snake;
    p.w = packed_weight;
    p.bias = bias;
    p.residual = nullptr;
    p.r_pitch = 0;
    p.y = y;
    p.y_pitch = y_stride;
    p.t_out = t_in + 1;  // columns q = 0 .. t_in of every phase
    p.c_in = static_cast<int32_t>(c_in);
    p.c_out = static_cast<int32_t>(c_out);
    p.pad = 1;
    p.dil = 1;
    p.b_width = 0;
    p.w_vec = 0;
    p.y_vec = 0;
    p.o_stride = static_cast<int32_t>(stride);
    p.o_base = static_cast<int32_t>(-padding);
    p.y_len = y_len;
    p.w_phase = c_out * c_in * 2;
    p.scatter = 1;
    p.param_ring = 0;
    p.splits = 1;
    if (ws != nullptr) {
        LEVO_REQUIRE(aligned16(ws) && ws_floats >= 0, "conv_transpose1d: workspace must be 16-byte aligned");
        const int64_t wgs = ceil_div(t_in + 1, kNT) * ceil_div(c_out, kMT) * stride;
        const int64_t chunks = ceil_div(c_in, conv_chunk<2>::CI);
        const int64_t pitch = split_pitch(t_in + 1);
        const bool w_vec = aligned16(packed_weight) && (c_in * 2) % 4 == 0 && (c_out * c_in * 2) % 4 == 0;
        int64_t splits = pick_splits<2>(wgs, chunks, c_in, 1, snake, w_vec);
        while (splits > 1 && (chunks / splits < 2 || splits * stride * c_out * pitch > ws_floats)) --splits;
        if (splits > 1) {
            const int64_t bytes = splits * stride * c_out * pitch * static_cast<int64_t>(sizeof(float));
            const int64_t elt = static_cast<int64_t>(sizeof(float));
            LEVO_REQUIRE(!ranges_overlap(ws, bytes, y, c_out * y_stride * elt) &&
                             !ranges_overlap(ws, bytes, x, c_in * x_stride * elt),
                         "conv_transpose1d: workspace overlaps a tensor");
            p.splits = static_cast<int32_t>(splits);
            p.part = ws;
            p.part_slice = c_out * pitch;
            p.part_pitch = pitch;
        }
    }
    return launch_conv<2>(p, static_cast<int>(stride), st, what);
}

}  // namespace
}  // namespace levo_hip

extern "C" int levo_hip_snake_conv_transpose1d(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                               const void * alpha_log, const void * beta_log,
                                               levo_hip_type param_type, const float * packed_weight,
                                               int64_t c_out, int64_t stride, const float * bias, int64_t padding,
                                               float * y, int64_t y_stride, levo_hip_stream_t stream) {
    return conv_transpose_entry(x, x_stride, c_in, t_in, alpha_log, beta_log, param_type, packed_weight, c_out,
                                stride, bias, padding, y, y_stride, nullptr, 0, as_hip(stream),
                                "levo_hip_snake_conv_transpose1d");
}

extern "C" int64_t levo_hip_snake_conv_transpose1d_split_workspace_floats(int64_t c_out, int64_t t_in,
                                                                         int64_t stride) {
    if (c_out <= 0 || t_in <= 0 || stride <= 0 || c_out > (1 << 20) || stride > 64 || t_in >= (int64_t{1} << 36))
        return -1;
    return kMaxSplits * stride * c_out * split_pitch(t_in + 1);
}

extern "C" int levo_hip_snake_conv_transpose1d_split(const float * x, int64_t x_stride, int64_t c_in, int64_t t_in,
                                                     const void * alpha_log, const void * beta_log,
                                                     levo_hip_type param_type, const float * packed_weight,
                                                     int64_t c_out, int64_t stride, const float * bias,
                                                     int64_t padding, float * y, int64_t y_stride, float * workspace,
                                                     int64_t workspace_floats, levo_hip_stream_t stream) {
    return conv_transpose_entry(x, x_stride, c_in, t_in, alpha_log, beta_log, param_type, packed_weight, c_out,
                                stride, bias, padding, y, y_stride, workspace, workspace_floats, as_hip(stream),
                                "levo_hip_snake_conv_transpose1d_split");
}
