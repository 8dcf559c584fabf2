// SnakeBeta activation, one HBM pass: y = x + sin^2(x * alpha_c) / beta_c.
//
// Replaces the five-node ggml chain of levo::detail::snake_beta
// (src/levo-audio-ops.cpp:146-151: mul -> sin -> sqr -> div -> add, plus the
// per-channel exp / scale_bias of the log-domain parameters) with one kernel
// that reads x once and writes y once (8 B/element instead of ~44).
//
// Layout: x is [channels][time] (ggml ne0 = time contiguous). The grid walks
// the flattened [channels x time] space in tiles of 256 * VPT dwordx4 vectors;
// a tile's channel span is resolved once and alpha_c, beta_c and 1/beta_c are
// computed into LDS by the tile's threads, so each element does one LDS read
// instead of two exp evaluations.
#include "common.hpp"
#include "snake_math.hpp"

#include <algorithm>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;

// LDS bytes for the parameters of every channel a tile of `items` consecutive
// vectors (or scalars) can touch, with `row` items per channel: a range of E
// flattened indices spans at most (E - 1) / row + 2 rows.
size_t tile_param_bytes(int64_t items, int64_t row, int64_t channels);

// Exact n / d for n < 2^31 (Granlund-Montgomery with N = 31):
// m = ceil(2^(31+l) / d), l = ceil(log2 d), q = (n * m) >> (31 + l).
struct fast_div {
    uint32_t d;
    uint32_t m;
    uint32_t s;
};

fast_div make_fast_div(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t{1} << l) < d) ++l;
    const uint64_t p = uint64_t{1} << (31 + l);
    fast_div f;
    f.d = d;
    f.m = static_cast<uint32_t>((p + d - 1) / d);
    f.s = 31 + l;
    return f;
}

__device__ __forceinline__ uint32_t div_of(uint32_t n, fast_div f) {
    return static_cast<uint32_t>((static_cast<uint64_t>(n) * f.m) >> f.s);
}

template <typename P>
__device__ __forceinline__ void load_tile_params(snake_param * lds, const P * alpha_log,
                                                 const P * beta_log, uint32_t c0, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
        lds[i] = make_snake_param(param_f32(alpha_log, c0 + i), param_f32(beta_log, c0 + i));
    }
}

// Vector path: time, both strides multiple of 4, pointers 16-byte aligned.
// y may equal x (in place): each thread loads all its vectors before storing.
template <typename P, int VPT>
__global__ __launch_bounds__(kThreads) void snake_beta_vec(
        const float * x, int64_t x_stride, const P * __restrict__ alpha_log,
        const P * __restrict__ beta_log, float * y, int64_t y_stride, uint32_t total4,
        fast_div div_t4) {
    extern __shared__ snake_param params[];  // sized by tile_param_bytes
    constexpr uint32_t tile = kThreads * VPT;
    const uint32_t first = blockIdx.x * tile;
    const uint32_t last = min(first + tile, total4) - 1;
    const uint32_t c0 = div_of(first, div_t4);
    const uint32_t c1 = div_of(last, div_t4);

    // Four vectors per thread (the mid-size tensors): x is requested first
    // and the parameter set-up overlaps its loads (128 x 48000: 9.87 -> 9.44
    // us); two (the largest): the parameters first, which measured 0.7%
    // faster there.
    if constexpr (VPT < 4) load_tile_params(params, alpha_log, beta_log, c0, c1 - c0 + 1);
    f32x4 v[VPT];
    uint32_t ch[VPT];
    uint32_t t4[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint32_t f = first + threadIdx.x + j * kThreads;
        ch[j] = div_of(f, div_t4);
        t4[j] = f - ch[j] * div_t4.d;
        if (f < total4) {
            v[j] = __builtin_nontemporal_load(
                reinterpret_cast<const f32x4 *>(x + static_cast<int64_t>(ch[j]) * x_stride) + t4[j]);
        }
    }
    if constexpr (VPT >= 4) {
        __builtin_amdgcn_sched_barrier(0);
        load_tile_params(params, alpha_log, beta_log, c0, c1 - c0 + 1);
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint32_t f = first + threadIdx.x + j * kThreads;
        if (f < total4) {
            const snake_param q = params[ch[j] - c0];
            f32x4 r;
            r.x = snake(v[j].x, q);
            r.y = snake(v[j].y, q);
            r.z = snake(v[j].z, q);
            r.w = snake(v[j].w, q);
            __builtin_nontemporal_store(
                r, reinterpret_cast<f32x4 *>(y + static_cast<int64_t>(ch[j]) * y_stride) + t4[j]);
        }
    }
}

// Small tensors (latency-bound launches): one vector per thread with the
// channel's parameters computed by the thread itself (two exps per four
// elements), so no LDS round trip or barrier sits on the critical path.
template <typename P>
__global__ __launch_bounds__(kThreads) void snake_beta_vec_direct(
        const float * x, int64_t x_stride, const P * __restrict__ alpha_log,
        const P * __restrict__ beta_log, float * y, int64_t y_stride, uint32_t total4,
        fast_div div_t4) {
    const uint32_t f = blockIdx.x * kThreads + threadIdx.x;
    if (f >= total4) return;
    const uint32_t ch = div_of(f, div_t4);
    const uint32_t t4 = f - ch * div_t4.d;
    const f32x4 v =
            __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(x + static_cast<int64_t>(ch) * x_stride) + t4);
    const snake_param q = make_snake_param(param_f32(alpha_log, ch), param_f32(beta_log, ch));
    f32x4 r;
    r.x = snake(v.x, q);
    r.y = snake(v.y, q);
    r.z = snake(v.z, q);
    r.w = snake(v.w, q);
    __builtin_nontemporal_store(r, reinterpret_cast<f32x4 *>(y + static_cast<int64_t>(ch) * y_stride) + t4);
}

// Scalar path for any time / stride / alignment.
template <typename P>
__global__ __launch_bounds__(kThreads) void snake_beta_scalar(
        const float * x, int64_t x_stride, const P * __restrict__ alpha_log,
        const P * __restrict__ beta_log, float * y, int64_t y_stride, uint32_t total,
        fast_div div_t) {
    extern __shared__ snake_param params[];  // sized by tile_param_bytes
    constexpr uint32_t tile = kThreads * 4;
    const uint32_t first = blockIdx.x * tile;
    const uint32_t last = min(first + tile, total) - 1;
    const uint32_t c0 = div_of(first, div_t);
    const uint32_t c1 = div_of(last, div_t);
    load_tile_params(params, alpha_log, beta_log, c0, c1 - c0 + 1);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t f = first + threadIdx.x + j * kThreads;
        if (f < total) {
            const uint32_t c = div_of(f, div_t);
            const uint32_t t = f - c * div_t.d;
            const float xv = x[static_cast<int64_t>(c) * x_stride + t];
            y[static_cast<int64_t>(c) * y_stride + t] = snake(xv, params[c - c0]);
        }
    }
}

size_t tile_param_bytes(int64_t items, int64_t row, int64_t channels) {
    const int64_t span = (items - 1) / row + 2;
    return static_cast<size_t>(span < channels ? span : channels) * sizeof(snake_param);
}

template <typename P, int VPT>
void launch_vec(const float * x, int64_t x_stride, const P * a, const P * b, float * y, int64_t y_stride,
                int64_t channels, uint32_t total4, uint32_t t4, hipStream_t stream) {
    const uint32_t grid = static_cast<uint32_t>(ceil_div(total4, kThreads * VPT));
    const size_t lds = tile_param_bytes(kThreads * VPT, t4, channels);
    snake_beta_vec<P, VPT><<<grid, kThreads, lds, stream>>>(x, x_stride, a, b, y, y_stride, total4,
                                                            make_fast_div(t4));
}

template <typename P>
int launch_snake(const float * x, int64_t x_stride, const P * a, const P * b, float * y,
                 int64_t y_stride, int64_t channels, int64_t time, hipStream_t stream) {
    const int64_t total = channels * time;
    const bool vec = (time % 4 == 0) && (x_stride % 4 == 0) && (y_stride % 4 == 0) &&
                     aligned16(x) && aligned16(y);
    if (vec) {
        const uint32_t total4 = static_cast<uint32_t>(total / 4);
        const uint32_t t4 = static_cast<uint32_t>(time / 4);
        // By size, as measured on MI355X: below 4 M elements one vector per
        // thread with per-thread parameters; four vectors per thread in the
        // mid range; two for the largest (fewest parameter set-ups without a
        // long tail).
        if (total4 < (1u << 20))
            snake_beta_vec_direct<P><<<static_cast<uint32_t>(ceil_div(total4, kThreads)), kThreads, 0, stream>>>(
                    x, x_stride, a, b, y, y_stride, total4, make_fast_div(t4));
        else if (total4 < (1u << 23)) launch_vec<P, 4>(x, x_stride, a, b, y, y_stride, channels, total4, t4, stream);
        else launch_vec<P, 2>(x, x_stride, a, b, y, y_stride, channels, total4, t4, stream);
    } else {
        const uint32_t grid = static_cast<uint32_t>(ceil_div(total, kThreads * 4));
        const size_t lds = tile_param_bytes(kThreads * 4, time, channels);
        snake_beta_scalar<P><<<grid, kThreads, lds, stream>>>(x, x_stride, a, b, y, y_stride,
                                                             static_cast<uint32_t>(total),
                                                             make_fast_div(static_cast<uint32_t>(time)));
    }
    return launch_status("levo_hip_snake_beta");
}

// ---- batch: independent SnakeBeta jobs in one launch -----------------------
//
// One workgroup per tile of 256 * kBatchVPT vectors of one job (the jobs'
// tiles laid end to end on the grid), with the tile's channel parameters in
// LDS as in snake_beta_vec: the small jobs' tiles run beside the large ones'
// instead of each paying a launch and a ramp of its own.
constexpr int kMaxBatchJobs = 16;
constexpr int kBatchVPT = 2;

struct batch_job {
    const float * x;
    float * y;
    const void * alpha_log;
    const void * beta_log;
    int64_t x_stride;
    int64_t y_stride;
    fast_div div_t4;   // vectors per row
    uint32_t total4;   // vectors of the job
    uint32_t tile0;    // first workgroup of the job
    int32_t param_f16;
};

struct batch_args {
    batch_job job[kMaxBatchJobs];
    int32_t n;
};

__device__ __forceinline__ float batch_param(const void * p, int f16, uint32_t i) {
    return f16 ? param_f32(static_cast<const uint16_t *>(p), i) : param_f32(static_cast<const float *>(p), i);
}

__global__ __launch_bounds__(kThreads) void snake_beta_batch_kernel(const batch_args args) {
    extern __shared__ snake_param params[];  // sized by the largest tile_param_bytes of the jobs
    int j = 0;
    for (int i = 1; i < args.n; ++i) {
        if (args.job[i].tile0 <= blockIdx.x) j = i;  // tiles are in job order
    }
    const batch_job & b = args.job[j];
    constexpr uint32_t tile = kThreads * kBatchVPT;
    const uint32_t first = (blockIdx.x - b.tile0) * tile;
    const uint32_t last = min(first + tile, b.total4) - 1;
    const uint32_t c0 = div_of(first, b.div_t4);
    const uint32_t c1 = div_of(last, b.div_t4);
    for (uint32_t i = threadIdx.x; i <= c1 - c0; i += kThreads) {
        params[i] = make_snake_param(batch_param(b.alpha_log, b.param_f16, c0 + i),
                                     batch_param(b.beta_log, b.param_f16, c0 + i));
    }
    f32x4 v[kBatchVPT];
    uint32_t ch[kBatchVPT];
    uint32_t t4[kBatchVPT];
#pragma unroll
    for (int k = 0; k < kBatchVPT; ++k) {
        const uint32_t f = first + threadIdx.x + k * kThreads;
        ch[k] = div_of(f, b.div_t4);
        t4[k] = f - ch[k] * b.div_t4.d;
        if (f < b.total4) {
            v[k] = __builtin_nontemporal_load(
                    reinterpret_cast<const f32x4 *>(b.x + static_cast<int64_t>(ch[k]) * b.x_stride) + t4[k]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kBatchVPT; ++k) {
        const uint32_t f = first + threadIdx.x + k * kThreads;
        if (f < b.total4) {
            const snake_param q = params[ch[k] - c0];
            f32x4 r;
            r.x = snake(v[k].x, q);
            r.y = snake(v[k].y, q);
            r.z = snake(v[k].z, q);
            r.w = snake(v[k].w, q);
            __builtin_nontemporal_store(
                    r, reinterpret_cast<f32x4 *>(b.y + static_cast<int64_t>(ch[k]) * b.y_stride) + t4[k]);
        }
    }
}

}  // namespace
}  // namespace levo_hip

extern "C" int levo_hip_snake_beta_batch(const levo_hip_snake_job * jobs, int n_jobs, levo_hip_stream_t stream) {
    using namespace levo_hip;
    LEVO_REQUIRE(n_jobs >= 0 && n_jobs <= kMaxBatchJobs, "snake_beta_batch: 0 to %d jobs", kMaxBatchJobs);
    LEVO_REQUIRE(n_jobs == 0 || jobs != nullptr, "snake_beta_batch: null job list");
    // Every job is checked before anything is launched, so a rejected call
    // leaves every output untouched.
    batch_args args{};
    args.n = 0;
    uint64_t tiles = 0;
    size_t lds = 0;
    bool scalar[kMaxBatchJobs] = {};
    for (int i = 0; i < n_jobs; ++i) {
        const levo_hip_snake_job & jb = jobs[i];
        LEVO_REQUIRE(jb.channels >= 0 && jb.time >= 0, "LeVo audio graph: SnakeBeta shape must be non-negative");
        if (jb.channels == 0 || jb.time == 0) continue;
        LEVO_REQUIRE(jb.x != nullptr && jb.y != nullptr, "LeVo audio graph: SnakeBeta input or output is null");
        LEVO_REQUIRE(jb.alpha_log != nullptr && jb.beta_log != nullptr,
                     "LeVo audio graph: SnakeBeta alpha_log or beta_log is null");
        LEVO_REQUIRE(jb.param_type == LEVO_HIP_TYPE_F32 || jb.param_type == LEVO_HIP_TYPE_F16,
                     "LeVo audio graph: SnakeBeta alpha_log must be F32 or F16");
        LEVO_REQUIRE(jb.x_stride >= jb.time && jb.y_stride >= jb.time,
                     "LeVo audio graph: SnakeBeta row stride is smaller than the time length");
        LEVO_REQUIRE(jb.x != jb.y || jb.x_stride == jb.y_stride,
                     "LeVo audio graph: in-place SnakeBeta needs equal input and output strides");
        LEVO_REQUIRE(jb.channels * jb.time < (int64_t{1} << 31) && jb.channels < (int64_t{1} << 30),
                     "LeVo audio graph: SnakeBeta tensor exceeds 2^31 elements");
        const bool vec = jb.time % 4 == 0 && jb.x_stride % 4 == 0 && jb.y_stride % 4 == 0 && aligned16(jb.x) &&
                         aligned16(jb.y);
        if (!vec) {  // the single-job path's scalar kernel, launched below
            scalar[i] = true;
            continue;
        }
        batch_job & b = args.job[args.n++];
        const uint32_t t4 = static_cast<uint32_t>(jb.time / 4);
        b.x = jb.x;
        b.y = jb.y;
        b.alpha_log = jb.alpha_log;
        b.beta_log = jb.beta_log;
        b.x_stride = jb.x_stride;
        b.y_stride = jb.y_stride;
        b.div_t4 = make_fast_div(t4);
        b.total4 = static_cast<uint32_t>(jb.channels * jb.time / 4);
        b.tile0 = static_cast<uint32_t>(tiles);
        b.param_f16 = jb.param_type == LEVO_HIP_TYPE_F16;
        tiles += ceil_div(b.total4, kThreads * kBatchVPT);
        lds = std::max(lds, tile_param_bytes(kThreads * kBatchVPT, t4, jb.channels));
    }
    LEVO_REQUIRE(tiles < (uint64_t{1} << 31), "snake_beta_batch: too many tiles");
    for (int i = 0; i < n_jobs; ++i) {
        if (!scalar[i]) continue;
        const levo_hip_snake_job & jb = jobs[i];
        const int st = levo_hip_snake_beta(jb.x, jb.x_stride, jb.alpha_log, jb.beta_log, jb.param_type, jb.y,
                                           jb.y_stride, jb.channels, jb.time, stream);
        if (st != LEVO_HIP_OK) return st;
    }
    if (args.n == 0) return LEVO_HIP_OK;
    snake_beta_batch_kernel<<<static_cast<uint32_t>(tiles), kThreads, lds, as_hip(stream)>>>(args);
    return launch_status("levo_hip_snake_beta_batch");
}

extern "C" int levo_hip_snake_beta(const float * x, int64_t x_stride, const void * alpha_log,
                                   const void * beta_log, levo_hip_type param_type, float * y,
                                   int64_t y_stride, int64_t channels, int64_t time,
                                   levo_hip_stream_t stream) {
    using namespace levo_hip;
    LEVO_REQUIRE(channels >= 0 && time >= 0, "LeVo audio graph: SnakeBeta shape must be non-negative");
    if (channels == 0 || time == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(x != nullptr, "LeVo audio graph: SnakeBeta input is null");
    LEVO_REQUIRE(y != nullptr, "LeVo audio graph: SnakeBeta output is null");
    LEVO_REQUIRE(alpha_log != nullptr, "LeVo audio graph: SnakeBeta alpha_log is null");
    LEVO_REQUIRE(beta_log != nullptr, "LeVo audio graph: SnakeBeta beta_log is null");
    LEVO_REQUIRE(param_type == LEVO_HIP_TYPE_F32 || param_type == LEVO_HIP_TYPE_F16,
                 "LeVo audio graph: SnakeBeta alpha_log must be F32 or F16");
    LEVO_REQUIRE(x_stride >= time && y_stride >= time,
                 "LeVo audio graph: SnakeBeta row stride is smaller than the time length");
    LEVO_REQUIRE(x != y || x_stride == y_stride,
                 "LeVo audio graph: in-place SnakeBeta needs equal input and output strides");
    LEVO_REQUIRE(channels * time < (int64_t{1} << 31) && channels < (int64_t{1} << 30),
                 "LeVo audio graph: SnakeBeta tensor exceeds 2^31 elements");
    if (param_type == LEVO_HIP_TYPE_F32)
        return launch_snake(x, x_stride, static_cast<const float *>(alpha_log),
                            static_cast<const float *>(beta_log), y, y_stride, channels, time,
                            as_hip(stream));
    return launch_snake(x, x_stride, static_cast<const uint16_t *>(alpha_log),
                        static_cast<const uint16_t *>(beta_log), y, y_stride, channels, time,
                        as_hip(stream));
}
