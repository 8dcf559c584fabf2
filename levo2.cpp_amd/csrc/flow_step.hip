// The Flow renderer's per-step host work with the estimator's tensors left in
// HBM: the input rows the estimator reads and the Euler step that consumes
// its output.
//
//   assemble_input: model_input[b][f] = mask_embedding[f] | context[f] |
//       (b unconditional ? 0 : conditioning[f]) | state_t[f]
//       -- append_model_row, src/levo-flow-renderer.cpp:35-53, for every row
//       of estimator_input (:287-295), with the step's in-context prefix
//       (:93-101) already applied to the state columns.
//   step: v = u + g * (c - u) read from the last `latent` columns of the
//       estimator output (src/levo-flow-estimator.cpp:390-399; CFG lambda
//       src/levo-flow-renderer.cpp:301-309); state = x_t + dt * v with x_t the
//       state after the prefix interpolation (:93-105); the finiteness checks
//       (:104, :106); then either the next step's state columns of
//       model_input, or, after the last step, the prefix restore (:112-113)
//       and denormalize_latents (src/levo-flow-conditioning.cpp:124-133).
//   normalize / denormalize: the per-channel latent statistics of
//       conditioning (src/levo-flow-conditioning.cpp:113-133) on their own.
//
// The state buffer always holds the reference's `state` after the step (its
// checkpoint), so a resume or checkpoint matches bit for bit. Arithmetic is
// the reference's F32 two-rounding chain (no FMA contraction in this
// library). Both kernels stream with dwordx4 accesses when every width, pitch
// and column offset is a multiple of 4 floats and the pointers are 16-byte
// aligned (LeVo's 24 | 64 | 2048 | 64 rows of 2200 are); otherwise one
// element per thread.
#include "common.hpp"

namespace levo_hip {
namespace {

constexpr int kThreads = 256;

template <int VEC>
struct vec_t;
template <>
struct vec_t<4> {
    typedef f32x4 type;
};
template <>
struct vec_t<1> {
    typedef float type;
};

template <int VEC>
__device__ __forceinline__ typename vec_t<VEC>::type load_vec(const float * p) {
    return *reinterpret_cast<const typename vec_t<VEC>::type *>(p);
}
template <int VEC>
__device__ __forceinline__ void store_vec(float * p, const typename vec_t<VEC>::type & v) {
    *reinterpret_cast<typename vec_t<VEC>::type *>(p) = v;
}

__device__ __forceinline__ float lane_of(const f32x4 & v, int k) { return v[k]; }
__device__ __forceinline__ float lane_of(float v, int) { return v; }
__device__ __forceinline__ void set_lane(f32x4 & v, int k, float x) { v[k] = x; }
__device__ __forceinline__ void set_lane(float & v, int, float x) { v = x; }

// Scalars of one step, computed on the host with the reference's float ops.
struct step_params {
    float * state;
    const float * output;
    int64_t out_pitch, vel_col;
    int32_t cfg;
    float guidance;
    int64_t frames, latent, prefix_frames;
    const float * noise;
    const float * context;
    float dt, time, noise_scale;            // this step (x_t of the prefix rows)
    float next_time, next_noise_scale;      // the next step's prefix rows
    int32_t last;
    float * next_input;
    int64_t in_pitch, state_col;
    int32_t batch;
    const float * mean;
    const float * stddev;
    float * denormalized;
    int32_t * flags;
};

template <int VEC>
__global__ __launch_bounds__(kThreads) void flow_step_kernel(const step_params p) {
    typedef typename vec_t<VEC>::type V;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t n = p.frames * p.latent;
    const int64_t e = i * VEC;
    if (e >= n) return;
    const int64_t f = e / p.latent;
    const int64_t c = e - f * p.latent;
    const bool prefix = f < p.prefix_frames;

    const V u = load_vec<VEC>(p.output + f * p.out_pitch + p.vel_col + c);
    V cnd = u;
    if (p.cfg) cnd = load_vec<VEC>(p.output + (p.frames + f) * p.out_pitch + p.vel_col + c);
    V x = u;
    V nz = u;
    V ctx = u;
    if (prefix) {
        nz = load_vec<VEC>(p.noise + e);
        ctx = load_vec<VEC>(p.context + e);
    } else {
        x = load_vec<VEC>(p.state + e);
    }
    V s, nx;
    bool bad_v = false;
    bool bad_s = false;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const float uk = lane_of(u, k);
        const float v = p.cfg ? uk + p.guidance * (lane_of(cnd, k) - uk) : uk;
        const float xk = prefix ? p.noise_scale * lane_of(nz, k) + p.time * lane_of(ctx, k) : lane_of(x, k);
        const float sk = xk + p.dt * v;
        bad_v |= !__builtin_isfinite(v);
        bad_s |= !__builtin_isfinite(sk);
        set_lane(s, k, p.last && prefix ? lane_of(ctx, k) : sk);
        set_lane(nx, k, prefix ? p.next_noise_scale * lane_of(nz, k) + p.next_time * lane_of(ctx, k) : sk);
    }
    store_vec<VEC>(p.state + e, s);
    if (p.last) {
        if (p.denormalized) {
            const V sd = load_vec<VEC>(p.stddev + c);
            const V mu = load_vec<VEC>(p.mean + c);
            V d;
#pragma unroll
            for (int k = 0; k < VEC; ++k) set_lane(d, k, lane_of(s, k) * lane_of(sd, k) + lane_of(mu, k));
            store_vec<VEC>(p.denormalized + e, d);
        }
    } else if (p.next_input) {
        for (int b = 0; b < p.batch; ++b) {
            store_vec<VEC>(p.next_input + (b * p.frames + f) * p.in_pitch + p.state_col + c, nx);
        }
    }
    if (p.flags) {
        const int32_t fl = (bad_v ? LEVO_HIP_NONFINITE_VELOCITY : 0) | (bad_s ? LEVO_HIP_NONFINITE_STATE : 0);
        if (fl) atomicOr(p.flags, fl);
    }
}

struct input_params {
    float * model_input;
    int32_t batch;
    int32_t uncond_first;  // row 0 of a batch of 2 is unconditional
    int64_t frames, mask_dim, latent, cond_width, hidden;
    const float * mask_embedding;
    const float * context;
    const float * conditioning;
    const float * state;
    const float * noise;
    int64_t prefix_frames;
    float time, noise_scale;
};

// One VEC-wide chunk of one model_input row per thread; a chunk never spans
// two segments (every segment width is a multiple of VEC).
template <int VEC>
__global__ __launch_bounds__(kThreads) void assemble_input_kernel(const input_params p) {
    typedef typename vec_t<VEC>::type V;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    const int64_t chunks = p.hidden / VEC;
    const int64_t row = i / chunks;
    if (row >= p.batch * p.frames) return;
    const int64_t col = (i - row * chunks) * VEC;
    const int64_t b = row / p.frames;
    const int64_t f = row - b * p.frames;
    const int64_t c_ctx = p.mask_dim;
    const int64_t c_cond = c_ctx + p.latent;
    const int64_t c_state = c_cond + p.cond_width;
    V out;
    if (col < c_ctx) {
        out = load_vec<VEC>(p.mask_embedding + f * p.mask_dim + col);
    } else if (col < c_cond) {
        out = load_vec<VEC>(p.context + f * p.latent + (col - c_ctx));
    } else if (col < c_state) {
        if (p.uncond_first && b == 0) {
#pragma unroll
            for (int k = 0; k < VEC; ++k) set_lane(out, k, 0.0f);
        } else {
            out = load_vec<VEC>(p.conditioning + f * p.cond_width + (col - c_cond));
        }
    } else {
        const int64_t e = f * p.latent + (col - c_state);
        if (f < p.prefix_frames) {
            const V nz = load_vec<VEC>(p.noise + e);
            const V ctx = load_vec<VEC>(p.context + e);
#pragma unroll
            for (int k = 0; k < VEC; ++k) {
                set_lane(out, k, p.noise_scale * lane_of(nz, k) + p.time * lane_of(ctx, k));
            }
        } else {
            out = load_vec<VEC>(p.state + e);
        }
    }
    store_vec<VEC>(p.model_input + row * p.hidden + col, out);
}

// normalize_latents / denormalize_latents (src/levo-flow-conditioning.cpp:
// 113-133): out = (x - mean) / stddev or x * stddev + mean per channel, two
// roundings; flags the bit when an input value is not finite.
template <int VEC, bool kNormalize>
__global__ __launch_bounds__(kThreads) void latent_stats_kernel(const float * __restrict__ x,
                                                                const float * __restrict__ mean,
                                                                const float * __restrict__ stddev, float * out,
                                                                int64_t n, int64_t latent, int32_t * flags,
                                                                int32_t bit) {
    typedef typename vec_t<VEC>::type V;
    const int64_t e = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) * VEC;
    if (e >= n) return;
    const int64_t c = e % latent;
    const V xv = load_vec<VEC>(x + e);
    const V mu = load_vec<VEC>(mean + c);
    const V sd = load_vec<VEC>(stddev + c);
    V o;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
        const float xk = lane_of(xv, k);
        bad |= !__builtin_isfinite(xk);
        set_lane(o, k, kNormalize ? (xk - lane_of(mu, k)) / lane_of(sd, k) : xk * lane_of(sd, k) + lane_of(mu, k));
    }
    store_vec<VEC>(out + e, o);
    if (bad && flags) atomicOr(flags, bit);
}

bool aligned(const void * p) { return p == nullptr || aligned16(p); }

template <bool kNormalize>
int launch_latent_stats(const float * x, const float * mean, const float * stddev, float * out, int64_t frames,
                        int64_t latent, int32_t * flags, hipStream_t stream, const char * what) {
    LEVO_REQUIRE(frames > 0 && latent > 0, "%s: dimensions must be positive", what);
    LEVO_REQUIRE(frames < (int64_t{1} << 40) / latent, "%s: tensor too large", what);
    LEVO_REQUIRE(x && mean && stddev && out, "%s: null tensor", what);
    const int64_t n = frames * latent;
    const bool vec = latent % 4 == 0 && aligned(x) && aligned(mean) && aligned(stddev) && aligned(out);
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(n / (vec ? 4 : 1), kThreads));
    if (vec) latent_stats_kernel<4, kNormalize><<<blocks, kThreads, 0, stream>>>(x, mean, stddev, out, n, latent, flags,
                                                                                 LEVO_HIP_NONFINITE_STATE);
    else latent_stats_kernel<1, kNormalize><<<blocks, kThreads, 0, stream>>>(x, mean, stddev, out, n, latent, flags,
                                                                             LEVO_HIP_NONFINITE_STATE);
    return launch_status(what);
}

// The reference's schedule (src/levo-flow-renderer.cpp:89-92) in float.
void schedule(int64_t step, int64_t steps, float sigma_min, float * dt, float * time, float * noise_scale) {
    *dt = 1.0f / static_cast<float>(steps);
    *time = static_cast<float>(step) * *dt;
    *noise_scale = 1.0f - (1.0f - sigma_min) * *time;
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_flow_assemble_input(const levo_hip_flow_input_args * args, levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "flow_assemble_input: null argument block");
    const levo_hip_flow_input_args & a = *args;
    LEVO_REQUIRE(a.batch == 1 || a.batch == 2, "flow_assemble_input: batch must be 1 or 2");
    LEVO_REQUIRE(a.frames > 0 && a.latent > 0 && a.mask_dim >= 0 && a.condition_width >= 0,
                 "flow_assemble_input: dimensions must be positive");
    LEVO_REQUIRE(a.frames < (int64_t{1} << 24) && a.latent < (int64_t{1} << 20) && a.mask_dim < (int64_t{1} << 20) &&
                     a.condition_width < (int64_t{1} << 24),
                 "flow_assemble_input: dimensions too large");
    LEVO_REQUIRE(a.prefix_frames >= 0 && a.prefix_frames <= a.frames,
                 "Euler in-context length exceeds frame count");
    LEVO_REQUIRE(a.steps > 0 && a.step >= 0 && a.step < a.steps, "flow_assemble_input: step out of range");
    LEVO_REQUIRE(__builtin_isfinite(a.sigma_min) && a.sigma_min > 0.0f,
                 "Euler sigma_min must be finite and positive");
    LEVO_REQUIRE(a.model_input && a.context && a.state && (a.mask_dim == 0 || a.mask_embedding) &&
                     (a.condition_width == 0 || a.conditioning) && (a.prefix_frames == 0 || a.noise),
                 "flow_assemble_input: null tensor");
    input_params p;
    p.model_input = a.model_input;
    p.batch = a.batch;
    p.uncond_first = a.batch == 2;
    p.frames = a.frames;
    p.mask_dim = a.mask_dim;
    p.latent = a.latent;
    p.cond_width = a.condition_width;
    p.hidden = a.mask_dim + 2 * a.latent + a.condition_width;
    p.mask_embedding = a.mask_embedding;
    p.context = a.context;
    p.conditioning = a.conditioning;
    p.state = a.state;
    p.noise = a.noise;
    p.prefix_frames = a.prefix_frames;
    float dt;
    schedule(a.step, a.steps, a.sigma_min, &dt, &p.time, &p.noise_scale);
    const bool vec = a.mask_dim % 4 == 0 && a.latent % 4 == 0 && a.condition_width % 4 == 0 &&
                     aligned(a.model_input) && aligned(a.mask_embedding) && aligned(a.context) &&
                     aligned(a.conditioning) && aligned(a.state) && aligned(a.noise);
    const int64_t threads = a.batch * a.frames * (p.hidden / (vec ? 4 : 1));
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(threads, kThreads));
    if (vec) assemble_input_kernel<4><<<blocks, kThreads, 0, as_hip(stream)>>>(p);
    else assemble_input_kernel<1><<<blocks, kThreads, 0, as_hip(stream)>>>(p);
    return launch_status("levo_hip_flow_assemble_input");
}

extern "C" int levo_hip_flow_step(const levo_hip_flow_step_args * args, levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "flow_step: null argument block");
    const levo_hip_flow_step_args & a = *args;
    LEVO_REQUIRE(a.batch == 1 || a.batch == 2, "flow_step: batch must be 1 or 2");
    LEVO_REQUIRE(a.frames > 0 && a.latent > 0, "flow_step: dimensions must be positive");
    LEVO_REQUIRE(a.frames < (int64_t{1} << 24) && a.latent < (int64_t{1} << 20), "flow_step: dimensions too large");
    LEVO_REQUIRE(a.vel_col >= 0 && a.out_pitch >= a.vel_col + a.latent,
                 "flow_step: velocity columns exceed the output row");
    LEVO_REQUIRE(a.next_input == nullptr || (a.state_col >= 0 && a.in_pitch >= a.state_col + a.latent),
                 "flow_step: state columns exceed the input row");
    LEVO_REQUIRE(a.out_pitch < (int64_t{1} << 24) && a.in_pitch < (int64_t{1} << 24), "flow_step: row pitch too large");
    LEVO_REQUIRE(a.prefix_frames >= 0 && a.prefix_frames <= a.frames, "Euler in-context length exceeds frame count");
    LEVO_REQUIRE(a.steps > 0 && a.step >= 0 && a.step < a.steps, "flow_step: step out of range");
    LEVO_REQUIRE(__builtin_isfinite(a.sigma_min) && a.sigma_min > 0.0f,
                 "Euler sigma_min must be finite and positive");
    LEVO_REQUIRE(a.state && a.output && a.context && (a.prefix_frames == 0 || a.noise), "flow_step: null tensor");
    LEVO_REQUIRE(a.denormalized == nullptr || (a.mean && a.stddev), "flow_step: denormalization needs mean and stddev");
    step_params p;
    p.state = a.state;
    p.output = a.output;
    p.out_pitch = a.out_pitch;
    p.vel_col = a.vel_col;
    p.cfg = a.batch == 2;
    p.guidance = a.guidance;
    p.frames = a.frames;
    p.latent = a.latent;
    p.prefix_frames = a.prefix_frames;
    p.noise = a.noise;
    p.context = a.context;
    schedule(a.step, a.steps, a.sigma_min, &p.dt, &p.time, &p.noise_scale);
    float next_dt;
    schedule(a.step + 1, a.steps, a.sigma_min, &next_dt, &p.next_time, &p.next_noise_scale);
    p.last = a.step + 1 == a.steps;
    p.next_input = a.next_input;
    p.in_pitch = a.in_pitch;
    p.state_col = a.state_col;
    p.batch = a.batch;
    p.mean = a.mean;
    p.stddev = a.stddev;
    p.denormalized = a.denormalized;
    p.flags = a.nonfinite;
    const bool vec = a.latent % 4 == 0 && a.out_pitch % 4 == 0 && a.vel_col % 4 == 0 &&
                     (a.next_input == nullptr || (a.in_pitch % 4 == 0 && a.state_col % 4 == 0)) &&
                     aligned(a.state) && aligned(a.output) && aligned(a.noise) && aligned(a.context) &&
                     aligned(a.next_input) && aligned(a.mean) && aligned(a.stddev) && aligned(a.denormalized);
    const int64_t threads = a.frames * a.latent / (vec ? 4 : 1);
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(threads, kThreads));
    if (vec) flow_step_kernel<4><<<blocks, kThreads, 0, as_hip(stream)>>>(p);
    else flow_step_kernel<1><<<blocks, kThreads, 0, as_hip(stream)>>>(p);
    return launch_status("levo_hip_flow_step");
}

extern "C" int levo_hip_flow_normalize(const float * raw, const float * mean, const float * stddev, float * normalized,
                                       int64_t frames, int64_t latent, int32_t * nonfinite,
                                       levo_hip_stream_t stream) {
    return launch_latent_stats<true>(raw, mean, stddev, normalized, frames, latent, nonfinite, as_hip(stream),
                                     "levo_hip_flow_normalize");
}

extern "C" int levo_hip_flow_denormalize(const float * normalized, const float * mean, const float * stddev,
                                         float * raw, int64_t frames, int64_t latent, int32_t * nonfinite,
                                         levo_hip_stream_t stream) {
    return launch_latent_stats<false>(normalized, mean, stddev, raw, frames, latent, nonfinite, as_hip(stream),
                                      "levo_hip_flow_denormalize");
}
