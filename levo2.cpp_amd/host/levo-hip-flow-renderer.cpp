// Euler solver of src/levo-flow-renderer.cpp:57-120 with the state on the GPU:
// levo_hip_flow_incontext for the prefix interpolation, levo_hip_check_finite
// for the entry checks and levo_hip_flow_cfg_euler_checked for the update and
// its per-step finiteness checks; for a whole window with the estimator's
// tensors in HBM, levo_hip_flow_assemble_input once and levo_hip_flow_step
// after every estimator call.
#include "levo-hip-flow-renderer.h"

#include <cmath>
#include <cstring>
#include <limits>
#include <string>

namespace levo::hip::flow {
namespace {

[[noreturn]] void fail(const std::string & message) {
    throw std::runtime_error("LeVo Flow renderer: " + message);
}

std::size_t element_count(std::size_t frames, std::size_t width) {
    if (frames == 0 || width == 0) fail("Euler state dimensions must be positive");
    if (width > std::numeric_limits<std::size_t>::max() / frames) fail("Euler state size overflow");
    const std::size_t n = frames * width;
    if (n > static_cast<std::size_t>(std::numeric_limits<int64_t>::max() / 4)) fail("Euler state size overflow");
    return n;
}

void validate_common(std::size_t steps, bool has_velocity) {
    if (steps == 0) fail("Euler step count must be positive");
    if (!has_velocity) fail("Euler velocity callback is required");
}

void validate_prefix(std::size_t frames, std::size_t incontext_frames, float sigma_min) {
    if (incontext_frames > frames) fail("Euler in-context length exceeds frame count");
    if (!std::isfinite(sigma_min) || sigma_min <= 0.0F) fail("Euler sigma_min must be finite and positive");
}

// Per-solve device state: the flag word and its pinned host mirror.
class flag_word {
public:
    flag_word() : device_(1), host_(1) {}
    void clear(stream_t stream) {
        check_hip(hipMemsetAsync(device_.data(), 0, sizeof(int32_t), stream), "flag clear");
    }
    int32_t * device() { return device_.data(); }
    int32_t read(stream_t stream) {
        device_.download(host_.data(), 1, stream);
        synchronize(stream);
        return host_[0];
    }

private:
    device_buffer<int32_t> device_;
    pinned_buffer<int32_t> host_;
};

constexpr int32_t kNoiseBit = 1;
constexpr int32_t kContextBit = 2;
constexpr int32_t kResumeBit = 4;

// Entry checks of the reference, in its order (src/levo-flow-renderer.cpp:70-80).
void check_inputs_finite(flag_word & flags, const float * noise, const float * context, std::size_t n,
                         stream_t stream) {
    flags.clear(stream);
    const auto count = static_cast<int64_t>(n);
    check_status(levo_hip_check_finite(noise, count, flags.device(), kNoiseBit, stream), error_kind::runtime_error);
    check_status(levo_hip_check_finite(context, count, flags.device(), kContextBit, stream), error_kind::runtime_error);
    const int32_t f = flags.read(stream);
    if (f & kNoiseBit) fail("Euler noise contains a non-finite value");
    if (f & kContextBit) fail("Euler in-context latent contains a non-finite value");
}

// A resume state uploaded to `state` must be finite (:80).
void check_resume_finite(flag_word & flags, const float * state, std::size_t n, stream_t stream) {
    flags.clear(stream);
    check_status(levo_hip_check_finite(state, static_cast<int64_t>(n), flags.device(), kResumeBit, stream),
                 error_kind::runtime_error);
    if (flags.read(stream) & kResumeBit) fail("Euler resume state contains a non-finite value");
}

// One Euler update with the reference's post-update checks (:104-106).
void update(flag_word & flags, float * state, const float * v_uncond, const float * v_cond, std::size_t n,
            float guidance, float dt, stream_t stream) {
    flags.clear(stream);
    check_status(levo_hip_flow_cfg_euler_checked(state, v_uncond, v_cond, static_cast<int64_t>(n), guidance, dt,
                                                 flags.device(), stream),
                 error_kind::runtime_error);
    const int32_t f = flags.read(stream);
    if (f & LEVO_HIP_NONFINITE_VELOCITY) fail("Euler velocity contains a non-finite value");
    if (f & LEVO_HIP_NONFINITE_STATE) fail("Euler state contains a non-finite value");
}

void interpolate_prefix(float * state, const float * noise, const float * context, std::size_t prefix, float time,
                        float sigma_min, stream_t stream) {
    check_status(levo_hip_flow_incontext(state, noise, context, static_cast<int64_t>(prefix), time, sigma_min,
                                         stream),
                 error_kind::runtime_error);
}

void save(euler_resume_state * checkpoint, std::size_t completed, const float * state, std::size_t n,
          stream_t stream) {
    if (!checkpoint) return;
    checkpoint->normalized_state.resize(n);
    check_hip(hipMemcpyAsync(checkpoint->normalized_state.data(), state, n * sizeof(float), hipMemcpyDeviceToHost,
                             stream),
              "device-to-host copy");
    synchronize(stream);
    checkpoint->completed_steps = completed;
}

// The steps [first, steps) of a solve without checkpoints, with one
// synchronization per step. After step s's update the next step's prefix
// interpolation and the copy of its state to pinned memory are queued behind
// it, with the copy of s's finiteness flags; the synchronization at the top
// of step s + 1 then covers all of them, and the host checks s's flags, calls
// progress and the cancellation poll in the reference's order before it
// hands the state to the velocity callback. A cancellation or a non-finite
// step throws before any further callback, as in the reference; the queued
// work only touches this solve's own buffers.
void pipelined_steps(const euler_input & input, std::size_t steps, std::size_t first, float dt,
                     const velocity_callback & velocity, const euler_progress_callback & progress,
                     const cancellation_callback & cancelled, device_buffer<float> & state,
                     const device_buffer<float> & noise, const device_buffer<float> & context,
                     device_buffer<float> & vel, std::vector<float> & host_state, stream_t stream) {
    const std::size_t n = host_state.size();
    const std::size_t prefix = input.incontext_frames * input.latent_dim;
    pinned_buffer<float> stage(n), vstage(n);
    device_buffer<int32_t> dflags(2);  // the finiteness flags of even and odd steps
    pinned_buffer<int32_t> hflags(2);
    const auto queue_state = [&](std::size_t step) {
        const float time = static_cast<float>(step) * dt;
        interpolate_prefix(state.data(), noise.data(), context.data(), prefix, time, input.sigma_min, stream);
        check_hip(hipMemcpyAsync(stage.data(), state.data(), n * sizeof(float), hipMemcpyDeviceToHost, stream),
                  "device-to-host copy");
    };
    const auto check_step = [&](std::size_t step) {
        const int32_t f = hflags[step & 1];
        if (f & LEVO_HIP_NONFINITE_VELOCITY) fail("Euler velocity contains a non-finite value");
        if (f & LEVO_HIP_NONFINITE_STATE) fail("Euler state contains a non-finite value");
        if (progress) progress(step + 1U, steps);
    };
    queue_state(first);
    for (std::size_t step = first; step < steps; ++step) {
        synchronize(stream);
        if (step > first) check_step(step - 1);
        if (cancelled && cancelled()) throw operation_cancelled();
        const float time = static_cast<float>(step) * dt;
        std::memcpy(host_state.data(), stage.data(), n * sizeof(float));
        const std::vector<float> current_velocity = velocity(host_state, time);
        if (current_velocity.size() != n) fail("Euler velocity callback returned an unexpected shape");
        std::memcpy(vstage.data(), current_velocity.data(), n * sizeof(float));
        vel.upload(vstage.data(), n, stream);
        int32_t * flag = dflags.data() + (step & 1);
        check_hip(hipMemsetAsync(flag, 0, sizeof(int32_t), stream), "flag clear");
        check_status(levo_hip_flow_cfg_euler_checked(state.data(), vel.data(), nullptr, static_cast<int64_t>(n), 1.0F,
                                                     dt, flag, stream),
                     error_kind::runtime_error);
        check_hip(hipMemcpyAsync(hflags.data() + (step & 1), flag, sizeof(int32_t), hipMemcpyDeviceToHost, stream),
                  "device-to-host copy");
        if (step + 1 < steps) queue_state(step + 1);
    }
    synchronize(stream);
    check_step(steps - 1);
}

} // namespace

std::vector<float> solve_flow_euler(const euler_input & input, std::size_t steps, const velocity_callback & velocity,
                                    const euler_progress_callback & progress, const cancellation_callback & cancelled,
                                    const euler_resume_state * resume, euler_resume_state * checkpoint) {
    validate_common(steps, static_cast<bool>(velocity));
    const std::size_t n = element_count(input.frames, input.latent_dim);
    if (input.initial_noise.size() != n || input.normalized_incontext.size() != n) {
        fail("Euler tensors must have shape [frames, latent_dim]");
    }
    validate_prefix(input.frames, input.incontext_frames, input.sigma_min);

    const stream_t stream = nullptr;
    device_buffer<float> noise(n), context(n), state(n), vel(n);
    noise.upload(input.initial_noise.data(), n, stream);
    context.upload(input.normalized_incontext.data(), n, stream);
    flag_word flags;
    check_inputs_finite(flags, noise.data(), context.data(), n, stream);

    std::size_t completed_steps = 0;
    std::vector<float> host_state = input.initial_noise;
    if (resume) {
        if (resume->completed_steps > steps) fail("Euler resume step exceeds total steps");
        if (resume->normalized_state.size() != n) fail("Euler resume state has an unexpected shape");
        state.upload(resume->normalized_state.data(), n, stream);
        check_resume_finite(flags, state.data(), n, stream);
        completed_steps = resume->completed_steps;
        host_state = resume->normalized_state;
    } else {
        state.upload(input.initial_noise.data(), n, stream);
    }
    if (checkpoint) {
        checkpoint->completed_steps = completed_steps;
        checkpoint->normalized_state = host_state;
    }

    const std::size_t prefix = input.incontext_frames * input.latent_dim;
    const float dt = 1.0F / static_cast<float>(steps);
    if (!checkpoint && completed_steps < steps) {
        pipelined_steps(input, steps, completed_steps, dt, velocity, progress, cancelled, state, noise, context, vel,
                        host_state, stream);
        completed_steps = steps;
    }
    for (std::size_t step = completed_steps; step < steps; ++step) {
        if (cancelled && cancelled()) throw operation_cancelled();
        const float time = static_cast<float>(step) * dt;
        interpolate_prefix(state.data(), noise.data(), context.data(), prefix, time, input.sigma_min, stream);
        state.download(host_state.data(), n, stream);
        synchronize(stream);
        const std::vector<float> current_velocity = velocity(host_state, time);
        if (current_velocity.size() != n) fail("Euler velocity callback returned an unexpected shape");
        vel.upload(current_velocity.data(), n, stream);
        update(flags, state.data(), vel.data(), nullptr, n, 1.0F, dt, stream);
        save(checkpoint, step + 1U, state.data(), n, stream);
        if (progress) progress(step + 1U, steps);
    }
    check_hip(hipMemcpyAsync(state.data(), context.data(), prefix * sizeof(float), hipMemcpyDeviceToDevice, stream),
              "device-to-device copy");
    state.download(host_state.data(), n, stream);
    synchronize(stream);
    if (checkpoint) {
        checkpoint->completed_steps = steps;
        checkpoint->normalized_state = host_state;
    }
    return host_state;
}

void solve_flow_euler_device(const device_euler_input & input, std::size_t steps, float guidance_scale,
                             const device_velocity_callback & velocity, float * state,
                             const euler_progress_callback & progress, const cancellation_callback & cancelled,
                             const euler_resume_state * resume, euler_resume_state * checkpoint, stream_t stream) {
    validate_common(steps, static_cast<bool>(velocity));
    const std::size_t n = element_count(input.frames, input.latent_dim);
    if (!input.initial_noise || !input.normalized_incontext || !state) {
        fail("Euler tensors must have shape [frames, latent_dim]");
    }
    validate_prefix(input.frames, input.incontext_frames, input.sigma_min);

    flag_word flags;
    check_inputs_finite(flags, input.initial_noise, input.normalized_incontext, n, stream);

    std::size_t completed_steps = 0;
    if (resume) {
        if (resume->completed_steps > steps) fail("Euler resume step exceeds total steps");
        if (resume->normalized_state.size() != n) fail("Euler resume state has an unexpected shape");
        check_hip(hipMemcpyAsync(state, resume->normalized_state.data(), n * sizeof(float), hipMemcpyHostToDevice,
                                 stream),
                  "host-to-device copy");
        check_resume_finite(flags, state, n, stream);
        completed_steps = resume->completed_steps;
    } else {
        check_hip(hipMemcpyAsync(state, input.initial_noise, n * sizeof(float), hipMemcpyDeviceToDevice, stream),
                  "device-to-device copy");
    }
    save(checkpoint, completed_steps, state, n, stream);

    device_buffer<float> vel(2 * n);
    float * v_uncond = vel.data();
    float * v_cond = vel.data() + n;
    const std::size_t prefix = input.incontext_frames * input.latent_dim;
    const float dt = 1.0F / static_cast<float>(steps);
    for (std::size_t step = completed_steps; step < steps; ++step) {
        if (cancelled && cancelled()) throw operation_cancelled();
        const float time = static_cast<float>(step) * dt;
        interpolate_prefix(state, input.initial_noise, input.normalized_incontext, prefix, time, input.sigma_min,
                           stream);
        velocity(state, time, v_uncond, v_cond, stream);
        update(flags, state, v_uncond, v_cond, n, guidance_scale, dt, stream);
        save(checkpoint, step + 1U, state, n, stream);
        if (progress) progress(step + 1U, steps);
    }
    check_hip(hipMemcpyAsync(state, input.normalized_incontext, prefix * sizeof(float), hipMemcpyDeviceToDevice,
                             stream),
              "device-to-device copy");
    save(checkpoint, steps, state, n, stream);
    synchronize(stream);
}

void solve_flow_window_device(const device_euler_input & input, const device_window_conditioning & conditioning,
                              std::size_t steps, float guidance_scale, const device_estimator_tensors & estimator_io,
                              const device_estimator_callback & estimator, float * state, float * denormalized,
                              const euler_progress_callback & progress, const cancellation_callback & cancelled,
                              const euler_resume_state * resume, euler_resume_state * checkpoint, stream_t stream) {
    validate_common(steps, static_cast<bool>(estimator));
    const std::size_t n = element_count(input.frames, input.latent_dim);
    if (!input.initial_noise || !input.normalized_incontext || !state) {
        fail("Euler tensors must have shape [frames, latent_dim]");
    }
    validate_prefix(input.frames, input.incontext_frames, input.sigma_min);
    if (!estimator_io.model_input || !estimator_io.output) fail("estimator tensors are required");
    if (estimator_io.hidden != conditioning.mask_dim + 2 * input.latent_dim + conditioning.condition_width) {
        fail("estimator rows must hold mask embedding, in-context latent, conditioning and state");
    }
    if ((conditioning.mask_dim && !conditioning.mask_embedding) ||
        (conditioning.condition_width && !conditioning.conditioning)) {
        fail("conditioning tensors are required");
    }
    if (denormalized && (!conditioning.latent_mean || !conditioning.latent_stddev)) {
        fail("denormalization needs the latent mean and standard deviation");
    }
    if (steps > static_cast<std::size_t>(std::numeric_limits<int64_t>::max())) fail("Euler step count is too large");

    flag_word flags;
    check_inputs_finite(flags, input.initial_noise, input.normalized_incontext, n, stream);

    std::size_t completed_steps = 0;
    if (resume) {
        if (resume->completed_steps > steps) fail("Euler resume step exceeds total steps");
        if (resume->normalized_state.size() != n) fail("Euler resume state has an unexpected shape");
        check_hip(hipMemcpyAsync(state, resume->normalized_state.data(), n * sizeof(float), hipMemcpyHostToDevice,
                                 stream),
                  "host-to-device copy");
        check_resume_finite(flags, state, n, stream);
        completed_steps = resume->completed_steps;
    } else {
        check_hip(hipMemcpyAsync(state, input.initial_noise, n * sizeof(float), hipMemcpyDeviceToDevice, stream),
                  "device-to-device copy");
    }
    save(checkpoint, completed_steps, state, n, stream);

    const int32_t batch = guidance_scale > 1.0F ? 2 : 1;
    const auto frames = static_cast<int64_t>(input.frames);
    const auto latent = static_cast<int64_t>(input.latent_dim);
    const auto hidden = static_cast<int64_t>(estimator_io.hidden);
    const std::size_t prefix = input.incontext_frames * input.latent_dim;
    if (completed_steps == steps) {
        // Nothing left to integrate: restore the prefix and denormalize.
        check_hip(hipMemcpyAsync(state, input.normalized_incontext, prefix * sizeof(float), hipMemcpyDeviceToDevice,
                                 stream),
                  "device-to-device copy");
        save(checkpoint, steps, state, n, stream);
        if (denormalized) {
            flags.clear(stream);
            check_status(levo_hip_flow_denormalize(state, conditioning.latent_mean, conditioning.latent_stddev,
                                                   denormalized, frames, latent, flags.device(), stream),
                         error_kind::runtime_error);
            if (flags.read(stream)) {
                throw std::runtime_error("LeVo Flow conditioning: normalized latent contains a non-finite value");
            }
        }
        synchronize(stream);
        return;
    }

    levo_hip_flow_input_args in{};
    in.model_input = estimator_io.model_input;
    in.batch = batch;
    in.frames = frames;
    in.mask_embedding = conditioning.mask_embedding;
    in.mask_dim = static_cast<int64_t>(conditioning.mask_dim);
    in.context = input.normalized_incontext;
    in.latent = latent;
    in.conditioning = conditioning.conditioning;
    in.condition_width = static_cast<int64_t>(conditioning.condition_width);
    in.state = state;
    in.noise = input.initial_noise;
    in.prefix_frames = static_cast<int64_t>(input.incontext_frames);
    in.step = static_cast<int64_t>(completed_steps);
    in.steps = static_cast<int64_t>(steps);
    in.sigma_min = input.sigma_min;
    check_status(levo_hip_flow_assemble_input(&in, stream), error_kind::runtime_error);

    levo_hip_flow_step_args st{};
    st.state = state;
    st.output = estimator_io.output;
    st.out_pitch = hidden;
    st.vel_col = hidden - latent;
    st.batch = batch;
    st.guidance = guidance_scale;
    st.frames = frames;
    st.latent = latent;
    st.steps = static_cast<int64_t>(steps);
    st.noise = input.initial_noise;
    st.context = input.normalized_incontext;
    st.prefix_frames = static_cast<int64_t>(input.incontext_frames);
    st.sigma_min = input.sigma_min;
    st.next_input = estimator_io.model_input;
    st.in_pitch = hidden;
    st.state_col = hidden - latent;
    st.mean = conditioning.latent_mean;
    st.stddev = conditioning.latent_stddev;
    st.denormalized = denormalized;
    const float dt = 1.0F / static_cast<float>(steps);
    for (std::size_t step = completed_steps; step < steps; ++step) {
        if (cancelled && cancelled()) throw operation_cancelled();
        const float time = static_cast<float>(step) * dt;
        estimator(time, stream);
        flags.clear(stream);
        st.step = static_cast<int64_t>(step);
        st.nonfinite = flags.device();
        check_status(levo_hip_flow_step(&st, stream), error_kind::runtime_error);
        const int32_t f = flags.read(stream);
        if (f & LEVO_HIP_NONFINITE_VELOCITY) fail("Euler velocity contains a non-finite value");
        if (f & LEVO_HIP_NONFINITE_STATE) fail("Euler state contains a non-finite value");
        save(checkpoint, step + 1U, state, n, stream);
        if (progress) progress(step + 1U, steps);
    }
    synchronize(stream);
}

} // namespace levo::hip::flow
