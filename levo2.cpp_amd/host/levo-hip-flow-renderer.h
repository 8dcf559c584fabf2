// Drop-in for the Flow renderer's Euler solver, src/levo-flow-renderer.h:13-51,
// with the state resident on the GPU.
//
// solve_flow_euler keeps the reference signature, callbacks, checkpoint /
// resume semantics and exceptions (std::runtime_error("LeVo Flow renderer:
// ...") and operation_cancelled). Its velocity callback still exchanges host
// vectors, as the reference's does; solve_flow_euler_device is the MI355X
// path, where the estimator writes both CFG velocity branches into device
// memory and one fused kernel applies u + g * (c - u) and the Euler update.
#pragma once

#include "levo-hip-device.h"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <stdexcept>
#include <vector>

namespace levo::hip {

// Thrown when the cancellation callback returns true (include/levo.h:21-26).
class operation_cancelled : public std::runtime_error {
public:
    operation_cancelled() : std::runtime_error("LeVo operation cancelled") {}
};

using cancellation_callback = std::function<bool()>;

namespace flow {

// Same fields as levo::flow::euler_input: C-order [frames, latent_dim] state.
struct euler_input {
    std::vector<float> initial_noise;
    std::vector<float> normalized_incontext;
    std::size_t frames = 0;
    std::size_t latent_dim = 0;
    std::size_t incontext_frames = 0;
    float sigma_min = 1.0e-4F;
};

using velocity_callback = std::function<std::vector<float>(
        const std::vector<float> & state, float timestep)>;
using euler_progress_callback = std::function<void(
        std::size_t completed_steps, std::size_t total_steps)>;

// Post-update state after `completed_steps` (host copy, serializable).
struct euler_resume_state {
    std::size_t completed_steps = 0;
    std::vector<float> normalized_state;
};

// Fixed-step Euler with in-context interpolation and final context restore;
// same contract as levo::flow::solve_flow_euler.
[[nodiscard]] std::vector<float> solve_flow_euler(
        const euler_input & input,
        std::size_t steps,
        const velocity_callback & velocity,
        const euler_progress_callback & progress = {},
        const cancellation_callback & cancelled = {},
        const euler_resume_state * resume = nullptr,
        euler_resume_state * checkpoint = nullptr);

// Device-resident input: both tensors are device pointers to
// [frames * latent_dim] floats.
struct device_euler_input {
    const float * initial_noise = nullptr;
    const float * normalized_incontext = nullptr;
    std::size_t frames = 0;
    std::size_t latent_dim = 0;
    std::size_t incontext_frames = 0;
    float sigma_min = 1.0e-4F;
};

// Writes the unconditional and conditional velocities for `state` at
// `timestep` into the device buffers v_uncond / v_cond (each frames *
// latent_dim floats), enqueued on `stream`.
using device_velocity_callback = std::function<void(
        const float * state, float timestep, float * v_uncond, float * v_cond, stream_t stream)>;

// solve_flow_euler with every tensor in device memory: `state` (device,
// frames * latent_dim floats) receives the solution. Each step runs the
// in-context interpolation kernel, the callback, and one fused
// state += dt * (u + guidance * (c - u)) kernel that also flags non-finite
// velocities / states, raising the reference's errors at the same step.
// A checkpoint, when given, receives a host copy of the state after every
// step (one device-to-host copy per step).
void solve_flow_euler_device(
        const device_euler_input & input,
        std::size_t steps,
        float guidance_scale,
        const device_velocity_callback & velocity,
        float * state,
        const euler_progress_callback & progress = {},
        const cancellation_callback & cancelled = {},
        const euler_resume_state * resume = nullptr,
        euler_resume_state * checkpoint = nullptr,
        stream_t stream = nullptr);

} // namespace flow
} // namespace levo::hip
