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

// ---- One Flow window with the estimator's tensors in HBM ---------------------

// The estimator's input and output as estimator::velocity lays them out
// (src/levo-flow-estimator.cpp:343-399), in device memory:
// model_input [batch][frames][hidden] with rows
//   mask_embedding | normalized_incontext | conditioning (zeros in the
//   unconditional row) | state       (append_model_row, src/levo-flow-renderer.cpp:35-53)
// and output [batch][frames][hidden] whose last latent_dim columns are the
// velocity. batch is 2 (row 0 unconditional, row 1 conditional) when
// guidance_scale > 1, else 1, as the renderer decides (:283-285).
struct device_estimator_tensors {
    float * model_input = nullptr;
    const float * output = nullptr;
    std::size_t hidden = 0;
};

// The window's conditioning_output in device memory
// (src/levo-flow-conditioning.h): the parts of the estimator rows that stay
// fixed over the steps, and the latent statistics for denormalize_latents.
struct device_window_conditioning {
    const float * mask_embedding = nullptr;  // [frames][mask_dim]
    std::size_t mask_dim = 0;
    const float * conditioning = nullptr;    // [frames][condition_width] (2 * condition_dim)
    std::size_t condition_width = 0;
    const float * latent_mean = nullptr;     // [latent_dim]; with latent_stddev, or both null
    const float * latent_stddev = nullptr;
};

// Runs the estimator graph for `timestep` (every batch row) on `stream`:
// reads model_input, writes output.
using device_estimator_callback = std::function<void(float timestep, stream_t stream)>;

// solve_flow_euler for one window as the renderer drives it
// (src/levo-flow-renderer.cpp:283-331): the estimator input rows are built
// once (levo_hip_flow_assemble_input), and after every estimator call one
// levo_hip_flow_step launch reads the velocity slice, applies the CFG lambda,
// the prefix interpolation and the Euler update with the reference's
// finiteness checks, and writes the next step's state columns. After the
// last step the prefix is restored and, when the statistics are given,
// `denormalized` receives denormalize_latents (state * stddev + mean).
// Per step only the 4-byte flag word comes back to the host. `state` (device,
// frames * latent_dim floats) holds the reference's state after every step,
// so a checkpoint or a resume matches bit for bit. Errors, progress,
// cancellation, resume and checkpoint behave as in solve_flow_euler.
void solve_flow_window_device(
        const device_euler_input & input,
        const device_window_conditioning & conditioning,
        std::size_t steps,
        float guidance_scale,
        const device_estimator_tensors & estimator_io,
        const device_estimator_callback & estimator,
        float * state,
        float * denormalized = nullptr,
        const euler_progress_callback & progress = {},
        const cancellation_callback & cancelled = {},
        const euler_resume_state * resume = nullptr,
        euler_resume_state * checkpoint = nullptr,
        stream_t stream = nullptr);

} // namespace flow
} // namespace levo::hip
