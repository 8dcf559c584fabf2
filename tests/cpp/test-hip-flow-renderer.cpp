// levo::hip::flow drop-in: the reference's tests/test-flow-renderer.cpp:33-127
// (KAT, pause/resume bit-exactness, invalid resumes, cancellation) restated
// against levo::hip::flow, the error messages of src/levo-flow-renderer.cpp,
// and seeded parity of both solvers with the oracle's Euler restatement at the
// renderer's per-window shape, and the window solver that leaves the
// estimator's tensors in device memory.
#include "check.h"
#include "levo-hip-flow-renderer.h"
#include "levo_oracle.h"

#include <cmath>
#include <iostream>
#include <limits>
#include <vector>

using namespace levo::hip::flow;
using levo::hip::device_buffer;
using levo::hip::stream_t;

namespace {

bool close(float lhs, float rhs) { return std::fabs(lhs - rhs) < 1.0e-6F; }

std::vector<float> ones_like(const std::vector<float> & s) { return std::vector<float>(s.size(), 1.0F); }

euler_input kat_input() {
    euler_input input;
    input.frames = 3;
    input.latent_dim = 2;
    input.incontext_frames = 1;
    input.sigma_min = 0.1F;
    input.initial_noise = {1.0F, 2.0F, 10.0F, 20.0F, 30.0F, 40.0F};
    input.normalized_incontext = {4.0F, 8.0F, 0.0F, 0.0F, 0.0F, 0.0F};
    return input;
}

void reference_assertions() {
    const euler_input input = kat_input();
    std::vector<float> times;
    std::vector<std::size_t> completed_steps;
    const std::vector<float> solved = solve_flow_euler(
            input, 2,
            [&times](const std::vector<float> & state, float time) {
                times.push_back(time);
                if (times.size() == 1) {
                    CHECK(close(state[0], 1.0F) && close(state[1], 2.0F));
                } else {
                    CHECK(close(state[0], 2.55F) && close(state[1], 5.10F));
                }
                return ones_like(state);
            },
            [&completed_steps](std::size_t completed, std::size_t total) {
                CHECK(total == 2);
                completed_steps.push_back(completed);
            });
    CHECK(times.size() == 2 && close(times[0], 0.0F) && close(times[1], 0.5F));
    CHECK((completed_steps == std::vector<std::size_t>{1, 2}));
    CHECK(close(solved[0], 4.0F) && close(solved[1], 8.0F));
    CHECK(close(solved[2], 11.0F) && close(solved[3], 21.0F));
    CHECK(close(solved[4], 31.0F) && close(solved[5], 41.0F));

    for (std::size_t pause_at = 0; pause_at < 2; ++pause_at) {
        euler_resume_state checkpoint;
        std::size_t polls = 0;
        bool paused = false;
        try {
            (void) solve_flow_euler(
                    input, 2, [](const std::vector<float> & state, float) { return ones_like(state); }, {},
                    [&polls, pause_at] { return polls++ >= pause_at; }, nullptr, &checkpoint);
        } catch (const levo::hip::operation_cancelled &) {
            paused = true;
        }
        CHECK(paused && checkpoint.completed_steps == pause_at);
        const std::vector<float> resumed = solve_flow_euler(
                input, 2, [](const std::vector<float> & state, float) { return ones_like(state); }, {}, {},
                &checkpoint);
        CHECK(resumed == solved);
    }

    euler_resume_state invalid{3, std::vector<float>(input.initial_noise.size(), 0.0F)};
    const auto ones = [](const std::vector<float> & state, float) { return ones_like(state); };
    expect_throw<std::runtime_error>("Euler resume step exceeds total steps",
                                     [&] { (void) solve_flow_euler(input, 2, ones, {}, {}, &invalid); });
    invalid = euler_resume_state{1, {}};
    expect_throw<std::runtime_error>("Euler resume state has an unexpected shape",
                                     [&] { (void) solve_flow_euler(input, 2, ones, {}, {}, &invalid); });
    expect_throw<std::runtime_error>("Euler step count must be positive", [&] {
        (void) solve_flow_euler(input, 0, [](const auto &, float) { return std::vector<float>{}; });
    });

    std::size_t cancel_polls = 0;
    std::size_t velocity_calls = 0;
    bool cancelled = false;
    try {
        (void) solve_flow_euler(
                input, 2,
                [&velocity_calls](const std::vector<float> & state, float) {
                    ++velocity_calls;
                    return ones_like(state);
                },
                {}, [&cancel_polls] { return cancel_polls++ != 0; });
    } catch (const levo::hip::operation_cancelled &) {
        cancelled = true;
    }
    CHECK(cancelled && velocity_calls == 1 && cancel_polls == 2);
}

void error_behaviour() {
    const auto ones = [](const std::vector<float> & state, float) { return ones_like(state); };
    euler_input input = kat_input();
    expect_throw<std::runtime_error>("Euler velocity callback is required",
                                     [&] { (void) solve_flow_euler(input, 2, velocity_callback{}); });
    input.frames = 0;
    expect_throw<std::runtime_error>("Euler state dimensions must be positive",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    input.initial_noise.pop_back();
    expect_throw<std::runtime_error>("Euler tensors must have shape [frames, latent_dim]",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    input.incontext_frames = 4;
    expect_throw<std::runtime_error>("Euler in-context length exceeds frame count",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    input.sigma_min = 0.0F;
    expect_throw<std::runtime_error>("Euler sigma_min must be finite and positive",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    input.initial_noise[5] = std::numeric_limits<float>::infinity();
    expect_throw<std::runtime_error>("Euler noise contains a non-finite value",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    input.normalized_incontext[1] = std::nanf("");
    expect_throw<std::runtime_error>("Euler in-context latent contains a non-finite value",
                                     [&] { (void) solve_flow_euler(input, 2, ones); });
    input = kat_input();
    euler_resume_state bad_resume{1, std::vector<float>(6, 0.0F)};
    bad_resume.normalized_state[3] = std::nanf("");
    expect_throw<std::runtime_error>("Euler resume state contains a non-finite value",
                                     [&] { (void) solve_flow_euler(input, 2, ones, {}, {}, &bad_resume); });
    expect_throw<std::runtime_error>("Euler velocity callback returned an unexpected shape", [&] {
        (void) solve_flow_euler(input, 2, [](const auto &, float) { return std::vector<float>(5, 1.0F); });
    });
    // A non-finite velocity at step 1 throws there; the checkpoint keeps step 1.
    euler_resume_state checkpoint;
    expect_throw<std::runtime_error>("Euler velocity contains a non-finite value", [&] {
        (void) solve_flow_euler(
                input, 3,
                [](const std::vector<float> & state, float t) {
                    std::vector<float> v(state.size(), 1.0F);
                    if (t > 0.3F) v[4] = std::nanf("");
                    return v;
                },
                {}, {}, nullptr, &checkpoint);
    });
    CHECK(checkpoint.completed_steps == 1);
    // A finite velocity that overflows a large (finite) resumed state.
    euler_resume_state large{1, std::vector<float>(6, 3.0e38F)};
    expect_throw<std::runtime_error>("Euler state contains a non-finite value", [&] {
        (void) solve_flow_euler(
                input, 2,
                [](const std::vector<float> & state, float) { return std::vector<float>(state.size(), 3.0e38F); },
                {}, {}, &large);
    });
}

// The host-vector solver and the device solver against lo_flow_* over a
// [1000 frames, 64] window with a 250-frame prefix, 50 steps, CFG 1.5.
void solver_parity() {
    const std::size_t frames = 1000, dim = 64, n = frames * dim, steps = 50, prefix = 250;
    const float g = 1.5F, sigma = 1.0e-4F;
    euler_input input;
    input.frames = frames;
    input.latent_dim = dim;
    input.incontext_frames = prefix;
    input.sigma_min = sigma;
    input.initial_noise.resize(n);
    input.normalized_incontext.assign(n, 0.0F);
    lo_gaussian_noise(input.initial_noise.data(), static_cast<int64_t>(n), 11);
    lo_gaussian_noise(input.normalized_incontext.data(), static_cast<int64_t>(prefix * dim), 12);

    // Velocities: v_u, v_c derived from the state so the callback depends on it.
    const auto branch = [](const float * state, uint64_t seed, std::vector<float> & out) {
        out.resize(n);
        lo_gaussian_noise(out.data(), static_cast<int64_t>(n), seed);
        for (std::size_t e = 0; e < n; ++e) out[e] = 0.5F * out[e] - 0.25F * state[e];
    };

    // Oracle.
    std::vector<float> want = input.initial_noise, vu, vc;
    const float dt = 1.0F / static_cast<float>(steps);
    for (std::size_t s = 0; s < steps; ++s) {
        const float t = static_cast<float>(s) * dt;
        lo_flow_incontext(want.data(), input.initial_noise.data(), input.normalized_incontext.data(),
                          static_cast<int64_t>(prefix * dim), t, sigma);
        branch(want.data(), 100 + s, vu);
        branch(want.data(), 200 + s, vc);
        lo_flow_cfg_euler(want.data(), vu.data(), vc.data(), static_cast<int64_t>(n), g, dt);
    }
    std::copy_n(input.normalized_incontext.begin(), prefix * dim, want.begin());

    // Host-vector solver: the callback returns the CFG-combined velocity.
    std::size_t step = 0;
    const std::vector<float> host = solve_flow_euler(input, steps, [&](const std::vector<float> & state, float) {
        std::vector<float> u, c, v(n);
        branch(state.data(), 100 + step, u);
        branch(state.data(), 200 + step, c);
        lo_apply_cfg(c.data(), u.data(), v.data(), static_cast<int64_t>(n), g);
        ++step;
        return v;
    });
    CHECK(bit_equal(host.data(), want.data(), n));

    // Device solver: the callback fills both branches in device memory.
    device_buffer<float> noise(n), context(n), state(n);
    noise.upload(input.initial_noise.data(), n, nullptr);
    context.upload(input.normalized_incontext.data(), n, nullptr);
    device_euler_input din;
    din.initial_noise = noise.data();
    din.normalized_incontext = context.data();
    din.frames = frames;
    din.latent_dim = dim;
    din.incontext_frames = prefix;
    din.sigma_min = sigma;
    std::vector<float> hstate(n);
    step = 0;
    euler_resume_state checkpoint;
    solve_flow_euler_device(
            din, steps, g,
            [&](const float * dstate, float, float * v_uncond, float * v_cond, stream_t stream) {
                levo::hip::check_hip(hipMemcpyAsync(hstate.data(), dstate, n * sizeof(float), hipMemcpyDeviceToHost,
                                                    stream),
                                     "copy");
                levo::hip::synchronize(stream);
                std::vector<float> u, c;
                branch(hstate.data(), 100 + step, u);
                branch(hstate.data(), 200 + step, c);
                levo::hip::check_hip(hipMemcpyAsync(v_uncond, u.data(), n * sizeof(float), hipMemcpyHostToDevice,
                                                    stream),
                                     "copy");
                levo::hip::check_hip(hipMemcpyAsync(v_cond, c.data(), n * sizeof(float), hipMemcpyHostToDevice,
                                                    stream),
                                     "copy");
                levo::hip::synchronize(stream);
                ++step;
            },
            state.data(), {}, {}, nullptr, &checkpoint);
    std::vector<float> dev(n);
    state.download(dev.data(), n, nullptr);
    levo::hip::synchronize(nullptr);
    CHECK(bit_equal(dev.data(), want.data(), n));
    CHECK(checkpoint.completed_steps == steps && checkpoint.normalized_state == dev);
}

// solve_flow_window_device at LeVo's window (1000 x 64, estimator rows
// 24 | 64 | 2048 | 64, 250 in-context frames, CFG 1.5) against the oracle's
// solver loop with the same stand-in estimator, computed on the host from
// the device input rows: velocity = (state column * 0.5 - t) +
// conditioning column * 0.25. The output columns outside the velocity slice
// hold NaN. Also: cancellation + resume from the checkpoint, a resume that
// has no step left, progress, and the errors.
void window_parity() {
    const std::size_t F = 1000, L = 64, M = 24, C = 2048, H = M + 2 * L + C, P = 250, n = F * L, steps = 12;
    const float g = 1.5F, sigma = 1.0e-4F;
    const auto gauss = [](std::size_t count, uint64_t seed) {
        std::vector<float> v(count);
        lo_gaussian_noise(v.data(), static_cast<int64_t>(count), seed);
        return v;
    };
    const std::vector<float> mask = gauss(F * M, 31), ctx = gauss(n, 32), cond = gauss(F * C, 33),
                             noise = gauss(n, 34);
    std::vector<float> mean = gauss(L, 35), sd = gauss(L, 36);
    for (auto & x : mean) x *= 0.1F;
    for (auto & x : sd) x = std::fabs(x) * 0.5F + 0.5F;
    const auto rows = [&](const std::vector<float> & state) {
        std::vector<float> mi(2 * F * H);
        for (std::size_t b = 0; b < 2; ++b) {
            for (std::size_t f = 0; f < F; ++f) {
                float * row = mi.data() + (b * F + f) * H;
                std::copy_n(mask.data() + f * M, M, row);
                std::copy_n(ctx.data() + f * L, L, row + M);
                if (b == 0) std::fill_n(row + M + L, C, 0.0F);
                else std::copy_n(cond.data() + f * C, C, row + M + L);
                std::copy_n(state.data() + f * L, L, row + M + L + C);
            }
        }
        return mi;
    };
    const auto velocity = [&](const float * mi, float t, std::size_t b, std::size_t f, std::size_t c) {
        const float * row = mi + (b * F + f) * H;
        return (row[H - L + c] * 0.5F - t) + row[M + L + c] * 0.25F;
    };

    // Oracle loop (src/levo-flow-renderer.cpp:89-117 + the CFG lambda).
    const float dt = 1.0F / static_cast<float>(steps);
    std::vector<float> want = noise, vu(n), vc(n);
    std::vector<std::vector<float>> after;
    for (std::size_t k = 0; k < steps; ++k) {
        const float t = static_cast<float>(k) * dt;
        lo_flow_incontext(want.data(), noise.data(), ctx.data(), static_cast<int64_t>(P * L), t, sigma);
        const std::vector<float> mi = rows(want);
        for (std::size_t f = 0; f < F; ++f) {
            for (std::size_t c = 0; c < L; ++c) {
                vu[f * L + c] = velocity(mi.data(), t, 0, f, c);
                vc[f * L + c] = velocity(mi.data(), t, 1, f, c);
            }
        }
        lo_flow_cfg_euler(want.data(), vu.data(), vc.data(), static_cast<int64_t>(n), g, dt);
        after.push_back(want);
    }
    std::copy_n(ctx.begin(), P * L, want.begin());
    std::vector<float> want_raw(n);
    for (std::size_t e = 0; e < n; ++e) want_raw[e] = want[e] * sd[e % L] + mean[e % L];

    device_buffer<float> d_mask(F * M), d_ctx(n), d_cond(F * C), d_noise(n), d_mean(L), d_sd(L), d_mi(2 * F * H),
            d_out(2 * F * H), d_state(n), d_raw(n);
    d_mask.upload(mask.data(), F * M, nullptr);
    d_ctx.upload(ctx.data(), n, nullptr);
    d_cond.upload(cond.data(), F * C, nullptr);
    d_noise.upload(noise.data(), n, nullptr);
    d_mean.upload(mean.data(), L, nullptr);
    d_sd.upload(sd.data(), L, nullptr);
    std::vector<float> host_out(2 * F * H, std::numeric_limits<float>::quiet_NaN()), host_mi(2 * F * H);
    device_euler_input din;
    din.initial_noise = d_noise.data();
    din.normalized_incontext = d_ctx.data();
    din.frames = F;
    din.latent_dim = L;
    din.incontext_frames = P;
    din.sigma_min = sigma;
    device_window_conditioning wc;
    wc.mask_embedding = d_mask.data();
    wc.mask_dim = M;
    wc.conditioning = d_cond.data();
    wc.condition_width = C;
    wc.latent_mean = d_mean.data();
    wc.latent_stddev = d_sd.data();
    device_estimator_tensors io;
    io.model_input = d_mi.data();
    io.output = d_out.data();
    io.hidden = H;
    std::vector<float> times;
    bool poison = false;
    const device_estimator_callback estimator = [&](float t, stream_t stream) {
        times.push_back(t);
        d_mi.download(host_mi.data(), 2 * F * H, stream);
        levo::hip::synchronize(stream);
        for (std::size_t b = 0; b < 2; ++b) {
            for (std::size_t f = 0; f < F; ++f) {
                for (std::size_t c = 0; c < L; ++c) host_out[(b * F + f) * H + H - L + c] = velocity(host_mi.data(), t, b, f, c);
            }
        }
        if (poison) host_out[(1 * F + 3) * H + H - 1] = std::numeric_limits<float>::quiet_NaN();
        d_out.upload(host_out.data(), 2 * F * H, stream);
    };
    const auto download = [&](const device_buffer<float> & d) {
        std::vector<float> h(n);
        d.download(h.data(), n, nullptr);
        levo::hip::synchronize(nullptr);
        return h;
    };

    // Whole window, checkpoint after every step.
    std::vector<std::size_t> progress;
    euler_resume_state checkpoint;
    solve_flow_window_device(din, wc, steps, g, io, estimator, d_state.data(), d_raw.data(),
                             [&](std::size_t done, std::size_t total) {
                                 CHECK(total == steps);
                                 progress.push_back(done);
                             },
                             {}, nullptr, &checkpoint);
    CHECK(progress.size() == steps && progress.back() == steps);
    CHECK(times.size() == steps && times[3] == 3.0F * dt);
    CHECK(bit_equal(download(d_state).data(), want.data(), n));
    CHECK(bit_equal(download(d_raw).data(), want_raw.data(), n));
    CHECK(checkpoint.completed_steps == steps && bit_equal(checkpoint.normalized_state.data(), want.data(), n));

    // Cancel after 5 steps: the checkpoint is the reference's state after
    // step 5; resuming from it finishes bit for bit.
    std::size_t polls = 0;
    euler_resume_state paused;
    expect_throw<levo::hip::operation_cancelled>("cancelled", [&] {
        solve_flow_window_device(din, wc, steps, g, io, estimator, d_state.data(), d_raw.data(), {},
                                 [&] { return polls++ == 5; }, nullptr, &paused);
    });
    CHECK(paused.completed_steps == 5 && bit_equal(paused.normalized_state.data(), after[4].data(), n));
    times.clear();
    solve_flow_window_device(din, wc, steps, g, io, estimator, d_state.data(), d_raw.data(), {}, {}, &paused);
    CHECK(times.size() == steps - 5 && times[0] == 5.0F * dt);
    CHECK(bit_equal(download(d_state).data(), want.data(), n));
    CHECK(bit_equal(download(d_raw).data(), want_raw.data(), n));

    // A resume with every step done: prefix restore and denormalization only.
    euler_resume_state done;
    done.completed_steps = steps;
    done.normalized_state = after.back();
    times.clear();
    solve_flow_window_device(din, wc, steps, g, io, estimator, d_state.data(), d_raw.data(), {}, {}, &done);
    CHECK(times.empty());
    CHECK(bit_equal(download(d_state).data(), want.data(), n));
    CHECK(bit_equal(download(d_raw).data(), want_raw.data(), n));

    // Errors.
    poison = true;
    expect_throw<std::runtime_error>("LeVo Flow renderer: Euler velocity contains a non-finite value", [&] {
        solve_flow_window_device(din, wc, steps, g, io, estimator, d_state.data());
    });
    poison = false;
    device_estimator_tensors bad = io;
    bad.hidden = H + 4;
    expect_throw<std::runtime_error>("estimator rows must hold", [&] {
        solve_flow_window_device(din, wc, steps, g, bad, estimator, d_state.data());
    });
    device_window_conditioning no_stats = wc;
    no_stats.latent_stddev = nullptr;
    expect_throw<std::runtime_error>("denormalization needs", [&] {
        solve_flow_window_device(din, no_stats, steps, g, io, estimator, d_state.data(), d_raw.data());
    });
    expect_throw<std::runtime_error>("Euler step count must be positive", [&] {
        solve_flow_window_device(din, wc, 0, g, io, estimator, d_state.data());
    });
}

} // namespace

int main() {
    try {
        reference_assertions();
        error_behaviour();
        solver_parity();
        window_parity();
    } catch (const std::exception & e) {
        std::cerr << "unexpected exception: " << e.what() << '\n';
        return 1;
    }
    std::cout << "hip flow renderer ok\n";
    return 0;
}
