// Wall-clock timings of the C++ drop-ins that keep the reference's
// host-vector signatures, transfers over PCIe included: what a caller that
// switches levo:: for levo::hip:: without moving its tensors to the GPU pays.
//   sample_streams   Sampler::sample_streams on three host rows of 16385
//                    logits (src/levo-sampling.cpp:129-152): penalty window
//                    50, three ignored ids, top-k 50 / 1 / 1, T = 0.9
//   solve_flow_euler flow::solve_flow_euler over a 1000 x 64 window (250
//                    in-context frames), 50 steps, with a host velocity
//                    callback that returns a fixed vector (the estimator's
//                    cost left out) (src/levo-flow-renderer.cpp:57-120)
//   quantize_chunk   a host F32 chunk of [4096, 1536] copied in, quantized
//                    to Q8_0 (ggml_quantize_chunk, tools/levo-quantize.cpp:
//                    386-388) and the blocks copied back
// Each: 3 warm-ups, then the median of N runs (std::chrono::steady_clock).
// Prints one JSON object. Part of the benchmark, not of the libraries.
#include "levo-hip-device.h"
#include "levo-hip-flow-renderer.h"
#include "levo-hip-quantize.h"
#include "levo-hip-sampling.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

namespace {

template <typename F>
double median_us(F && f, int runs) {
    for (int i = 0; i < 3; ++i) f();
    std::vector<double> t;
    for (int i = 0; i < runs; ++i) {
        const auto a = std::chrono::steady_clock::now();
        f();
        const auto b = std::chrono::steady_clock::now();
        t.push_back(std::chrono::duration<double, std::micro>(b - a).count());
    }
    std::sort(t.begin(), t.end());
    return t[t.size() / 2];
}

std::vector<float> gaussian(std::size_t n, uint32_t seed, float scale) {
    std::mt19937 rng(seed);
    std::normal_distribution<float> d(0.0f, scale);
    std::vector<float> v(n);
    for (auto & x : v) x = d(rng);
    return v;
}

}  // namespace

int main() {
    // ---- Sampler::sample_streams on host rows --------------------------------------
    const std::size_t V = 16385;
    std::vector<levo::hip::logits> streams;
    for (uint32_t q = 0; q < 3; ++q) streams.push_back(gaussian(V, 10 + q, 3.0f));
    std::vector<std::vector<int64_t>> recent(3);
    for (std::size_t q = 0; q < 3; ++q)
        for (int64_t i = 0; i < 50; ++i) recent[q].push_back((i * 97 + static_cast<int64_t>(q) * 31) % (V - 1));
    levo::hip::sampling_config cfg;
    cfg.ignore_tokens = {0, 1, 2};
    levo::hip::Sampler sampler(1234);
    int64_t sink = 0;
    const double sample_us = median_us([&] { sink += sampler.sample_streams(streams, cfg, recent)[0]; }, 200);

    // ---- flow::solve_flow_euler with a host velocity callback ----------------------
    const std::size_t frames = 1000, latent = 64, prefix = 250, steps = 50;
    levo::hip::flow::euler_input in;
    in.initial_noise = gaussian(frames * latent, 20, 1.0f);
    in.normalized_incontext = gaussian(frames * latent, 21, 1.0f);
    in.frames = frames;
    in.latent_dim = latent;
    in.incontext_frames = prefix;
    const std::vector<float> velocity = gaussian(frames * latent, 22, 0.1f);
    const auto cb = [&](const std::vector<float> &, float) { return velocity; };
    float fsink = 0.0f;
    const double flow_us = median_us([&] { fsink += levo::hip::flow::solve_flow_euler(in, steps, cb)[7]; }, 20);

    // ---- quantize_chunk from a host F32 chunk --------------------------------------
    const int64_t R = 4096, C = 1536;
    const std::vector<float> chunk = gaussian(static_cast<std::size_t>(R * C), 30, 0.02f);
    const std::size_t qbytes = levo::hip::row_size(LEVO_HIP_TYPE_Q8_0, C) * static_cast<std::size_t>(R);
    std::vector<uint8_t> blocks(qbytes);
    levo::hip::device_buffer<float> dsrc(static_cast<std::size_t>(R * C));
    levo::hip::device_buffer<uint8_t> ddst(qbytes);
    const double quant_us = median_us([&] {
        dsrc.upload(chunk.data(), chunk.size(), nullptr);
        levo::hip::quantize_chunk(LEVO_HIP_TYPE_Q8_0, dsrc.data(), ddst.data(), 0, R, C);
        ddst.download(blocks.data(), blocks.size(), nullptr);
        levo::hip::synchronize(nullptr);
    }, 20);

    std::printf("{\"sample_streams_3x16385_us\": %.1f, \"solve_flow_euler_1000x64_50_steps_us\": %.1f, "
                "\"quantize_chunk_q8_0_4096x1536_host_us\": %.1f, \"check\": %lld}\n",
                sample_us, flow_us, quant_us, static_cast<long long>(sink + static_cast<int64_t>(fsink) + blocks[5]));
    return 0;
}
