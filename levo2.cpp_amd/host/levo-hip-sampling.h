// Drop-in for the LeLM sampling surface of src/levo-sampling.h:10-64 with the
// per-token work on the GPU.
//
// Same names, arguments, defaults, results and exceptions as namespace levo:
// apply_cfg, sampling_config, apply_unique_token_repetition_penalty, Sampler
// (seed / draw_count / restore / uniform_bits / uniform01 / sample /
// sample_streams) and sample_top_k. A caller switches with
// `namespace levo_sampling = levo::hip;` or a using-declaration.
//
// What runs where: CFG, the repetition penalty, the ignore list, the NaN
// check, the first-maximum argmax and the top-k candidate set (all ties with
// the k-th value kept, ascending id order) run in one levo_hip_cfg_sample
// launch; a levo_hip_sample_draw launch turns the candidates into the
// reference's double weights exp((double)((v - max) / T)) and makes the
// uniform draw. The host keeps the mt19937_64 engine and its draw cursor: it
// hands the device the engine's next raw values and afterwards advances the
// engine by the number the rows consumed, so the sampled ids and the cursor
// are the reference's for the same seed. Per call only the ids and draw
// counts come back from the device.
//
// Limit: at most 32768 logits per row (LeVo's vocabulary is 16385).
#pragma once

#include "levo-hip-device.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <random>
#include <vector>

namespace levo::hip {

using logits = std::vector<float>;

// uncond + scale * (cond - uncond), two roundings (src/levo-sampling.cpp:22-37).
// Throws std::invalid_argument("CFG logits have different sizes") /
// ("CFG batch sizes differ").
logits apply_cfg(const logits & conditional, const logits & unconditional, float scale);
std::vector<logits> apply_cfg(const std::vector<logits> & conditional,
                              const std::vector<logits> & unconditional, float scale);

// Same fields and defaults as levo::sampling_config (src/levo-sampling.h:17-25).
struct sampling_config {
    bool use_sampling = true;
    float temperature = 0.9F;
    std::size_t top_k_mixed = 50;
    std::size_t top_k_detail = 1;
    std::size_t repetition_window = 50;
    float repetition_penalty = 1.1F;
    std::vector<int64_t> ignore_tokens;
};

// Each distinct id of recent_tokens inside [0, vocabulary_limit or size) is
// divided once (src/levo-sampling.cpp:39-53), computed on the GPU.
void apply_unique_token_repetition_penalty(logits & stream_logits,
                                           const std::vector<int64_t> & recent_tokens,
                                           float penalty = 1.1F,
                                           std::size_t vocabulary_limit = 0);
logits apply_unique_token_repetition_penalty(const logits & stream_logits,
                                             const std::vector<int64_t> & recent_tokens,
                                             float penalty = 1.1F,
                                             std::size_t vocabulary_limit = 0);

// A batch of logits rows already resident in device memory: the hot path.
// Row r belongs to stream r % streams (rows are [position][stream]).
struct device_logits {
    const float * conditional = nullptr;    // [rows][row_pitch]
    const float * unconditional = nullptr;  // [rows][row_pitch], or null: no CFG
    std::size_t rows = 0;
    std::size_t streams = 1;                // 1 .. LEVO_HIP_MAX_STREAMS
    std::size_t vocab = 0;
    std::size_t row_pitch = 0;              // 0 = vocab
    float cfg_scale = 1.0F;                 // logits = u + cfg_scale * (c - u)
};

namespace detail {
struct sample_workspace;

// The sampled branch of sample_top_k_counted (src/levo-sampling.cpp:97-115)
// over a candidate set (ids ascending, their logits) with the uniform taken
// from one raw mt19937_64 value: the host's draw for a row the device marks
// LEVO_HIP_TOKEN_RECHECK. Returns `best` when the weight total is not a
// positive finite number, as the reference does.
int64_t pick_candidate(const int32_t * ids, const float * values, std::size_t n, int32_t best, float temperature,
                       uint64_t raw);
}

class Sampler {
public:
    explicit Sampler(uint64_t seed = 0);
    ~Sampler();
    Sampler(Sampler &&) noexcept;
    Sampler & operator=(Sampler &&) noexcept;
    Sampler(const Sampler &) = delete;
    Sampler & operator=(const Sampler &) = delete;

    void seed(uint64_t seed);
    // Raw mt19937_64 values consumed since the last seed/restore.
    uint64_t draw_count() const noexcept { return draws_; }
    void restore(uint64_t seed, uint64_t draw_count);
    uint64_t uniform_bits();
    double uniform01();

    int64_t sample(const logits & input, std::size_t top_k = 0,
                   float temperature = 1.0F, bool use_sampling = true);
    std::vector<int64_t> sample_streams(const std::vector<logits> & streams,
                                        const sampling_config & config = {},
                                        const std::vector<std::vector<int64_t>> & recent = {});

    // sample_streams over device-resident rows with CFG fused in: for every
    // row in order, the id that levo::Sampler::sample_streams would return for
    // apply_cfg(cond_row, uncond_row, cfg_scale). `recent` is empty or has one
    // window per row (the trailing config.repetition_window ids are used).
    std::vector<int64_t> sample_device(const device_logits & batch, const sampling_config & config = {},
                                       const std::vector<std::vector<int64_t>> & recent = {});

    // Stream the sampler's kernels and copies are issued on (default: null stream).
    stream_t stream() const noexcept { return stream_; }
    void set_stream(stream_t stream) noexcept { stream_ = stream; }

private:
    std::mt19937_64 engine_;
    uint64_t draws_ = 0;
    stream_t stream_ = nullptr;
    std::unique_ptr<detail::sample_workspace> workspace_;
};

// Stateless entry point with an explicit engine (src/levo-sampling.h:62-64).
int64_t sample_top_k(const logits & input, std::size_t top_k, float temperature,
                     bool use_sampling, std::mt19937_64 & rng);

} // namespace levo::hip
