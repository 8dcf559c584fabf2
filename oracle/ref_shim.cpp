// ref_shim.cpp — C entry points over the reference's own std-only sources.
//
// TEST INFRASTRUCTURE ONLY. oracle/Makefile compiles this file together with
// src/levo-sampling.cpp and src/levo-renderer-pattern.cpp straight from the
// reference checkout into oracle/_ref/libref_levo.so. Tests use it to pin the
// oracle's restatement bit-for-bit; bench.py's cpu_baseline leg may time it.
// Nothing from the reference is copied here: this file only calls its public
// API (src/levo-sampling.h:13-64, src/levo-renderer-pattern.h:65-72).
#include "levo-renderer-pattern.h"
#include "levo-sampling.h"

#include <cstdint>
#include <cstring>
#include <exception>
#include <random>
#include <string>
#include <vector>

namespace {
thread_local std::string g_error;

template <typename F>
int guarded(F && f) {
    try {
        f();
        return 0;
    } catch (const std::exception & e) {
        g_error = e.what();
        return -1;
    }
}
} // namespace

extern "C" {

const char * ref_last_error(void) { return g_error.c_str(); }

int ref_apply_cfg(const float * cond, const float * uncond, int64_t n, float scale, float * out) {
    return guarded([&] {
        const levo::logits c(cond, cond + n), u(uncond, uncond + n);
        const levo::logits r = levo::apply_cfg(c, u, scale);
        std::memcpy(out, r.data(), sizeof(float) * r.size());
    });
}

int ref_combine_renderer_cfg(const float * uncond, const float * cond, int64_t n, float guidance,
                             float * out) {
    return guarded([&] {
        const std::vector<float> u(uncond, uncond + n), c(cond, cond + n);
        const std::vector<float> r = levo::combine_renderer_cfg(u, c, guidance);
        std::memcpy(out, r.data(), sizeof(float) * r.size());
    });
}

int ref_euler_schedule(int64_t steps, float * times, float * dt) {
    return guarded([&] {
        const auto s = levo::make_renderer_euler_schedule(static_cast<std::size_t>(steps));
        std::memcpy(times, s.times.data(), sizeof(float) * s.times.size());
        *dt = s.dt;
    });
}

int ref_repetition_penalty(float * logits, int64_t n, const int64_t * recent, int64_t n_recent,
                           float penalty, int64_t vocabulary_limit) {
    return guarded([&] {
        levo::logits l(logits, logits + n);
        const std::vector<int64_t> r(recent, recent + n_recent);
        levo::apply_unique_token_repetition_penalty(l, r, penalty,
                                                    static_cast<std::size_t>(vocabulary_limit));
        std::memcpy(logits, l.data(), sizeof(float) * l.size());
    });
}

uint64_t ref_mt19937_64_after(uint64_t seed, uint64_t discard) {
    std::mt19937_64 engine(seed);
    engine.discard(discard);
    return engine();
}

void * ref_sampler_new(uint64_t seed) { return new levo::Sampler(seed); }
void ref_sampler_free(void * s) { delete static_cast<levo::Sampler *>(s); }
uint64_t ref_sampler_draw_count(void * s) { return static_cast<levo::Sampler *>(s)->draw_count(); }
void ref_sampler_restore(void * s, uint64_t seed, uint64_t draws) {
    static_cast<levo::Sampler *>(s)->restore(seed, draws);
}

int ref_sampler_sample(void * s, const float * logits, int64_t n, int64_t top_k, float temperature,
                       int use_sampling, int64_t * token) {
    return guarded([&] {
        const levo::logits l(logits, logits + n);
        *token = static_cast<levo::Sampler *>(s)->sample(l, static_cast<std::size_t>(top_k), temperature,
                                                         use_sampling != 0);
    });
}

// One position of Sampler::sample_streams. recent is [n_streams][n_recent]
// with negative padding removed per stream; pass recent == nullptr for none.
int ref_sampler_sample_streams(void * s, const float * logits, int64_t n_streams, int64_t vocab,
                               int use_sampling, float temperature, int64_t top_k_mixed,
                               int64_t top_k_detail, int64_t repetition_window,
                               float repetition_penalty, const int64_t * recent,
                               int64_t n_recent, const int64_t * ignore, int64_t n_ignore,
                               int64_t * tokens) {
    return guarded([&] {
        std::vector<levo::logits> streams;
        for (int64_t q = 0; q < n_streams; ++q)
            streams.emplace_back(logits + q * vocab, logits + (q + 1) * vocab);
        levo::sampling_config config;
        config.use_sampling = use_sampling != 0;
        config.temperature = temperature;
        config.top_k_mixed = static_cast<std::size_t>(top_k_mixed);
        config.top_k_detail = static_cast<std::size_t>(top_k_detail);
        config.repetition_window = static_cast<std::size_t>(repetition_window);
        config.repetition_penalty = repetition_penalty;
        config.ignore_tokens.assign(ignore, ignore + n_ignore);
        std::vector<std::vector<int64_t>> history;
        if (recent) {
            for (int64_t q = 0; q < n_streams; ++q) {
                std::vector<int64_t> h;
                for (int64_t i = 0; i < n_recent; ++i) {
                    const int64_t t = recent[q * n_recent + i];
                    if (t >= 0) h.push_back(t);
                }
                history.push_back(std::move(h));
            }
        }
        const std::vector<int64_t> out =
            static_cast<levo::Sampler *>(s)->sample_streams(streams, config, history);
        std::memcpy(tokens, out.data(), sizeof(int64_t) * out.size());
    });
}

} // extern "C"
