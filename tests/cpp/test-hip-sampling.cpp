// levo::hip sampling drop-in: the assertions of the reference's
// tests/test-sampling.cpp:8-48 restated against levo::hip, its error
// behaviour, and seeded parity with the oracle's restatement of
// src/levo-sampling.cpp at LeVo's shape (3 streams x 16385 logits).
#include "check.h"
#include "levo-hip-sampling.h"
#include "levo_oracle.h"

#include <cmath>
#include <iostream>
#include <limits>
#include <random>
#include <vector>

using namespace levo::hip;

namespace {

constexpr std::size_t kVocab = 16385;

std::vector<float> gaussian(std::size_t n, uint64_t seed, float scale) {
    std::vector<float> v(n);
    lo_gaussian_noise(v.data(), static_cast<int64_t>(n), seed);
    for (auto & x : v) x *= scale;
    return v;
}

void reference_assertions() {
    CHECK(apply_cfg({2, 4}, {1, 1}, 1.5F) == logits({2.5F, 5.5F}));
    logits x{10, 8, 6};
    apply_unique_token_repetition_penalty(x, {0, 0, 1}, 2.0F);
    CHECK(x[0] == 5 && x[1] == 4 && x[2] == 6);
    sampling_config config;
    config.use_sampling = false;
    config.repetition_penalty = 2.0F;
    Sampler upstream(0);
    CHECK(upstream.sample_streams({{9, 8, 10, 7}}, config, {{2, 3}})[0] == 0);
    Sampler a(1234), b(1234);
    for (int i = 0; i < 20; ++i) CHECK(a.sample({0, 1, 2}, 3, 1, true) == b.sample({0, 1, 2}, 3, 1, true));
    Sampler cursor(1234), uninterrupted(1234);
    std::vector<int64_t> full;
    for (int i = 0; i < 20; ++i) full.push_back(uninterrupted.sample({0, 1, 2, 3}, 4, 0.8F, true));
    for (int i = 0; i < 7; ++i) CHECK(cursor.sample({0, 1, 2, 3}, 4, 0.8F, true) == full[static_cast<std::size_t>(i)]);
    CHECK(cursor.draw_count() == 7);
    Sampler restored;
    restored.restore(1234, cursor.draw_count());
    for (int i = 7; i < 20; ++i) CHECK(restored.sample({0, 1, 2, 3}, 4, 0.8F, true) == full[static_cast<std::size_t>(i)]);
    (void) cursor.uniform_bits();
    CHECK(cursor.draw_count() == 8);
    (void) cursor.uniform01();
    CHECK(cursor.draw_count() == 9);
    Sampler greedy(12);
    CHECK(greedy.sample({0, 1, 2}, 3, 1.0F, false) == 2);
    CHECK(greedy.sample({0, 1, 2}, 3, 0.0F, true) == 2);
    sampling_config no_sampling;
    no_sampling.use_sampling = false;
    CHECK(greedy.sample_streams({{0, 2, 1}, {1, 4, 0}}, no_sampling) == std::vector<int64_t>({1, 1}));
    CHECK(greedy.draw_count() == 0);
    CHECK(Sampler(1).sample({-1, 3, -2}, 1, 1, true) == 1);
    std::mt19937_64 tie_rng(7);
    bool saw_first = false, saw_second = false;
    for (int i = 0; i < 64; ++i) {
        const auto token = sample_top_k({5, 5, 0}, 1, 1, true, tie_rng);
        saw_first |= token == 0;
        saw_second |= token == 1;
    }
    CHECK(saw_first && saw_second);
}

void error_behaviour() {
    expect_throw<std::invalid_argument>("cannot sample an empty vocabulary", [] { Sampler().sample({}); });
    expect_throw<std::invalid_argument>("temperature must be finite and non-negative",
                                        [] { Sampler().sample({1, 2}, 0, -1.0F); });
    expect_throw<std::invalid_argument>("temperature must be finite and non-negative",
                                        [] { Sampler().sample({1, 2}, 0, std::nanf("")); });
    expect_throw<std::invalid_argument>("logits contain NaN",
                                        [] { Sampler().sample({1, std::nanf(""), 2}, 0, 1.0F, false); });
    expect_throw<std::invalid_argument>("CFG logits have different sizes", [] { (void) apply_cfg({1, 2}, {1}, 1.5F); });
    expect_throw<std::invalid_argument>("CFG batch sizes differ",
                                        [] { (void) apply_cfg(std::vector<logits>{{1}}, std::vector<logits>{}, 1.5F); });
    expect_throw<std::invalid_argument>("CFG logits have different sizes", [] {
        (void) apply_cfg(std::vector<logits>{{1, 2}, {1, 2, 3}}, std::vector<logits>{{1, 2}, {1, 2}}, 1.5F);
    });
    // One launch over rows of different lengths, an empty row among them.
    {
        const std::vector<logits> c{{2, 4}, {}, {1, 2, 3}}, u{{1, 1}, {}, {3, 6, 0.5F}};
        const std::vector<logits> got = apply_cfg(c, u, 1.5F);
        CHECK(got.size() == 3 && got[1].empty());
        for (int i : {0, 2}) CHECK(got[static_cast<std::size_t>(i)] == apply_cfg(c[static_cast<std::size_t>(i)],
                                                                                  u[static_cast<std::size_t>(i)], 1.5F));
        CHECK(got[0] == logits({2.5F, 5.5F}));  // tests/test-sampling.cpp:8
    }
    expect_throw<std::invalid_argument>("recent-token stream count differs",
                                        [] { Sampler().sample_streams({{1, 2}, {3, 4}}, {}, {{1}}); });
    sampling_config bad;
    bad.repetition_penalty = 0.0F;
    expect_throw<std::invalid_argument>("repetition penalty must be finite and positive",
                                        [&] { Sampler().sample_streams({{1, 2}}, bad, {{1}}); });
    logits x{1, 2};
    expect_throw<std::invalid_argument>("repetition penalty must be finite and positive",
                                        [&] { apply_unique_token_repetition_penalty(x, {0}, -1.0F); });
    // A NaN in the second stream throws after the first stream's draw, as the
    // reference's per-stream loop does.
    Sampler s(5);
    expect_throw<std::invalid_argument>("logits contain NaN",
                                        [&] { s.sample_streams({{0, 1, 2}, {0, std::nanf(""), 1}}, {}, {}); });
    CHECK(s.draw_count() == 1);
}

// sample() against lo_sample_top_k over rows with forced ties at the k-th
// value and at the maximum, every top_k regime and temperature.
void sample_parity() {
    const std::vector<std::size_t> ks = {0, 1, 2, 50, 257, kVocab - 1, kVocab, kVocab + 5};
    const std::vector<float> temps = {0.0F, 0.5F, 0.9F, 1.0F, 2.0F};
    Sampler hip(99);
    lo_mt19937_64 rng;
    lo_mt_seed(&rng, 99);
    uint64_t draws = 0;
    int row = 0;
    for (std::size_t k : ks) {
        for (float t : temps) {
            for (int use = 0; use < 2; ++use) {
                std::vector<float> v = gaussian(kVocab, 1000 + static_cast<uint64_t>(row), 3.0F);
                for (int i = 0; i < 12; ++i) v[static_cast<std::size_t>(97 * i + row)] = 6.5F;      // tied maxima
                for (int i = 0; i < 9; ++i) v[static_cast<std::size_t>(1301 * i + 11)] = 2.25F;    // ties mid-rank
                v[kVocab - 1] = -std::numeric_limits<float>::infinity();
                ++row;
                int64_t want = -1;
                CHECK(lo_sample_top_k(v.data(), static_cast<int64_t>(kVocab), static_cast<int64_t>(k), t, use, &rng,
                                      &draws, &want) == 0);
                const int64_t got = hip.sample(v, k, t, use != 0);
                if (got != want || hip.draw_count() != draws) {
                    std::fprintf(stderr, "sample mismatch k=%zu t=%g use=%d: %lld vs %lld (draws %llu vs %llu)\n", k,
                                 static_cast<double>(t), use, static_cast<long long>(got), static_cast<long long>(want),
                                 static_cast<unsigned long long>(hip.draw_count()),
                                 static_cast<unsigned long long>(draws));
                    std::exit(1);
                }
            }
        }
    }
}

// detail::pick_candidate (the host draw for rows the device flags) against
// the oracle's sample_top_k_counted with top_k = 0 over the same candidate
// values and the same next raw engine value: ties, -inf entries, one
// candidate, all -inf (no draw: the first maximum).
void pick_candidate_parity() {
    lo_mt19937_64 rng;
    lo_mt_seed(&rng, 4242);
    uint64_t draws = 0;
    const float ninf = -std::numeric_limits<float>::infinity();
    for (int set = 0; set < 300; ++set) {
        const std::size_t n = 1 + static_cast<std::size_t>(set * 37) % 300;
        std::vector<float> v = gaussian(n, 5000 + static_cast<uint64_t>(set), 2.0F);
        if (set % 3 == 0) for (std::size_t i = 0; i < n; i += 7) v[i] = v[0];
        if (set % 5 == 0) for (std::size_t i = 1; i < n; i += 4) v[i] = ninf;
        if (set == 7) std::fill(v.begin(), v.end(), ninf);
        std::vector<int32_t> ids(n);
        for (std::size_t i = 0; i < n; ++i) ids[i] = static_cast<int32_t>(3 * i + 1);
        std::size_t first_max = 0;
        for (std::size_t i = 1; i < n; ++i) if (v[i] > v[first_max]) first_max = i;
        const float t = set % 4 == 0 ? 0.25F : set % 4 == 1 ? 0.9F : 2.0F;
        lo_mt19937_64 peek = rng;
        const uint64_t raw = lo_mt_next(&peek);
        int64_t want = -1;
        CHECK(lo_sample_top_k(v.data(), static_cast<int64_t>(n), 0, t, 1, &rng, &draws, &want) == 0);
        const int64_t got = detail::pick_candidate(ids.data(), v.data(), n, ids[first_max], t, raw);
        CHECK(got == ids[static_cast<std::size_t>(want)]);
    }
    CHECK(draws == 299);  // every set draws except the all -inf one
}

// A 40-step generation loop at LeVo's shape: CFG on the host, the penalty
// window fed back from the sampled ids, the prompt ignore list on stream 0.
void streams_parity() {
    sampling_config config;
    config.ignore_tokens = {3, 17, 16000, 40000, -2};
    Sampler hip(2024);
    lo_mt19937_64 rng;
    lo_mt_seed(&rng, 2024);
    uint64_t draws = 0;
    std::vector<std::vector<int64_t>> history(3);
    for (int step = 0; step < 40; ++step) {
        std::vector<logits> cond(3), uncond(3);
        for (int q = 0; q < 3; ++q) {
            cond[q] = gaussian(kVocab, 50000 + static_cast<uint64_t>(step * 6 + q), 3.0F);
            uncond[q] = gaussian(kVocab, 60000 + static_cast<uint64_t>(step * 6 + q), 3.0F);
        }
        const std::vector<logits> mixed = apply_cfg(cond, uncond, 1.5F);
        std::vector<float> flat(3 * kVocab);
        for (int q = 0; q < 3; ++q) {
            std::vector<float> want_row(kVocab);
            lo_apply_cfg(cond[q].data(), uncond[q].data(), want_row.data(), static_cast<int64_t>(kVocab), 1.5F);
            CHECK(bit_equal(want_row.data(), mixed[q].data(), kVocab));
            std::copy(want_row.begin(), want_row.end(), flat.begin() + q * static_cast<std::ptrdiff_t>(kVocab));
        }
        const std::size_t width = std::min<std::size_t>(config.repetition_window, history[0].size());
        std::vector<int64_t> windows(3 * width, -1);
        for (int q = 0; q < 3; ++q) {
            const auto & h = history[static_cast<std::size_t>(q)];
            std::copy(h.end() - static_cast<std::ptrdiff_t>(width), h.end(), windows.begin() + q * static_cast<std::ptrdiff_t>(width));
        }
        std::vector<int64_t> want(3);
        CHECK(lo_sample_streams(flat.data(), 3, static_cast<int64_t>(kVocab), 1, config.temperature,
                                static_cast<int64_t>(config.top_k_mixed), static_cast<int64_t>(config.top_k_detail),
                                config.repetition_penalty, width ? windows.data() : nullptr,
                                static_cast<int64_t>(width), config.ignore_tokens.data(),
                                static_cast<int64_t>(config.ignore_tokens.size()), &rng, &draws, want.data()) == 0);
        const std::vector<int64_t> got = hip.sample_streams(mixed, config, history);
        CHECK(got == want);
        CHECK(hip.draw_count() == draws);
        for (int q = 0; q < 3; ++q) history[static_cast<std::size_t>(q)].push_back(got[static_cast<std::size_t>(q)]);
    }
}

// sample_device over [positions][3][V] device rows with CFG fused in.
void device_parity() {
    const std::size_t positions = 24, rows = positions * 3;
    std::vector<float> cond(rows * kVocab), uncond(rows * kVocab);
    lo_gaussian_noise(cond.data(), static_cast<int64_t>(cond.size()), 71);
    lo_gaussian_noise(uncond.data(), static_cast<int64_t>(uncond.size()), 72);
    for (auto & v : cond) v *= 3.0F;
    for (auto & v : uncond) v *= 3.0F;
    device_buffer<float> dc(cond.size()), du(uncond.size());
    dc.upload(cond.data(), cond.size(), nullptr);
    du.upload(uncond.data(), uncond.size(), nullptr);
    synchronize(nullptr);
    std::vector<std::vector<int64_t>> recent(rows);
    for (std::size_t r = 0; r < rows; ++r) {
        for (std::size_t j = 0; j < 60; ++j) recent[r].push_back(static_cast<int64_t>((r * 7919 + j * 104729) % kVocab));
    }
    for (int use = 0; use < 2; ++use) {
        sampling_config config;
        config.use_sampling = use != 0;
        config.ignore_tokens = {5, 6, 7};
        device_logits batch;
        batch.conditional = dc.data();
        batch.unconditional = du.data();
        batch.rows = rows;
        batch.streams = 3;
        batch.vocab = kVocab;
        batch.cfg_scale = 1.5F;
        Sampler hip(314);
        const std::vector<int64_t> got = hip.sample_device(batch, config, recent);
        lo_mt19937_64 rng;
        lo_mt_seed(&rng, 314);
        uint64_t draws = 0;
        for (std::size_t p = 0; p < positions; ++p) {
            std::vector<float> flat(3 * kVocab);
            std::vector<int64_t> windows(3 * 50);
            for (std::size_t q = 0; q < 3; ++q) {
                const std::size_t r = p * 3 + q;
                lo_apply_cfg(cond.data() + r * kVocab, uncond.data() + r * kVocab, flat.data() + q * kVocab,
                             static_cast<int64_t>(kVocab), 1.5F);
                std::copy(recent[r].end() - 50, recent[r].end(), windows.begin() + static_cast<std::ptrdiff_t>(q * 50));
            }
            std::vector<int64_t> want(3);
            CHECK(lo_sample_streams(flat.data(), 3, static_cast<int64_t>(kVocab), use, config.temperature, 50, 1,
                                    config.repetition_penalty, windows.data(), 50, config.ignore_tokens.data(), 3,
                                    &rng, &draws, want.data()) == 0);
            for (std::size_t q = 0; q < 3; ++q) CHECK(got[p * 3 + q] == want[q]);
        }
        CHECK(hip.draw_count() == draws);
    }
}

// Streams of different lengths take one launch per stream.
void ragged_streams() {
    Sampler hip(8);
    lo_mt19937_64 rng;
    lo_mt_seed(&rng, 8);
    uint64_t draws = 0;
    const logits s0 = gaussian(5, 1, 2.0F), s1 = gaussian(7, 2, 2.0F);
    sampling_config config;
    config.top_k_mixed = 3;
    config.top_k_detail = 2;
    const auto got = hip.sample_streams({s0, s1}, config);
    int64_t w0 = -1, w1 = -1;
    CHECK(lo_sample_top_k(s0.data(), 5, 3, config.temperature, 1, &rng, &draws, &w0) == 0);
    CHECK(lo_sample_top_k(s1.data(), 7, 2, config.temperature, 1, &rng, &draws, &w1) == 0);
    CHECK(got == std::vector<int64_t>({w0, w1}));
    CHECK(hip.draw_count() == draws);
}

} // namespace

int main() {
    try {
        reference_assertions();
        error_behaviour();
        sample_parity();
        pick_candidate_parity();
        streams_parity();
        device_parity();
        ragged_streams();
    } catch (const std::exception & e) {
        std::cerr << "unexpected exception: " << e.what() << '\n';
        return 1;
    }
    std::cout << "hip sampling ok\n";
    return 0;
}
