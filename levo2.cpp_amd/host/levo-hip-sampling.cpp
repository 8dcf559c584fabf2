// levo::hip sampling surface over levo_hip_sample_step (levo_hip_cfg_sample /
// levo_hip_sample_draw for many rows) / levo_hip_cfg_combine /
// levo_hip_repetition_penalty. Behaviour follows src/levo-sampling.cpp:12-152.
#include "levo-hip-sampling.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <map>
#include <mutex>
#include <stdexcept>

namespace levo::hip {

namespace detail {

// Device and pinned buffers reused across calls of one Sampler.
struct sample_workspace {
    device_buffer<float> logits;      // uploaded host rows
    device_buffer<int64_t> recent;    // [rows][window] penalty windows, -1 padded
    device_buffer<int64_t> ignore;
    device_buffer<int32_t> best;
    device_buffer<int32_t> count;
    device_buffer<int32_t> cand_ids;
    device_buffer<float> cand_logits;
    device_buffer<float> row_max;
    device_buffer<uint64_t> bits;     // next raw engine values for the device draw
    device_buffer<int64_t> tokens;
    device_buffer<int32_t> draws;
    pinned_buffer<float> stage;       // host rows staged for upload
    pinned_buffer<int64_t> stage_ids; // recent windows + ignore list staged for upload
    pinned_buffer<int32_t> h_best;
    pinned_buffer<int32_t> h_count;
    pinned_buffer<int32_t> h_ids;
    pinned_buffer<float> h_logits;
    pinned_buffer<uint64_t> h_bits;
    pinned_buffer<int64_t> h_tokens;
    pinned_buffer<int32_t> h_draws;
    device_buffer<uint8_t> step;      // levo_hip_sample_step's hand-over workspace
    std::size_t capacity = 64;        // candidate slots per row; grows on demand
};

// Rows per call that levo_hip_sample_step takes (the decode step's few rows);
// more rows take levo_hip_cfg_sample and levo_hip_sample_draw.
constexpr int64_t kStepRows = 4095;

// The candidates of args.rows rows and, with d, their draws: one
// levo_hip_sample_step call (a part launch and a join-and-draw launch, the
// same results as levo_hip_cfg_sample followed by levo_hip_sample_draw) when
// the rows fit it, else those two launches.
void launch_rows(sample_workspace & ws, const levo_hip_sample_args & args, const levo_hip_draw_args * d,
                 stream_t stream) {
    if (args.rows >= 1 && args.rows <= kStepRows) {
        // < 0 for a vocabulary the kernels do not take: the two launches
        // below then report it with their own message
        const int64_t bytes = levo_hip_sample_step_workspace_bytes(args.rows, args.vocab);
        if (bytes >= 0) {
            ws.step.reserve_discard(static_cast<std::size_t>(bytes));
            check_status(levo_hip_sample_step(&args, d, ws.step.data(), bytes, stream));
            return;
        }
    }
    check_status(levo_hip_cfg_sample(&args, stream));
    if (d) check_status(levo_hip_sample_draw(d, stream));
}

int64_t pick_candidate(const int32_t * ids, const float * values, std::size_t n, int32_t best, float temperature,
                       uint64_t raw) {
    thread_local std::vector<double> weights;
    float max_logit = -std::numeric_limits<float>::infinity();
    for (std::size_t i = 0; i < n; ++i) max_logit = std::max(max_logit, values[i]);
    weights.resize(n);
    double total = 0.0;
    for (std::size_t i = 0; i < n; ++i) {
        const float v = values[i];
        weights[i] = (std::isinf(v) && v < 0.0F)
                         ? 0.0
                         : std::exp(static_cast<double>((v - max_logit) / temperature));
        total += weights[i];
    }
    if (!(total > 0.0) || !std::isfinite(total)) return best;
    const double target = (static_cast<double>(raw >> 11) + 0.5) / 9007199254740992.0 * total;
    double cumulative = 0.0;
    for (std::size_t i = 0; i < n; ++i) {
        cumulative += weights[i];
        if (target < cumulative) return ids[i];
    }
    return ids[n - 1];
}

} // namespace detail

namespace {

using detail::sample_workspace;

constexpr double kTwoPow53 = 9007199254740992.0;

// (53 random bits + 0.5) / 2^53: never 0 or 1 (src/levo-sampling.cpp:12-18).
double manual_uniform(std::mt19937_64 & rng, uint64_t * draws) {
    if (draws) ++*draws;
    return (static_cast<double>(rng() >> 11) + 0.5) / kTwoPow53;
}

void require_temperature(float temperature) {
    if (!std::isfinite(temperature) || temperature < 0.0F) {
        throw std::invalid_argument("temperature must be finite and non-negative");
    }
}

void require_penalty(float penalty) {
    if (!(penalty > 0.0F) || !std::isfinite(penalty)) {
        throw std::invalid_argument("repetition penalty must be finite and positive");
    }
}

// top_k as the kernel takes it: 0 keeps every id (reference: top_k == 0 or
// top_k >= vocabulary size skips the cut).
int32_t kernel_top_k(std::size_t top_k, std::size_t vocab) {
    if (top_k == 0 || top_k >= vocab || top_k > static_cast<std::size_t>(std::numeric_limits<int32_t>::max())) {
        return 0;
    }
    return static_cast<int32_t>(top_k);
}

// Advances the engine past the `n` raw values the rows consumed.
void advance(std::mt19937_64 & rng, uint64_t * draws, uint64_t n) {
    rng.discard(n);
    if (draws) *draws += n;
}

// Host draw of one row whose device pick was flagged LEVO_HIP_TOKEN_RECHECK:
// its candidates come back and pick_candidate (the reference's libm exp)
// decides with the same raw value.
int64_t recheck_row(sample_workspace & ws, std::size_t r, std::size_t cap, float temperature, uint64_t raw,
                    stream_t stream) {
    ws.h_best.reserve_discard(1);
    ws.h_count.reserve_discard(1);
    ws.h_ids.reserve_discard(cap);
    ws.h_logits.reserve_discard(cap);
    check_hip(hipMemcpyAsync(ws.h_best.data(), ws.best.data() + r, sizeof(int32_t), hipMemcpyDeviceToHost, stream),
              "device-to-host copy");
    check_hip(hipMemcpyAsync(ws.h_count.data(), ws.count.data() + r, sizeof(int32_t), hipMemcpyDeviceToHost,
                             stream),
              "device-to-host copy");
    check_hip(hipMemcpyAsync(ws.h_ids.data(), ws.cand_ids.data() + r * cap, cap * sizeof(int32_t),
                             hipMemcpyDeviceToHost, stream),
              "device-to-host copy");
    check_hip(hipMemcpyAsync(ws.h_logits.data(), ws.cand_logits.data() + r * cap, cap * sizeof(float),
                             hipMemcpyDeviceToHost, stream),
              "device-to-host copy");
    synchronize(stream);
    return detail::pick_candidate(ws.h_ids.data(), ws.h_logits.data(), static_cast<std::size_t>(ws.h_count[0]),
                                  ws.h_best[0], temperature, raw);
}

// The ids sample_top_k_counted returns (src/levo-sampling.cpp:75-116) for
// args.rows consecutive rows, in row order as sample_streams takes them
// (:135-150). The candidates and, for sampled rows, the draws fed with the
// engine's next raw values (read from a copy, so nothing is consumed yet)
// come from launch_rows. Only the ids and the draw counts
// come back; the engine then advances by exactly the values the reference's
// rows would have consumed, also when a NaN row ends the batch.
std::vector<int64_t> sample_rows(sample_workspace & ws, levo_hip_sample_args args, bool greedy, float temperature,
                                 std::mt19937_64 & rng, uint64_t * draws, stream_t stream) {
    const std::size_t rows = static_cast<std::size_t>(args.rows);
    std::vector<int64_t> out(rows);
    ws.best.reserve_discard(rows);
    ws.count.reserve_discard(rows);
    args.best = ws.best.data();
    args.count = ws.count.data();
    args.cand_probs = nullptr;
    args.row_lse = nullptr;
    if (greedy) {
        ws.cand_ids.reserve_discard(rows);
        ws.h_best.reserve_discard(rows);
        args.cand_ids = ws.cand_ids.data();
        args.cand_logits = nullptr;
        args.row_max = nullptr;
        args.capacity = 1;
        launch_rows(ws, args, nullptr, stream);
        ws.best.download(ws.h_best.data(), rows, stream);
        synchronize(stream);
        for (std::size_t r = 0; r < rows; ++r) {
            if (ws.h_best[r] < 0) throw std::invalid_argument("logits contain NaN");
            out[r] = ws.h_best[r];
        }
        return out;
    }

    ws.h_bits.reserve_discard(rows);
    ws.bits.reserve_discard(rows);
    {
        std::mt19937_64 peek = rng;
        for (std::size_t r = 0; r < rows; ++r) ws.h_bits[r] = peek();
    }
    ws.bits.upload(ws.h_bits.data(), rows, stream);
    ws.row_max.reserve_discard(rows);
    ws.tokens.reserve_discard(rows);
    ws.draws.reserve_discard(rows);
    ws.h_tokens.reserve_discard(rows);
    ws.h_draws.reserve_discard(rows);
    for (;;) {
        const std::size_t cap = ws.capacity;
        ws.cand_ids.reserve_discard(rows * cap);
        ws.cand_logits.reserve_discard(rows * cap);
        args.cand_ids = ws.cand_ids.data();
        args.cand_logits = ws.cand_logits.data();
        args.row_max = ws.row_max.data();
        args.capacity = static_cast<int32_t>(cap);
        levo_hip_draw_args d;
        std::memset(&d, 0, sizeof(d));
        d.best = ws.best.data();
        d.count = ws.count.data();
        d.cand_ids = ws.cand_ids.data();
        d.cand_logits = ws.cand_logits.data();
        d.row_max = ws.row_max.data();
        d.rows = args.rows;
        d.capacity = args.capacity;
        d.temperature = temperature;
        d.use_sampling = 1;
        d.bits = ws.bits.data();
        d.tokens = ws.tokens.data();
        d.draws = ws.draws.data();
        launch_rows(ws, args, &d, stream);
        ws.tokens.download(ws.h_tokens.data(), rows, stream);
        ws.draws.download(ws.h_draws.data(), rows, stream);
        synchronize(stream);
        std::size_t r = 0;
        while (r < rows && ws.h_tokens[r] != LEVO_HIP_TOKEN_NAN && ws.h_tokens[r] != LEVO_HIP_TOKEN_OVERFLOW) ++r;
        if (r == rows || ws.h_tokens[r] == LEVO_HIP_TOKEN_NAN) break;
        // A candidate set outgrew the slots: size them for the largest set and
        // run again with the same raw values (none has been consumed).
        ws.h_count.reserve_discard(rows);
        ws.count.download(ws.h_count.data(), rows, stream);
        synchronize(stream);
        std::size_t needed = cap;
        for (std::size_t q = 0; q < rows; ++q) {
            if (ws.h_count[q] > 0) needed = std::max(needed, static_cast<std::size_t>(ws.h_count[q]));
        }
        ws.capacity = (needed + 63) / 64 * 64;
    }
    for (std::size_t r = 0; r < rows; ++r) {
        const int64_t t = ws.h_tokens[r];
        if (t == LEVO_HIP_TOKEN_NAN) {
            advance(rng, draws, r == 0 ? 0 : static_cast<uint64_t>(ws.h_draws[r - 1]));
            throw std::invalid_argument("logits contain NaN");
        }
        out[r] = t == LEVO_HIP_TOKEN_RECHECK
                     ? recheck_row(ws, r, ws.capacity, temperature, ws.h_bits[ws.h_draws[r] - 1], stream)
                     : t;
    }
    advance(rng, draws, static_cast<uint64_t>(ws.h_draws[rows - 1]));
    return out;
}

// Uploads penalty windows ([rows][width], -1 padded) and the ignore list.
void stage_lists(sample_workspace & ws, levo_hip_sample_args & args,
                 const std::vector<std::vector<int64_t>> & windows,
                 const std::vector<int64_t> & ignore, float penalty, stream_t stream) {
    std::size_t width = 0;
    for (const auto & w : windows) width = std::max(width, w.size());
    const std::size_t n_recent = windows.size() * width;
    const std::size_t total = n_recent + ignore.size();
    args.recent = nullptr;
    args.n_recent = 0;
    args.ignore = nullptr;
    args.n_ignore = 0;
    if (total == 0) return;
    if (width > static_cast<std::size_t>(std::numeric_limits<int32_t>::max()) ||
        ignore.size() > static_cast<std::size_t>(std::numeric_limits<int32_t>::max())) {
        throw std::invalid_argument("LeVo HIP sampler: token list is too long");
    }
    ws.stage_ids.reserve_discard(total);
    for (std::size_t r = 0; r < windows.size(); ++r) {
        int64_t * dst = ws.stage_ids.data() + r * width;
        std::copy(windows[r].begin(), windows[r].end(), dst);
        std::fill(dst + windows[r].size(), dst + width, int64_t{-1});
    }
    std::copy(ignore.begin(), ignore.end(), ws.stage_ids.data() + n_recent);
    if (n_recent > 0) {
        ws.recent.reserve_discard(n_recent);
        ws.recent.upload(ws.stage_ids.data(), n_recent, stream);
        args.recent = ws.recent.data();
        args.n_recent = static_cast<int32_t>(width);
        args.repetition_penalty = penalty;
    }
    if (!ignore.empty()) {
        ws.ignore.reserve_discard(ignore.size());
        ws.ignore.upload(ws.stage_ids.data() + n_recent, ignore.size(), stream);
        args.ignore = ws.ignore.data();
        args.n_ignore = static_cast<int32_t>(ignore.size());
    }
}

// The trailing `window` ids of a stream's history (src/levo-sampling.cpp:138-139).
std::vector<int64_t> trailing(const std::vector<int64_t> & history, std::size_t window) {
    const std::size_t begin = history.size() > window ? history.size() - window : 0;
    return std::vector<int64_t>(history.begin() + static_cast<std::ptrdiff_t>(begin), history.end());
}

levo_hip_sample_args base_args() {
    levo_hip_sample_args a;
    std::memset(&a, 0, sizeof(a));
    a.cfg_scale = 1.0F;
    a.temperature = 1.0F;
    a.n_streams = 1;
    a.repetition_penalty = 1.0F;
    return a;
}

// One host row through the kernels (uploading it first).
int64_t sample_host_row(sample_workspace & ws, const logits & input, std::size_t top_k, float temperature,
                        bool use_sampling, std::mt19937_64 & rng, uint64_t * draws, stream_t stream,
                        const std::vector<int64_t> * window, float penalty,
                        const std::vector<int64_t> * ignore) {
    if (input.empty()) throw std::invalid_argument("cannot sample an empty vocabulary");
    require_temperature(temperature);
    const bool greedy = !use_sampling || temperature == 0.0F;
    const std::size_t V = input.size();
    ws.stage.reserve_discard(V);
    std::copy(input.begin(), input.end(), ws.stage.data());
    ws.logits.reserve_discard(V);
    ws.logits.upload(ws.stage.data(), V, stream);
    levo_hip_sample_args args = base_args();
    args.cond = ws.logits.data();
    args.rows = 1;
    args.vocab = static_cast<int64_t>(V);
    args.row_pitch = static_cast<int64_t>(V);
    args.top_k[0] = kernel_top_k(top_k, V);
    std::vector<std::vector<int64_t>> windows;
    if (window) windows.push_back(*window);
    args.penalty_limit = static_cast<int64_t>(V - 1);
    stage_lists(ws, args, windows, ignore ? *ignore : std::vector<int64_t>{}, penalty, stream);
    return sample_rows(ws, args, greedy, temperature, rng, draws, stream)[0];
}

} // namespace

// ---- CFG ----------------------------------------------------------------------

namespace {

// Device and pinned staging for the host-vector CFG calls, one per GPU, kept
// (and grown) for the process's lifetime; calls are serialized.
struct cfg_workspace {
    device_buffer<float> dev;   // [uncond | cond | out]
    pinned_buffer<float> host;  // the same, staged
};

std::mutex cfg_mutex;

cfg_workspace & cfg_workspace_for_current_device() {
    static std::map<int, cfg_workspace *> per_device;  // never freed: the runtime may be gone at exit
    int device = 0;
    check_hip(hipGetDevice(&device), "current device");
    cfg_workspace *& ws = per_device[device];
    if (ws == nullptr) ws = new cfg_workspace;
    return *ws;
}

// out[i] = apply_cfg(cond[i], uncond[i], scale) for every pair at once: one
// upload of all rows, one levo_hip_cfg_combine launch over them, one download.
void cfg_batch(const logits * const * cond, const logits * const * uncond, std::size_t pairs, float scale,
               logits * out) {
    std::size_t total = 0;
    for (std::size_t i = 0; i < pairs; ++i) total += cond[i]->size();
    for (std::size_t i = 0; i < pairs; ++i) out[i].assign(cond[i]->size(), 0.0F);
    if (total == 0) return;
    std::lock_guard<std::mutex> lock(cfg_mutex);
    cfg_workspace & ws = cfg_workspace_for_current_device();
    ws.dev.reserve_discard(3 * total);
    ws.host.reserve_discard(3 * total);
    float * hu = ws.host.data();
    float * hc = hu + total;
    for (std::size_t i = 0, at = 0; i < pairs; at += cond[i]->size(), ++i) {
        std::copy(uncond[i]->begin(), uncond[i]->end(), hu + at);
        std::copy(cond[i]->begin(), cond[i]->end(), hc + at);
    }
    ws.dev.upload(hu, 2 * total, nullptr);
    float * du = ws.dev.data();
    check_status(levo_hip_cfg_combine(du + 2 * total, du, du + total, static_cast<int64_t>(total), scale, nullptr));
    check_hip(hipMemcpyAsync(hu + 2 * total, du + 2 * total, total * sizeof(float), hipMemcpyDeviceToHost, nullptr),
              "device-to-host copy");
    synchronize(nullptr);
    for (std::size_t i = 0, at = 0; i < pairs; at += out[i].size(), ++i) {
        std::copy(hu + 2 * total + at, hu + 2 * total + at + out[i].size(), out[i].begin());
    }
}

} // namespace

logits apply_cfg(const logits & conditional, const logits & unconditional, float scale) {
    if (conditional.size() != unconditional.size()) throw std::invalid_argument("CFG logits have different sizes");
    const logits * c = &conditional;
    const logits * u = &unconditional;
    logits out;
    cfg_batch(&c, &u, 1, scale, &out);
    return out;
}

std::vector<logits> apply_cfg(const std::vector<logits> & conditional,
                              const std::vector<logits> & unconditional, float scale) {
    if (conditional.size() != unconditional.size()) throw std::invalid_argument("CFG batch sizes differ");
    // The reference (src/levo-sampling.cpp:30-37) throws at the first pair of
    // different sizes; every pair is checked before any work starts.
    std::vector<const logits *> c(conditional.size()), u(conditional.size());
    for (std::size_t i = 0; i < conditional.size(); ++i) {
        if (conditional[i].size() != unconditional[i].size()) {
            throw std::invalid_argument("CFG logits have different sizes");
        }
        c[i] = &conditional[i];
        u[i] = &unconditional[i];
    }
    std::vector<logits> out(conditional.size());
    cfg_batch(c.data(), u.data(), c.size(), scale, out.data());
    return out;
}

// ---- repetition penalty ---------------------------------------------------------

void apply_unique_token_repetition_penalty(logits & stream_logits, const std::vector<int64_t> & recent_tokens,
                                           float penalty, std::size_t vocabulary_limit) {
    require_penalty(penalty);
    if (stream_logits.empty() || recent_tokens.empty()) return;
    if (recent_tokens.size() > static_cast<std::size_t>(std::numeric_limits<int32_t>::max())) {
        throw std::invalid_argument("LeVo HIP sampler: token list is too long");
    }
    const std::size_t V = stream_logits.size();
    const std::size_t limit = vocabulary_limit == 0 ? V : std::min(vocabulary_limit, V);
    device_buffer<float> d(V);
    device_buffer<int64_t> ids(recent_tokens.size());
    d.upload(stream_logits.data(), V, nullptr);
    ids.upload(recent_tokens.data(), recent_tokens.size(), nullptr);
    check_status(levo_hip_repetition_penalty(d.data(), static_cast<int64_t>(V), ids.data(),
                                             static_cast<int32_t>(recent_tokens.size()), penalty,
                                             static_cast<int64_t>(limit), nullptr));
    d.download(stream_logits.data(), V, nullptr);
    synchronize(nullptr);
}

logits apply_unique_token_repetition_penalty(const logits & stream_logits, const std::vector<int64_t> & recent_tokens,
                                             float penalty, std::size_t vocabulary_limit) {
    logits out = stream_logits;
    apply_unique_token_repetition_penalty(out, recent_tokens, penalty, vocabulary_limit);
    return out;
}

// ---- Sampler --------------------------------------------------------------------

Sampler::Sampler(uint64_t seed) : engine_(seed) {}
Sampler::~Sampler() = default;
Sampler::Sampler(Sampler &&) noexcept = default;
Sampler & Sampler::operator=(Sampler &&) noexcept = default;

void Sampler::seed(uint64_t seed) {
    engine_.seed(seed);
    draws_ = 0;
}

void Sampler::restore(uint64_t seed, uint64_t draw_count) {
    engine_.seed(seed);
    engine_.discard(draw_count);
    draws_ = draw_count;
}

uint64_t Sampler::uniform_bits() {
    ++draws_;
    return engine_();
}

double Sampler::uniform01() { return manual_uniform(engine_, &draws_); }

int64_t Sampler::sample(const logits & input, std::size_t top_k, float temperature, bool use_sampling) {
    if (!workspace_) workspace_ = std::make_unique<sample_workspace>();
    return sample_host_row(*workspace_, input, top_k, temperature, use_sampling, engine_, &draws_, stream_,
                           nullptr, 1.0F, nullptr);
}

std::vector<int64_t> Sampler::sample_streams(const std::vector<logits> & streams, const sampling_config & config,
                                             const std::vector<std::vector<int64_t>> & recent) {
    if (!recent.empty() && recent.size() != streams.size()) throw std::invalid_argument("recent-token stream count differs");
    std::vector<int64_t> out;
    out.reserve(streams.size());
    if (streams.empty()) return out;
    if (!recent.empty()) require_penalty(config.repetition_penalty);
    if (!workspace_) workspace_ = std::make_unique<sample_workspace>();
    sample_workspace & ws = *workspace_;

    const std::size_t V = streams[0].size();
    const bool uniform = std::all_of(streams.begin(), streams.end(), [V](const logits & s) { return s.size() == V; });
    if (!uniform || V == 0 || streams.size() > LEVO_HIP_MAX_STREAMS) {
        // Rows of different lengths: one launch per stream, in order.
        for (std::size_t q = 0; q < streams.size(); ++q) {
            std::vector<int64_t> window;
            if (!recent.empty()) window = trailing(recent[q], config.repetition_window);
            const std::size_t top_k = q == 0 ? config.top_k_mixed : config.top_k_detail;
            out.push_back(sample_host_row(ws, streams[q], top_k, config.temperature, config.use_sampling, engine_,
                                          &draws_, stream_, recent.empty() ? nullptr : &window,
                                          config.repetition_penalty, q == 0 ? &config.ignore_tokens : nullptr));
        }
        return out;
    }

    require_temperature(config.temperature);
    const bool greedy = !config.use_sampling || config.temperature == 0.0F;
    const std::size_t rows = streams.size();
    ws.stage.reserve_discard(rows * V);
    for (std::size_t q = 0; q < rows; ++q) std::copy(streams[q].begin(), streams[q].end(), ws.stage.data() + q * V);
    ws.logits.reserve_discard(rows * V);
    ws.logits.upload(ws.stage.data(), rows * V, stream_);

    levo_hip_sample_args args = base_args();
    args.cond = ws.logits.data();
    args.rows = static_cast<int64_t>(rows);
    args.vocab = static_cast<int64_t>(V);
    args.row_pitch = static_cast<int64_t>(V);
    args.n_streams = static_cast<int32_t>(rows);
    for (std::size_t q = 0; q < rows; ++q) {
        args.top_k[q] = kernel_top_k(q == 0 ? config.top_k_mixed : config.top_k_detail, V);
    }
    std::vector<std::vector<int64_t>> windows;
    for (const auto & history : recent) windows.push_back(trailing(history, config.repetition_window));
    args.penalty_limit = static_cast<int64_t>(V - 1);  // upstream code_size includes EOS; exclude it
    stage_lists(ws, args, windows, config.ignore_tokens, config.repetition_penalty, stream_);
    return sample_rows(ws, args, greedy, config.temperature, engine_, &draws_, stream_);
}

std::vector<int64_t> Sampler::sample_device(const device_logits & batch, const sampling_config & config,
                                            const std::vector<std::vector<int64_t>> & recent) {
    std::vector<int64_t> out;
    if (batch.rows == 0) return out;
    if (batch.vocab == 0) throw std::invalid_argument("cannot sample an empty vocabulary");
    if (batch.streams == 0 || batch.streams > LEVO_HIP_MAX_STREAMS) {
        throw std::invalid_argument("LeVo HIP sampler: stream count must be 1..8");
    }
    if (batch.rows > static_cast<std::size_t>(std::numeric_limits<int32_t>::max())) {
        throw std::invalid_argument("LeVo HIP sampler: too many rows");
    }
    if (!recent.empty() && recent.size() != batch.rows) throw std::invalid_argument("recent-token stream count differs");
    if (!recent.empty()) require_penalty(config.repetition_penalty);
    require_temperature(config.temperature);
    if (!workspace_) workspace_ = std::make_unique<sample_workspace>();
    sample_workspace & ws = *workspace_;
    const bool greedy = !config.use_sampling || config.temperature == 0.0F;

    levo_hip_sample_args args = base_args();
    args.cond = batch.conditional;
    args.uncond = batch.unconditional;
    args.rows = static_cast<int64_t>(batch.rows);
    args.vocab = static_cast<int64_t>(batch.vocab);
    args.row_pitch = static_cast<int64_t>(batch.row_pitch == 0 ? batch.vocab : batch.row_pitch);
    args.cfg_scale = batch.cfg_scale;
    args.n_streams = static_cast<int32_t>(batch.streams);
    for (std::size_t q = 0; q < batch.streams; ++q) {
        args.top_k[q] = kernel_top_k(q == 0 ? config.top_k_mixed : config.top_k_detail, batch.vocab);
    }
    std::vector<std::vector<int64_t>> windows;
    for (const auto & history : recent) windows.push_back(trailing(history, config.repetition_window));
    args.penalty_limit = static_cast<int64_t>(batch.vocab - 1);
    stage_lists(ws, args, windows, config.ignore_tokens, config.repetition_penalty, stream_);
    return sample_rows(ws, args, greedy, config.temperature, engine_, &draws_, stream_);
}

int64_t sample_top_k(const logits & input, std::size_t top_k, float temperature, bool use_sampling,
                     std::mt19937_64 & rng) {
    sample_workspace ws;
    return sample_host_row(ws, input, top_k, temperature, use_sampling, rng, nullptr, nullptr, nullptr, 1.0F,
                           nullptr);
}

} // namespace levo::hip
