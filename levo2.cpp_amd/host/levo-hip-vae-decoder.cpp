#include "levo-hip-vae-decoder.h"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <string>

namespace levo::hip {
namespace {

constexpr int64_t kStrides[5] = {10, 6, 4, 4, 2};
constexpr int64_t kWidths[5] = {1024, 512, 256, 128, 128};

[[noreturn]] void fail(const std::string & message) { throw std::runtime_error("LeVo VAE: " + message); }

// A failing C ABI status as the reference's error: "LeVo VAE: <message>".
void check_vae(int status) {
    if (status == LEVO_HIP_OK) return;
    std::string message = levo_hip_last_error();
    const std::string prefix = "vae_decode: ";
    if (message.compare(0, prefix.size(), prefix) == 0) message.erase(0, prefix.size());
    fail(message);
}

} // namespace

int64_t vae_decoder::stage_width(int stage) { return kWidths[stage]; }

int64_t vae_decoder::stage_samples(int stage, std::size_t frames) {
    int64_t n = static_cast<int64_t>(frames);
    for (int s = 0; s <= stage; ++s) n *= kStrides[s];
    return n;
}

vae_decoder::vae_decoder(const levo_hip_vae_decoder_weights & weights, stream_t stream)
    : weights_(weights), stream_(stream) {
    check_vae(levo_hip_vae_validate_weights(&weights_));
}

void vae_decoder::reserve(std::size_t frames) {
    const int64_t bytes = levo_hip_vae_decode_workspace_bytes(static_cast<int64_t>(frames));
    if (bytes < 0) fail("latent frame count must be positive and representable");
    workspace_.reserve_discard(static_cast<std::size_t>(bytes) / sizeof(float));
}

void vae_decoder::decode_device(const float * latent, std::size_t frames, float * audio) {
    if (frames == 0 || frames > static_cast<std::size_t>(std::numeric_limits<int64_t>::max())) {
        fail("latent frame count must be positive and representable");
    }
    reserve(frames);
    check_vae(levo_hip_vae_decode(&weights_, latent, static_cast<int64_t>(frames), audio, nullptr, workspace_.data(),
                                  static_cast<int64_t>(workspace_.size() * sizeof(float)), stream_));
}

vae_decode_result vae_decoder::decode(const std::vector<float> & latent, std::size_t frames, bool capture_stages,
                                      const cancellation_callback & cancelled) {
    // The reference's host-side checks, in its order (src/levo-vae.cpp:177-191).
    if (frames == 0 || frames > static_cast<std::size_t>(std::numeric_limits<int64_t>::max())) {
        fail("latent frame count must be positive and representable");
    }
    if (frames > std::numeric_limits<std::size_t>::max() / latent_dim || latent.size() != frames * latent_dim) {
        fail("latent payload does not have shape [64,frames]");
    }
    if (frames > std::numeric_limits<std::size_t>::max() / downsampling_ratio) {
        fail("decoded sample count overflows size_t");
    }
    for (const float value : latent) {
        if (!std::isfinite(value)) fail("latent payload contains a non-finite value");
    }
    reserve(frames);
    const std::size_t samples = frames * downsampling_ratio;
    latent_.reserve_discard(latent.size());
    audio_.reserve_discard(audio_channels * samples);
    float * stage_ptr[5] = {};
    if (capture_stages) {
        std::size_t total = 0;
        for (int s = 0; s < 5; ++s) total += stage_width(s) * stage_samples(s, frames);
        stages_.reserve_discard(total);
        std::size_t at = 0;
        for (int s = 0; s < 5; ++s) {
            stage_ptr[s] = stages_.data() + at;
            at += stage_width(s) * stage_samples(s, frames);
        }
    }
    latent_.upload(latent.data(), latent.size(), stream_);
    check_vae(levo_hip_vae_decode(&weights_, latent_.data(), static_cast<int64_t>(frames), audio_.data(),
                                  capture_stages ? stage_ptr : nullptr, workspace_.data(),
                                  static_cast<int64_t>(workspace_.size() * sizeof(float)), stream_));
    vae_decode_result result;
    result.frames = frames;
    result.samples_per_channel = samples;
    result.audio.resize(audio_channels * samples);
    audio_.download(result.audio.data(), result.audio.size(), stream_);
    if (capture_stages) {
        result.stage_outputs.resize(5);
        for (int s = 0; s < 5; ++s) {
            auto & out = result.stage_outputs[s];
            out.resize(stage_width(s) * stage_samples(s, frames));
            check_hip(hipMemcpyAsync(out.data(), stage_ptr[s], out.size() * sizeof(float), hipMemcpyDeviceToHost,
                                     stream_),
                      "device-to-host copy");
        }
    }
    synchronize(stream_);
    // The reference honours a stop once its graph ends (src/levo-vae.cpp:252-254).
    if (cancelled && cancelled()) throw operation_cancelled();
    return result;
}

} // namespace levo::hip
