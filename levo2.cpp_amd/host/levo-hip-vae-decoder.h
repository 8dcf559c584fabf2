// levo::detail::vae_decoder (src/levo-vae.h:12-44, src/levo-vae.cpp:157-276)
// over decoder weights already in device memory: the same decode() contract,
// latent [64][frames] channel-major F32 in, audio [2][frames * 1920] out,
// optional stage tensors, cancellation checked when the decode ends, and the
// reference's errors (std::runtime_error("LeVo VAE: ...")). The 31 launches of
// levo_hip_vae_decode run on the decoder's stream; only the latent and the
// audio cross PCIe. decode_device() is the same decode with the latent and the
// audio in device memory.
#pragma once

#include "levo-hip-device.h"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace levo::hip {

struct vae_decode_result {
    std::size_t frames = 0;
    std::size_t samples_per_channel = 0;
    std::vector<float> audio;                        // [2][samples_per_channel]
    std::vector<std::vector<float>> stage_outputs;   // capture_stages: 5 tensors
};

class vae_decoder final {
public:
    static constexpr int64_t latent_dim = 64;
    static constexpr int64_t audio_channels = 2;
    static constexpr int64_t downsampling_ratio = 1920;

    // weights: device pointers that outlive the decoder. Throws
    // std::runtime_error("LeVo VAE: <weight> must be present") as the
    // reference's constructor does (src/levo-vae.cpp:56-78, :157-161).
    explicit vae_decoder(const levo_hip_vae_decoder_weights & weights, stream_t stream = nullptr);

    vae_decoder(const vae_decoder &) = delete;
    vae_decoder & operator=(const vae_decoder &) = delete;

    [[nodiscard]] vae_decode_result decode(const std::vector<float> & latent, std::size_t frames,
                                           bool capture_stages = false,
                                           const cancellation_callback & cancelled = {});

    // latent [64][frames] and audio [2][frames * 1920] in device memory; the
    // latent is not scanned for non-finite values. Enqueued on the decoder's
    // stream; returns without waiting.
    void decode_device(const float * latent, std::size_t frames, float * audio);

    // Width and samples of stage s's output for `frames` latent frames.
    static int64_t stage_width(int stage);
    static int64_t stage_samples(int stage, std::size_t frames);

private:
    void reserve(std::size_t frames);

    levo_hip_vae_decoder_weights weights_;
    stream_t stream_;
    device_buffer<float> workspace_;
    device_buffer<float> latent_;
    device_buffer<float> audio_;
    device_buffer<float> stages_;
};

} // namespace levo::hip
