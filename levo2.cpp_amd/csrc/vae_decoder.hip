// The Oobleck VAE decoder of vae_decoder::decode (src/levo-vae.cpp:172-276)
// as a sequence of fused launches on one stream, every activation in HBM:
//   input conv (64 -> 2048, k 7, padding 3)
//   5 x [SnakeBeta + ConvTranspose1d upsample (stride s, kernel 2s,
//        padding (s + 1) / 2) + 3 residual units (SnakeBeta + conv k 7 at
//        dilation 1 / 3 / 9, SnakeBeta + conv k 1, + input)]
//   SnakeBeta + output conv (128 -> 2, k 7, padding 3, no bias)
// with the reference's fixed hyper-parameters (src/levo-vae-model.h:18-33,
// decode order: strides 10, 6, 4, 4, 2; widths 2048 -> 1024 -> 512 -> 256
// -> 128 -> 128). Host code only: it orders levo_hip_snake_conv1d,
// levo_hip_snake_conv_transpose1d and residual-unit launches over three
// workspace buffers. A residual unit at 128 channels (stages 4 and 5) is one
// launch: the k = 1 conv runs in the k = 7 conv's epilogue.
#include "common.hpp"

#include <algorithm>
#include <utility>

namespace levo_hip {
namespace {

constexpr int64_t kLatent = 64;
constexpr int64_t kAudio = 2;
constexpr int64_t kStrides[5] = {10, 6, 4, 4, 2};
constexpr int64_t kInWidth[5] = {2048, 1024, 512, 256, 128};
constexpr int64_t kOutWidth[5] = {1024, 512, 256, 128, 128};
constexpr int64_t kDilations[3] = {1, 3, 9};

// Largest channels x samples of any activation: the last stage's 128 x 1920 T.
int64_t buffer_floats(int64_t frames) {
    int64_t n = kInWidth[0] * frames;
    int64_t len = frames;
    for (int i = 0; i < 5; ++i) {
        len *= kStrides[i];
        n = std::max(n, kOutWidth[i] * len);
    }
    return (n + 63) / 64 * 64;  // 256-byte aligned thirds
}

// The first weight validate_weights (src/levo-vae.cpp:56-78) would reject as
// absent, in its order, or nullptr when every one is present.
const char * missing_weight(const levo_hip_vae_decoder_weights & w) {
    const auto snake = [](const levo_hip_vae_snake & v) -> const char * {
        if (v.alpha_log == nullptr) return "SnakeBeta alpha";
        if (v.beta_log == nullptr) return "SnakeBeta beta";
        return nullptr;
    };
    const auto conv = [](const levo_hip_vae_conv & v) -> const char * {
        if (v.weight == nullptr) return "convolution weight";
        if (v.bias == nullptr) return "convolution bias";
        return nullptr;
    };
    const char * m = conv(w.input);
    for (int s = 0; m == nullptr && s < 5; ++s) {
        const levo_hip_vae_stage & sg = w.stage[s];
        if ((m = snake(sg.activation)) || (m = conv(sg.upsample))) break;
        for (int r = 0; m == nullptr && r < 3; ++r) {
            const levo_hip_vae_residual & ru = sg.residual[r];
            if (!(m = snake(ru.pre)) && !(m = conv(ru.conv_0)) && !(m = snake(ru.post))) m = conv(ru.conv_1);
        }
    }
    if (m == nullptr) m = snake(w.output_activation);
    if (m == nullptr && w.output_weight == nullptr) m = "output convolution weight";
    return m;
}

bool weights_present(const levo_hip_vae_decoder_weights & w) { return missing_weight(w) == nullptr; }

// The free tail of a decoder buffer of n floats whose first `used` floats
// hold a tensor: workspace for a split-K convolution writing that tensor.
struct tail {
    float * p;
    int64_t floats;
};
tail tail_of(float * buf, int64_t n, int64_t used) {
    const int64_t start = (used + 63) / 64 * 64;  // 256-byte aligned
    return start < n ? tail{buf + start, n - start} : tail{nullptr, 0};
}

// run_residual (src/levo-vae.cpp:91-100); conv_0 writes h, conv_1 writes y.
// Inside the decoder (post_in_h): conv_0 stores snake_post(h), computed once
// per sample in its epilogue, and conv_1 reads it without a SnakeBeta of its
// own (the same F32 values the k = 1 conv's staging would compute from h),
// and both convolutions take the split-K path with the free tails of the
// decoder's h and y buffers. The public unit keeps h = conv_0's output.
int residual_unit(const float * x, int64_t c, int64_t len, const levo_hip_vae_residual & u, int64_t dilation,
                  levo_hip_type pt, float * y, float * h, bool post_in_h, tail ws_h, tail ws_y,
                  levo_hip_stream_t stream) {
    const int fused = launch_residual_unit_fused(x, c, len, u.pre.alpha_log, u.pre.beta_log, u.conv_0.weight,
                                                 u.conv_0.bias, u.post.alpha_log, u.post.beta_log, u.conv_1.weight,
                                                 u.conv_1.bias, dilation, pt, y, as_hip(stream));
    if (fused != kNotFused) return fused;
    const bool post = post_in_h && u.post.alpha_log != nullptr && u.post.beta_log != nullptr && c > 4;
    int st;
    if (post) {
        st = snake_conv1d_post(x, c, len, u.pre.alpha_log, u.pre.beta_log, pt, u.conv_0.weight, c, 7, u.conv_0.bias,
                               3 * dilation, dilation, h, u.post.alpha_log, u.post.beta_log, ws_h.p, ws_h.floats,
                               as_hip(stream));
    } else {
        st = levo_hip_snake_conv1d_split(x, len, c, len, u.pre.alpha_log, u.pre.beta_log, pt, u.conv_0.weight, c, 7,
                                         u.conv_0.bias, 3 * dilation, dilation, nullptr, 0, h, len, ws_h.p,
                                         ws_h.floats, stream);
    }
    if (st != LEVO_HIP_OK) return st;
    return levo_hip_snake_conv1d_split(h, len, c, len, post ? nullptr : u.post.alpha_log,
                                       post ? nullptr : u.post.beta_log, pt, u.conv_1.weight, c, 1, u.conv_1.bias, 0,
                                       1, x, len, y, len, ws_y.p, ws_y.floats, stream);
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int64_t levo_hip_vae_decode_workspace_bytes(int64_t frames) {
    if (frames <= 0 || frames > (int64_t{1} << 24)) return -1;
    return 3 * buffer_floats(frames) * static_cast<int64_t>(sizeof(float));
}

extern "C" int levo_hip_vae_validate_weights(const levo_hip_vae_decoder_weights * w) {
    clear_error();
    LEVO_REQUIRE(w != nullptr, "vae_decode: null weights");
    LEVO_REQUIRE(w->param_type == LEVO_HIP_TYPE_F32 || w->param_type == LEVO_HIP_TYPE_F16,
                 "vae_decode: SnakeBeta parameters must be F32 or F16");
    LEVO_REQUIRE(weights_present(*w), "vae_decode: %s must be present", missing_weight(*w));
    return LEVO_HIP_OK;
}

extern "C" int levo_hip_vae_residual_unit(const float * x, int64_t channels, int64_t time,
                                          const levo_hip_vae_residual * unit, int64_t dilation,
                                          levo_hip_type param_type, float * y, float * h,
                                          levo_hip_stream_t stream) {
    LEVO_REQUIRE(unit != nullptr, "vae_residual_unit: null unit");
    LEVO_REQUIRE(param_type == LEVO_HIP_TYPE_F32 || param_type == LEVO_HIP_TYPE_F16,
                 "vae_residual_unit: SnakeBeta parameters must be F32 or F16");
    LEVO_REQUIRE(x != nullptr && y != nullptr && h != nullptr, "vae_residual_unit: null tensor");
    LEVO_REQUIRE(unit->conv_0.weight != nullptr && unit->conv_1.weight != nullptr,
                 "vae_residual_unit: null convolution weight");
    // time < 2^37: ceil(time / 128) sample tiles stay far inside a 32-bit grid
    LEVO_REQUIRE(channels > 0 && time > 0 && channels <= (1 << 20) && time < (int64_t{1} << 37),
                 "vae_residual_unit: invalid shape");
    LEVO_REQUIRE(dilation > 0 && dilation < (1 << 16), "vae_residual_unit: invalid dilation");
    const uintptr_t xb = reinterpret_cast<uintptr_t>(x);
    const uintptr_t yb = reinterpret_cast<uintptr_t>(y);
    const uintptr_t n = static_cast<uintptr_t>(channels * time) * sizeof(float);
    LEVO_REQUIRE(yb + n <= xb || xb + n <= yb, "vae_residual_unit: y must not overlap x");
    return residual_unit(x, channels, time, *unit, dilation, param_type, y, h, false, tail{nullptr, 0},
                         tail{nullptr, 0}, stream);
}

extern "C" int levo_hip_vae_decode(const levo_hip_vae_decoder_weights * w, const float * latent, int64_t frames,
                                   float * audio, float * const * stage_outputs, void * workspace,
                                   int64_t workspace_bytes, levo_hip_stream_t stream) {
    const int valid = levo_hip_vae_validate_weights(w);
    if (valid != LEVO_HIP_OK) return valid;
    LEVO_REQUIRE(frames > 0 && frames <= (int64_t{1} << 24), "latent frame count must be positive and representable");
    LEVO_REQUIRE(latent != nullptr && audio != nullptr && workspace != nullptr, "vae_decode: null tensor");
    LEVO_REQUIRE(aligned16(workspace), "vae_decode: workspace must be 16-byte aligned");
    LEVO_REQUIRE(workspace_bytes >= levo_hip_vae_decode_workspace_bytes(frames),
                 "vae_decode: workspace smaller than levo_hip_vae_decode_workspace_bytes");
    const int64_t n = buffer_floats(frames);
    float * a = static_cast<float *>(workspace);
    float * b = a + n;
    float * h = b + n;
    const levo_hip_type pt = w->param_type;
    int st;
#define LEVO_STEP(call)                   \
    do {                                  \
        st = (call);                      \
        if (st != LEVO_HIP_OK) return st; \
    } while (0)
    // input projection: no SnakeBeta in front (src/levo-vae.cpp:219-221)
    const tail ws_in = tail_of(a, n, kInWidth[0] * frames);
    LEVO_STEP(levo_hip_snake_conv1d_split(latent, frames, kLatent, frames, nullptr, nullptr, pt, w->input.weight,
                                          kInWidth[0], 7, w->input.bias, 3, 1, nullptr, 0, a, frames, ws_in.p,
                                          ws_in.floats, stream));
    int64_t len = frames;
    for (int s = 0; s < 5; ++s) {
        const levo_hip_vae_stage & sg = w->stage[s];
        const int64_t stride = kStrides[s];
        const int64_t out_len = len * stride;  // (len + 1) s - 2 ((s + 1) / 2) for even s
        const tail ws_up = tail_of(b, n, kOutWidth[s] * out_len);
        LEVO_STEP(levo_hip_snake_conv_transpose1d_split(a, len, kInWidth[s], len, sg.activation.alpha_log,
                                                        sg.activation.beta_log, pt, sg.upsample.weight,
                                                        kOutWidth[s], stride, sg.upsample.bias, (stride + 1) / 2, b,
                                                        out_len, ws_up.p, ws_up.floats, stream));
        len = out_len;
        const int64_t c = kOutWidth[s];
        // residual units: x in b, y into a (free since the upsample read it),
        // then the two swap
        for (int r = 0; r < 3; ++r) {
            LEVO_STEP(residual_unit(b, c, len, sg.residual[r], kDilations[r], pt, a, h, true, tail_of(h, n, c * len),
                                    tail_of(a, n, c * len), stream));
            std::swap(a, b);
        }
        if (stage_outputs != nullptr && stage_outputs[s] != nullptr) {
            const hipError_t e = hipMemcpyAsync(stage_outputs[s], b, sizeof(float) * c * len,
                                                hipMemcpyDeviceToDevice, as_hip(stream));
            if (e != hipSuccess) {
                set_error("vae_decode: stage %d copy: %s", s, hipGetErrorString(e));
                return LEVO_HIP_ERR_RUNTIME;
            }
        }
        std::swap(a, b);
    }
    // output: SnakeBeta + conv 128 -> 2, no bias (src/levo-vae.cpp:258-262)
    LEVO_STEP(levo_hip_snake_conv1d(a, len, kOutWidth[4], len, w->output_activation.alpha_log,
                                    w->output_activation.beta_log, pt, w->output_weight, kAudio, 7, nullptr, 3, 1,
                                    nullptr, 0, audio, len, stream));
#undef LEVO_STEP
    return LEVO_HIP_OK;
}
