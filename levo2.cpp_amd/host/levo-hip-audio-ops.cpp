// levo::hip::detail::snake_beta over levo_hip_snake_beta, with the checks of
// src/levo-audio-ops.cpp:10-30, 129-141.
#include "levo-hip-audio-ops.h"

#include <stdexcept>
#include <string>

namespace levo::hip::detail {
namespace {

[[noreturn]] void fail(const std::string & message) {
    throw std::invalid_argument("LeVo audio graph: " + message);
}

void require_f32(const tensor_view * t, const char * name) {
    if (t == nullptr) fail(std::string(name) + " is null");
    if (t->type != LEVO_HIP_TYPE_F32) fail(std::string(name) + " must be F32");
}

void require_weight(const tensor_view * t, const char * name) {
    if (t == nullptr) fail(std::string(name) + " is null");
    if (t->type != LEVO_HIP_TYPE_F32 && t->type != LEVO_HIP_TYPE_F16) fail(std::string(name) + " must be F32 or F16");
}

bool same_shape(const tensor_view & a, const tensor_view & b) {
    for (int d = 0; d < 4; ++d) {
        if (a.ne[d] != b.ne[d]) return false;
    }
    return true;
}

} // namespace

void snake_beta(const tensor_view * input, const tensor_view * alpha_log, const tensor_view * beta_log,
                const tensor_view * output, stream_t stream) {
    require_f32(input, "SnakeBeta input");
    require_weight(alpha_log, "SnakeBeta alpha_log");
    require_weight(beta_log, "SnakeBeta beta_log");
    const auto valid_parameter = [input](const tensor_view * p) {
        return p->ne[0] == 1 && p->ne[1] == input->ne[1] && p->ne[2] == 1 && p->ne[3] == 1;
    };
    if (!valid_parameter(alpha_log) || !valid_parameter(beta_log)) {
        fail("SnakeBeta parameters must have shape [1, channels, 1]");
    }
    require_f32(output, "SnakeBeta output");
    if (!same_shape(*input, *output)) fail("SnakeBeta output must have the input shape");
    const int64_t T = input->ne[0];
    const int64_t C = input->ne[1];
    if (T == 0 || C == 0 || input->ne[2] == 0 || input->ne[3] == 0) return;
    if (input->nb[0] != sizeof(float) || output->nb[0] != sizeof(float) || input->nb[1] % sizeof(float) != 0 ||
        output->nb[1] % sizeof(float) != 0) {
        fail("SnakeBeta rows must be contiguous in time");
    }
    for (const tensor_view * p : {alpha_log, beta_log}) {
        if (C > 1 && p->nb[1] != element_size(p->type)) fail("SnakeBeta parameters must be contiguous");
        if (p->data == nullptr) fail("SnakeBeta parameter data is null");
    }
    if (input->data == nullptr || output->data == nullptr) fail("SnakeBeta tensor data is null");

    // Mixed parameter types: widen the F16 one to F32 (exact, as the
    // reference's ggml_cast to F32), so one kernel type serves both.
    const void * a = alpha_log->data;
    const void * b = beta_log->data;
    levo_hip_type ptype = alpha_log->type;
    device_buffer<float> widened;
    if (alpha_log->type != beta_log->type) {
        widened.reserve_discard(static_cast<std::size_t>(C));
        const tensor_view * half = alpha_log->type == LEVO_HIP_TYPE_F16 ? alpha_log : beta_log;
        check_status(levo_hip_fp16_to_fp32_row(static_cast<const uint16_t *>(half->data), widened.data(), C, stream));
        if (half == alpha_log) a = widened.data();
        else b = widened.data();
        ptype = LEVO_HIP_TYPE_F32;
    }

    const int64_t xs = static_cast<int64_t>(input->nb[1] / sizeof(float));
    const int64_t ys = static_cast<int64_t>(output->nb[1] / sizeof(float));
    for (int64_t i3 = 0; i3 < input->ne[3]; ++i3) {
        for (int64_t i2 = 0; i2 < input->ne[2]; ++i2) {
            const auto * x = reinterpret_cast<const float *>(static_cast<const char *>(input->data) +
                                                             i2 * input->nb[2] + i3 * input->nb[3]);
            auto * y = reinterpret_cast<float *>(static_cast<char *>(output->data) + i2 * output->nb[2] +
                                                 i3 * output->nb[3]);
            check_status(levo_hip_snake_beta(x, xs, a, b, ptype, y, ys, C, T, stream));
        }
    }
    if (widened.data()) synchronize(stream);  // keep the widened copy alive until the kernels ran
}

} // namespace levo::hip::detail
