// Drop-in for the VAE's SnakeBeta builder, levo::detail::snake_beta
// (src/levo-audio-ops.h:28-33, src/levo-audio-ops.cpp:125-152).
//
// The reference returns a ggml node for the chain exp -> scale_bias -> mul ->
// sin -> sqr -> div -> add; this version executes the same arithmetic as one
// fused gfx950 kernel on device tensor views (one read of x, one write of y),
// enqueued on `stream`. Validation and messages follow the reference:
// std::invalid_argument("LeVo audio graph: ...").
#pragma once

#include "levo-hip-tensor.h"

namespace levo::hip::detail {

// y = x + sin(x * exp(alpha_log))^2 / (exp(beta_log) + 1e-9) per channel.
// input / output: F32 [time, channels, batch, 1] in ggml order, each time row
// contiguous (nb[0] == 4); output may alias input. alpha_log / beta_log: F32
// or F16 of shape [1, channels, 1, 1], F16 promoted exactly to F32.
void snake_beta(const tensor_view * input, const tensor_view * alpha_log, const tensor_view * beta_log,
                const tensor_view * output, stream_t stream = nullptr);

} // namespace levo::hip::detail
