// Fused residual add + RMSNorm / LayerNorm on device tensor views, standing in
// for the ggml op compositions of the LeLM and the Flow estimator:
//   LeLM F16 activations: round_f16(ggml_add(x, delta)) then rms_norm_weighted
//     (src/levo-kv.cpp:153-160, :462, :507)
//   LeLM F32: ggml_mul(ggml_rms_norm(h, eps), weight) (src/levo-lm.cpp:131-137)
//   Flow estimator: ggml_add(ggml_mul(ggml_norm(h, eps), gamma), beta)
//     (src/levo-flow-estimator.cpp:106-109) after its residual adds (:221-247),
//     and with the gated residual and the AdaLN modulation around it (:89-93)
// Errors are std::invalid_argument("LeVo HIP norm: ...").
#pragma once

#include "levo-hip-tensor.h"

namespace levo::hip {

// x, delta, h_out, y: F32 or F16 (all the same type) of shape [dim, rows...],
// contiguous. delta and h_out may be null (h = x; h not stored). weight: [dim]
// F32 or F16 (F16 activations need an F16 weight, as the LeLM stores it).
void residual_rms_norm(const tensor_view * x, const tensor_view * delta, const tensor_view * weight, float eps,
                       const tensor_view * h_out, const tensor_view * y, stream_t stream = nullptr);

// As above with y = norm(h, eps) * gamma + beta; gamma and beta share a type.
void residual_layer_norm(const tensor_view * x, const tensor_view * delta, const tensor_view * gamma,
                         const tensor_view * beta, float eps, const tensor_view * h_out, const tensor_view * y,
                         stream_t stream = nullptr);

// One per-batch modulation vector of the Flow estimator (modulation_chunk,
// src/levo-flow-estimator.cpp:95-104): dynamic is an F32 [dim, batch] view
// whose batch entries lie nb[1] bytes apart (the ggml_view_2d of the time
// modulation), learned an F32 [dim] vector added to every entry, or null. A
// vector with a null dynamic is absent.
struct batch_vector_view {
    const tensor_view * dynamic = nullptr;
    const tensor_view * learned = nullptr;
};

// A Flow estimator block boundary in one pass (src/levo-flow-estimator.cpp:
// 221-233, 243-261): h = ggml_add(ggml_mul(delta, gate), x); then
// y = add_scale_shift(layer_norm(h, gamma, beta), scale, shift) (:89-93,
// :106-109). x, delta, h_out, y: F32 [dim, frames, batch] contiguous; row
// (frame f, batch b) takes entry b of gate / scale / shift. delta null: h = x;
// gate absent: h = x + delta; scale and shift absent together: y is the
// LayerNorm. gamma / beta: [dim] F32 or F16.
void residual_layer_norm_modulated(const tensor_view * x, const tensor_view * delta,
                                   const batch_vector_view & gate, const tensor_view * gamma,
                                   const tensor_view * beta, const batch_vector_view & scale,
                                   const batch_vector_view & shift, float eps, const tensor_view * h_out,
                                   const tensor_view * y, stream_t stream = nullptr);

} // namespace levo::hip
