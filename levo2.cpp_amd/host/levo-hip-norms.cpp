#include "levo-hip-norms.h"

#include <stdexcept>
#include <string>

namespace levo::hip {
namespace {

[[noreturn]] void fail(const std::string & message) {
    throw std::invalid_argument("LeVo HIP norm: " + message);
}

bool same_shape(const tensor_view & a, const tensor_view & b) {
    for (int d = 0; d < 4; ++d) {
        if (a.ne[d] != b.ne[d]) return false;
    }
    return true;
}

// Checks the activation tensors and returns the row count.
int64_t check_activations(const tensor_view * x, const tensor_view * delta, const tensor_view * h_out,
                          const tensor_view * y) {
    if (x == nullptr || y == nullptr) fail("input and output are required");
    if (x->type != LEVO_HIP_TYPE_F32 && x->type != LEVO_HIP_TYPE_F16) fail("activations must be F32 or F16");
    for (const tensor_view * t : {delta, h_out, y}) {
        if (t == nullptr) continue;
        if (t->type != x->type) fail("activation tensors must share one type");
        if (!same_shape(*t, *x)) fail("activation tensors must share one shape");
        if (!is_contiguous(*t)) fail("activation tensors must be contiguous");
    }
    if (!is_contiguous(*x)) fail("activation tensors must be contiguous");
    return x->ne[1] * x->ne[2] * x->ne[3];
}

void check_param(const tensor_view * p, const tensor_view * x, const char * name) {
    if (p == nullptr) fail(std::string(name) + " is null");
    if (p->type != LEVO_HIP_TYPE_F32 && p->type != LEVO_HIP_TYPE_F16) fail(std::string(name) + " must be F32 or F16");
    if (p->ne[0] != x->ne[0] || p->ne[1] * p->ne[2] * p->ne[3] != 1) fail(std::string(name) + " must have shape [dim]");
    if (!is_contiguous(*p)) fail(std::string(name) + " must be contiguous");
}

const void * data_or_null(const tensor_view * t) { return t ? t->data : nullptr; }
void * data_or_null_mut(const tensor_view * t) { return t ? t->data : nullptr; }

} // namespace

void residual_rms_norm(const tensor_view * x, const tensor_view * delta, const tensor_view * weight, float eps,
                       const tensor_view * h_out, const tensor_view * y, stream_t stream) {
    const int64_t rows = check_activations(x, delta, h_out, y);
    check_param(weight, x, "weight");
    check_status(levo_hip_residual_rms_norm(x->type, x->data, data_or_null(delta), weight->data, weight->type,
                                            data_or_null_mut(h_out), y->data, rows, x->ne[0], eps, stream));
}

void residual_layer_norm(const tensor_view * x, const tensor_view * delta, const tensor_view * gamma,
                         const tensor_view * beta, float eps, const tensor_view * h_out, const tensor_view * y,
                         stream_t stream) {
    const int64_t rows = check_activations(x, delta, h_out, y);
    check_param(gamma, x, "gamma");
    check_param(beta, x, "beta");
    if (gamma->type != beta->type) fail("gamma and beta must share one type");
    check_status(levo_hip_residual_layer_norm(x->type, x->data, data_or_null(delta), gamma->data, beta->data,
                                              gamma->type, data_or_null_mut(h_out), y->data, rows, x->ne[0], eps,
                                              stream));
}

namespace {

// levo_hip_batch_vector of a view; `batches` entries of `dim` values.
levo_hip_batch_vector batch_vector(const batch_vector_view & v, int64_t dim, int64_t batches, const char * name) {
    levo_hip_batch_vector out{nullptr, 0, nullptr};
    if (v.dynamic == nullptr) {
        if (v.learned != nullptr) fail(std::string(name) + ": a learned part needs a dynamic part");
        return out;
    }
    const tensor_view & d = *v.dynamic;
    if (d.type != LEVO_HIP_TYPE_F32) fail(std::string(name) + " must be F32");
    if (d.ne[0] != dim || d.ne[1] * d.ne[2] * d.ne[3] != batches) {
        fail(std::string(name) + " must have shape [dim, batch]");
    }
    if (d.nb[0] != sizeof(float) || d.nb[1] % sizeof(float) != 0) fail(std::string(name) + " rows must be dense floats");
    if (d.ne[1] > 1 && d.ne[2] * d.ne[3] != 1) fail(std::string(name) + " must be two-dimensional");
    out.dynamic = static_cast<const float *>(d.data);
    out.stride = d.ne[1] > 1 ? static_cast<int64_t>(d.nb[1] / sizeof(float)) : dim;
    if (v.learned != nullptr) {
        const tensor_view & l = *v.learned;
        if (l.type != LEVO_HIP_TYPE_F32 || l.ne[0] != dim || l.ne[1] * l.ne[2] * l.ne[3] != 1 || !is_contiguous(l)) {
            fail(std::string(name) + ": the learned part must be an F32 [dim] vector");
        }
        out.learned = static_cast<const float *>(l.data);
    }
    return out;
}

} // namespace

void residual_layer_norm_modulated(const tensor_view * x, const tensor_view * delta, const batch_vector_view & gate,
                                   const tensor_view * gamma, const tensor_view * beta,
                                   const batch_vector_view & scale, const batch_vector_view & shift, float eps,
                                   const tensor_view * h_out, const tensor_view * y, stream_t stream) {
    const int64_t rows = check_activations(x, delta, h_out, y);
    if (x->type != LEVO_HIP_TYPE_F32) fail("the modulated LayerNorm takes F32 activations");
    check_param(gamma, x, "gamma");
    check_param(beta, x, "beta");
    if (gamma->type != beta->type) fail("gamma and beta must share one type");
    if ((scale.dynamic == nullptr) != (shift.dynamic == nullptr)) fail("scale and shift come together");
    if (gate.dynamic != nullptr && delta == nullptr) fail("a gate needs delta");
    const int64_t dim = x->ne[0];
    const int64_t batches = x->ne[2] * x->ne[3];
    levo_hip_modulated_norm_args a{};
    a.x = static_cast<const float *>(x->data);
    a.delta = delta ? static_cast<const float *>(delta->data) : nullptr;
    a.gate = batch_vector(gate, dim, batches, "gate");
    a.gamma = gamma->data;
    a.beta = beta->data;
    a.param_type = gamma->type;
    a.scale = batch_vector(scale, dim, batches, "scale");
    a.shift = batch_vector(shift, dim, batches, "shift");
    a.h_out = h_out ? static_cast<float *>(h_out->data) : nullptr;
    a.y = static_cast<float *>(y->data);
    a.rows = rows;
    a.rows_per_batch = x->ne[1];
    a.dim = dim;
    a.eps = eps;
    check_status(levo_hip_residual_layer_norm_modulated(&a, stream));
}

} // namespace levo::hip
