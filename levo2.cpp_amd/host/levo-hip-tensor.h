// A view of a device tensor in ggml's conventions, so a ggml caller hands
// over `{t->data, t->type, t->ne, t->nb}` of a backend tensor unchanged.
#pragma once

#include "levo-hip-device.h"

#include <cstddef>
#include <cstdint>

namespace levo::hip {

struct tensor_view {
    void * data = nullptr;                 // device memory
    levo_hip_type type = LEVO_HIP_TYPE_F32;
    int64_t ne[4] = {1, 1, 1, 1};          // elements per dimension, ne[0] innermost
    std::size_t nb[4] = {0, 0, 0, 0};      // byte strides per dimension
};

// Bytes of one element of an F32 / F16 view (0 for block types).
std::size_t element_size(levo_hip_type type) noexcept;

// Contiguous view of an F32 or F16 tensor of shape [ne0, ne1, ne2, ne3].
tensor_view make_tensor_view(void * data, levo_hip_type type, int64_t ne0, int64_t ne1 = 1, int64_t ne2 = 1,
                             int64_t ne3 = 1);

// Rows (ne1 * ne2 * ne3) of ne0 elements packed back to back.
bool is_contiguous(const tensor_view & t) noexcept;

} // namespace levo::hip
