#include "levo-hip-tensor.h"

namespace levo::hip {

std::size_t element_size(levo_hip_type type) noexcept {
    switch (type) {
        case LEVO_HIP_TYPE_F32: return 4;
        case LEVO_HIP_TYPE_F16: return 2;
        default: return 0;
    }
}

tensor_view make_tensor_view(void * data, levo_hip_type type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    tensor_view t;
    t.data = data;
    t.type = type;
    t.ne[0] = ne0;
    t.ne[1] = ne1;
    t.ne[2] = ne2;
    t.ne[3] = ne3;
    t.nb[0] = element_size(type);
    for (int d = 1; d < 4; ++d) t.nb[d] = t.nb[d - 1] * static_cast<std::size_t>(t.ne[d - 1]);
    return t;
}

bool is_contiguous(const tensor_view & t) noexcept {
    std::size_t expected = element_size(t.type);
    if (expected == 0) return false;
    for (int d = 0; d < 4; ++d) {
        if (t.ne[d] > 1 && t.nb[d] != expected) return false;
        expected *= static_cast<std::size_t>(t.ne[d]);
    }
    return true;
}

} // namespace levo::hip
