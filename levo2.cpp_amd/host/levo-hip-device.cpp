#include "levo-hip-device.h"

namespace levo::hip {

void check_hip(hipError_t status, const char * what) {
    if (status != hipSuccess) {
        throw std::runtime_error(std::string("LeVo HIP: ") + what + ": " + hipGetErrorString(status));
    }
}

int64_t check_status(int64_t status, error_kind kind) {
    if (status >= 0) return status;
    const std::string message = levo_hip_last_error();
    if (status == LEVO_HIP_ERR_RUNTIME || kind == error_kind::runtime_error) throw std::runtime_error(message);
    throw std::invalid_argument(message);
}

void synchronize(stream_t stream) { check_hip(hipStreamSynchronize(stream), "stream synchronize"); }

} // namespace levo::hip
