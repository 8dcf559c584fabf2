#include "sample_draw.hpp"

namespace levo_hip {
namespace {

// One wave per row; no LDS, no barriers.
__global__ __launch_bounds__(64) void sample_draw_kernel(const levo_hip_draw_args a) { draw_row(a, blockIdx.x); }

}  // namespace
}  // namespace levo_hip


using namespace levo_hip;

extern "C" int levo_hip_sample_draw(const levo_hip_draw_args * args, levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "sample_draw: null argument block");
    const levo_hip_draw_args & a = *args;
    LEVO_REQUIRE(a.rows >= 0 && a.rows < (int64_t{1} << 31), "sample_draw: row count out of range");
    if (a.rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(__builtin_isfinite(a.temperature) && a.temperature >= 0.0f,
                 "temperature must be finite and non-negative");
    LEVO_REQUIRE(a.capacity >= 1, "sample_draw: candidate capacity must be positive");
    LEVO_REQUIRE(a.best != nullptr && a.count != nullptr && a.cand_ids != nullptr && a.cand_logits != nullptr &&
                     a.row_max != nullptr,
                 "sample_draw: null candidate input");
    LEVO_REQUIRE(a.tokens != nullptr && a.draws != nullptr, "sample_draw: null output");
    LEVO_REQUIRE(a.bits != nullptr || a.use_sampling == 0 || a.temperature == 0.0f,
                 "sample_draw: null uniform bits");
    sample_draw_kernel<<<static_cast<uint32_t>(a.rows), 64, 0, as_hip(stream)>>>(a);
    return launch_status("levo_hip_sample_draw");
}
