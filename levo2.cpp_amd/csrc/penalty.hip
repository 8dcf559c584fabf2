// Unique-token repetition penalty on one logits row, in place:
// every distinct id of `recent` inside [0, limit) has its logit divided once
// by `penalty`, however often it occurs (src/levo-sampling.cpp:39-47).
//
// One workgroup. Each id claims a bit of an LDS bitmap with atomicOr; only the
// thread that set the bit divides, so duplicates divide once. Limits beyond
// the bitmap fall back to a first-occurrence scan over the window.
#include "common.hpp"

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int64_t kBitmapIds = int64_t{1} << 19;  // 64 KiB of LDS
constexpr int kBitmapWords = static_cast<int>(kBitmapIds / 32);

__global__ __launch_bounds__(kThreads) void penalty_bitmap_kernel(float * logits, const int64_t * recent,
                                                                  int32_t n, float penalty, int64_t limit) {
    __shared__ uint32_t seen[kBitmapWords];
    const int words = static_cast<int>((limit + 31) / 32);
    for (int w = threadIdx.x; w < words; w += kThreads) seen[w] = 0u;
    __syncthreads();
    for (int j = threadIdx.x; j < n; j += kThreads) {
        const int64_t id = recent[j];
        if (id < 0 || id >= limit) continue;
        const uint32_t bit = 1u << (id & 31);
        const uint32_t old = atomicOr(&seen[id >> 5], bit);
        if ((old & bit) == 0u) logits[id] /= penalty;
    }
}

__global__ __launch_bounds__(kThreads) void penalty_scan_kernel(float * logits, const int64_t * recent,
                                                                int32_t n, float penalty, int64_t limit) {
    for (int j = threadIdx.x; j < n; j += kThreads) {
        const int64_t id = recent[j];
        if (id < 0 || id >= limit) continue;
        bool first = true;
        for (int k = 0; k < j && first; ++k) first = recent[k] != id;
        if (first) logits[id] /= penalty;
    }
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_repetition_penalty(float * logits, int64_t vocab, const int64_t * recent,
                                           int32_t n_recent, float penalty, int64_t limit,
                                           levo_hip_stream_t stream) {
    LEVO_REQUIRE(penalty > 0.0f && __builtin_isfinite(penalty),
                 "repetition penalty must be finite and positive");
    LEVO_REQUIRE(vocab >= 0 && n_recent >= 0 && limit >= 0, "repetition penalty: negative size");
    const int64_t lim = (limit == 0 || limit > vocab) ? vocab : limit;
    if (lim == 0 || n_recent == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(logits != nullptr && recent != nullptr, "repetition penalty: null pointer");
    if (lim <= kBitmapIds)
        penalty_bitmap_kernel<<<1, kThreads, 0, as_hip(stream)>>>(logits, recent, n_recent, penalty, lim);
    else
        penalty_scan_kernel<<<1, kThreads, 0, as_hip(stream)>>>(logits, recent, n_recent, penalty, lim);
    return launch_status("levo_hip_repetition_penalty");
}
