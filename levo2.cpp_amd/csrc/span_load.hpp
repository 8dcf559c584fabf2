// A wave's contiguous span of matrix bytes, loaded with coalesced dwordx4
// loads into registers and stored to the wave's LDS stage area, shared by
// the decode mat-vecs (Q8_0 and the K-quants): the weight requests of the
// whole span are in flight at once, and the blocks are parsed from LDS at
// any byte offset afterwards.
#pragma once

#include "common.hpp"

namespace levo_hip {

// Coalesced loads of the 16-byte chunks covering bytes [a0, b1) of `base`
// (a0 16-byte aligned): lane l takes chunks l, l + 64, ... (CH per lane). A
// chunk that would cross `limit` (the end of the buffer) is read as
// half-words, so nothing past the buffer is touched.
template <int CH>
__device__ __forceinline__ void load_span(const uint8_t * base, int64_t limit, int64_t a0, int64_t b1, int lane,
                                          u32x4 (&r)[CH]) {
    const int nchunks = static_cast<int>((b1 - a0 + 15) >> 4);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        const int64_t at = a0 + 16 * static_cast<int64_t>(c);
        if (c < nchunks) {
            if (at + 16 <= limit) {
                r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + at));
            } else {
                uint32_t h[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    h[k] = at + 2 * k + 2 <= limit ? *reinterpret_cast<const uint16_t *>(base + at + 2 * k) : 0u;
                }
                r[i] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
            }
        }
    }
}

template <int CH>
__device__ __forceinline__ void store_span(uint8_t * stage, int64_t a0, int64_t b1, int lane, const u32x4 (&r)[CH]) {
    const int nchunks = static_cast<int>((b1 - a0 + 15) >> 4);
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunks) reinterpret_cast<u32x4 *>(stage)[c] = r[i];
    }
}

// The wave's own LDS stores are visible to all its lanes.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace levo_hip
