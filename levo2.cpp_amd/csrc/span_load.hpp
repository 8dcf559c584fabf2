// A wave's contiguous span of matrix bytes, loaded with coalesced dwordx4
// loads into registers and stored to the wave's LDS stage area, shared by
// the decode mat-vecs (Q8_0 and the K-quants): the weight requests of the
// whole span are in flight at once, and the blocks are parsed from LDS at
// any byte offset afterwards.
#pragma once

#include "common.hpp"

namespace levo_hip {

// Coalesced loads of the 16-byte chunks covering bytes [a0, b1) of `base`
// (a0 16-byte aligned): lane l takes chunks l, l + 64, ... (CH per lane).
// Every lane issues all CH loads, with no branch around or after them, so
// that a later wait for a load issued before them can count them (a load
// under a branch, or a register a branch may overwrite, makes the compiler
// wait for everything). A chunk past the span re-reads the span's last
// chunk (a repeated address within one wave's request is served once); the
// chunk that would cross `limit` (the end of the buffer) reads the chunk
// before it (a span holds at least one 34-byte block, so that one is in the
// span) and store_span writes its bytes itself; an inactive wave reads the
// buffer's first chunk.
template <int CH>
__device__ __forceinline__ void load_span(const uint8_t * base, int64_t limit, int64_t a0, int64_t b1, bool active,
                                          int lane, u32x4 (&r)[CH]) {
    const int nchunks = active ? static_cast<int>((b1 - a0 + 15) >> 4) : 0;
    const int64_t last = a0 + 16 * static_cast<int64_t>(nchunks - 1);
    const int64_t last_whole = last + 16 <= limit ? last : last - 16;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        const int64_t at = a0 + 16 * static_cast<int64_t>(c);
        const int64_t from = !active ? 0 : at < last_whole ? at : last_whole;
        r[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(base + from));
    }
}

// The span's chunks into the wave's LDS stage area; the chunk that crosses
// the end of the buffer (if any) is read again here as half-words below
// `limit` (zero past it).
template <int CH>
__device__ __forceinline__ void store_span(uint8_t * stage, const uint8_t * base, int64_t limit, int64_t a0,
                                           int64_t b1, bool active, int lane, const u32x4 (&r)[CH]) {
    const int nchunks = active ? static_cast<int>((b1 - a0 + 15) >> 4) : 0;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
        const int c = lane + 64 * i;
        if (c >= nchunks) continue;
        const int64_t at = a0 + 16 * static_cast<int64_t>(c);
        u32x4 v = r[i];
        if (at + 16 > limit) {
            uint32_t h[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                h[k] = at + 2 * k + 2 <= limit ? *reinterpret_cast<const uint16_t *>(base + at + 2 * k) : 0u;
            }
            v = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
        }
        reinterpret_cast<u32x4 *>(stage)[c] = v;
    }
}

// The wave's own LDS stores are visible to all its lanes.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

}  // namespace levo_hip
