#pragma once
// The sampled branch of sample_top_k_counted (src/levo-sampling.cpp:97-115)
// on the device, after levo_hip_cfg_sample has produced each row's candidate
// set: the reference's double weights exp((double)((v - max) / T)), their
// sequential sum, one uniform (53 bits + 0.5) / 2^53 and the sequential
// cumulative search. Only the token ids and the draw counts leave the GPU.
//
// The mt19937_64 engine stays with the caller: `bits` holds the next raw
// values of the caller's engine, and row r takes the j-th of them when it is
// the j-th row (in row order) that draws. A row draws exactly when the
// reference would: sampling on, T != 0, no NaN, and a finite maximum (then the
// weight total is finite and >= 1; with a +-inf maximum the reference returns
// the first maximum without a draw, :108). draws[r] is the number of values
// rows 0..r consumed, so the caller advances its engine by draws[rows - 1].
//
// One wave per row; no LDS, no barriers. Lane i computes the weights of
// candidates i, i + 64, ...; the cumulative sums in candidate (ascending id)
// order come from one prefix scan per 64 candidates (six DPP steps) instead
// of the reference's chain of n dependent additions. Up to 64 candidates
// (top-k 50) take one pass that leaves each lane its own cumulative sum;
// larger sets take two (total, then the search).
//
// Exactness: the F32 steps (v - max, / T) are IEEE and equal to the host's;
// the double exp of the device library and of the host's libm may differ in
// the last bit, and the scan rounds its sums in another order than the
// reference's sequential loop (each prefix of non-negative terms is then off
// by at most (depth + 1) * 2^-53 of the total, depth <= 6 + n / 64, against
// (n - 1) * 2^-53 for the sequential sum). Together these move a cumulative
// boundary or the target by at most about (2 n + 16) * 2^-52 * total, so the
// pick can differ from the reference's only when the target lies that close
// to a boundary. The kernel flags those rows (margin (n + 4) * 2^-44 * total,
// over a hundred times wider) as LEVO_HIP_TOKEN_RECHECK for the caller to
// draw on the host with the same raw value; for random targets that happens
// with probability about (n + 4) * 2^-43 per draw.

#include "common.hpp"

namespace levo_hip {
namespace draw_detail {

constexpr double kTwoPowMinus53 = 0x1p-53;
constexpr double kMarginUlps = 0x1p-44;

__device__ __forceinline__ double read_lane_f64(double v, int lane) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), lane));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), lane));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// Weight of candidate value v (src/levo-sampling.cpp:103-105): -inf gives 0,
// otherwise exp of the F32 quotient widened to double.
__device__ __forceinline__ double draw_weight(float v, float m, float t) {
    if (v == -__builtin_inff()) return 0.0;
    return exp(static_cast<double>((v - m) / t));
}

__device__ __forceinline__ bool row_draws(const levo_hip_draw_args & a, int64_t r) {
    return a.best[r] >= 0 && __builtin_isfinite(a.row_max[r]);
}

// The token of a row that draws, computed by one whole wave: its n
// candidates in ascending id order (lane l holds candidate l in v0 / id0 when
// l < n; `vals` / `ids` hold the whole list and are read only when n > 64),
// the maximum m, the temperature t and the row's raw value. Returns the id,
// or LEVO_HIP_TOKEN_RECHECK; the same value in every lane.
__device__ __forceinline__ int64_t draw_token(const float * vals, const int32_t * ids, float v0, int32_t id0, int n,
                                              float m, float t, uint64_t raw) {
    const int lane = static_cast<int>(threadIdx.x & 63);
    const double u = (static_cast<double>(raw >> 11) + 0.5) * kTwoPowMinus53;

    double total = 0.0;
    double cumulative = 0.0;
    double below = 0.0;
    double above = 0.0;
    double target;
    int found = -1;
    if (n <= 64) {
        // Lane l's cumulative sum through candidate l by one prefix scan;
        // lanes past n add +0.0.
        const double w = lane < n ? draw_weight(v0, m, t) : 0.0;
        const double mine = wave_inclusive_scan_f64(w);
        total = read_lane_f64(mine, 63);
        target = u * total;
        const uint64_t hit = __ballot(lane < n && target < mine);
        if (hit != 0) {
            found = __builtin_ctzll(hit);
            above = read_lane_f64(mine, found);
            if (found > 0) below = read_lane_f64(mine, found - 1);
        } else {
            below = total;
        }
        cumulative = total;
    } else {
        // Pass 1: the total, 64 candidates per prefix scan.
        for (int base = 0; base < n; base += 64) {
            const int i = base + lane;
            const double w = i < n ? draw_weight(vals[i], m, t) : 0.0;
            total += read_lane_f64(wave_inclusive_scan_f64(w), 63);
        }
        // Pass 2: the first candidate whose cumulative sum exceeds the
        // target; `below` / `above` are the sums on either side of it.
        target = u * total;
        for (int base = 0; base < n && found < 0; base += 64) {
            const int i = base + lane;
            const double w = i < n ? draw_weight(vals[i], m, t) : 0.0;
            const double mine = cumulative + wave_inclusive_scan_f64(w);
            const uint64_t hit = __ballot(i < n && target < mine);
            if (hit != 0) {
                const int l = __builtin_ctzll(hit);
                found = base + l;
                above = read_lane_f64(mine, l);
                below = l > 0 ? read_lane_f64(mine, l - 1) : cumulative;
            } else {
                cumulative = read_lane_f64(mine, 63);
                below = cumulative;
            }
        }
    }
    const double margin = static_cast<double>(n + 4) * kMarginUlps * total;
    bool recheck = target - below <= margin && below != 0.0;
    if (found >= 0) recheck = recheck || above - target <= margin;
    else recheck = recheck || target - cumulative <= margin;
    if (recheck) return LEVO_HIP_TOKEN_RECHECK;
    const int pick = found >= 0 ? found : n - 1;
    if (n <= 64) return __builtin_amdgcn_readlane(id0, pick);
    return ids[pick];
}

// Row r's token and draw count, computed by one whole wave.
__device__ __forceinline__ void draw_row(const levo_hip_draw_args & a, int64_t r) {
    const int lane = static_cast<int>(threadIdx.x & 63);
    const bool sampling = a.use_sampling != 0 && a.temperature != 0.0f;

    // Every load of the common case (n <= 64) is issued before any branch on
    // loaded data, so the row costs one memory round trip: the row's own
    // scalars, the first 64 candidates, the raw value at the row index (the
    // draw index equals it whenever no earlier row skipped its draw) and the
    // first 64 earlier rows' draw conditions.
    const int32_t best = a.best[r];
    const int32_t n = a.count[r];
    const float m = a.row_max[r];
    const float * vals = a.cand_logits + r * a.capacity;
    const int32_t * ids = a.cand_ids + r * a.capacity;
    const int first = lane < a.capacity ? lane : 0;
    const float v0 = vals[first];
    const int32_t id0 = ids[first];
    const uint64_t raw_at_r = sampling ? a.bits[r] : 0;
    bool d0 = false;
    if (sampling && lane < r) d0 = row_draws(a, lane);

    // Draws taken by the rows before r.
    int before = static_cast<int>(__popcll(__ballot(d0)));
    if (sampling) {
        for (int64_t base = 64; base < r; base += 64) {
            const int64_t j = base + lane;
            const bool d = j < r && row_draws(a, j);
            before += static_cast<int>(__popcll(__ballot(d)));
        }
    }
    const bool draws = sampling && best >= 0 && __builtin_isfinite(m);
    if (lane == 0) a.draws[r] = before + (draws ? 1 : 0);
    if (best < 0) {
        if (lane == 0) a.tokens[r] = LEVO_HIP_TOKEN_NAN;
        return;
    }
    if (!draws) {
        if (lane == 0) a.tokens[r] = best;
        return;
    }
    if (n > a.capacity) {
        if (lane == 0) a.tokens[r] = LEVO_HIP_TOKEN_OVERFLOW;
        return;
    }
    const uint64_t raw = before == r ? raw_at_r : a.bits[before];
    const int64_t token = draw_token(vals, ids, v0, id0, n, m, a.temperature, raw);
    if (lane == 0) a.tokens[r] = token;
}

}  // namespace draw_detail

using draw_detail::draw_row;
using draw_detail::draw_token;

}  // namespace levo_hip
