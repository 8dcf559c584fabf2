// CFG combine + temperature softmax + argmax / top-k over codebook logits.
//
// One workgroup (4 wave64s) per logit row. The row is read once from HBM
// (cond and uncond, dwordx4), combined l = u + s*(c - u) in registers and
// never written back: everything the sampler needs is produced from the
// register-resident row:
//   1. unique-token repetition penalty and stream-0 ignore list via LDS
//      bitmaps (src/levo-sampling.cpp:39-47, :137-147);
//   2. NaN rejection and the first maximum (std::max_element, :94-96);
//   3. the exact top-k threshold of the stable descending sort (:84-93):
//      each wave finds the k-th largest of its 64 lane maxima with a ballot
//      bisection (a lower bound of the row's k-th value), the workgroup keeps
//      only the few elements above the largest such bound, and one wave
//      bisects their order-preserving keys to the exact k-th value;
//   4. every id >= that value, in ascending id order (ties with the k-th
//      value kept, as the reference keeps them), with its logit and its
//      probability exp((l - max)/T) / sum (:98-107, weights in double);
//   5. optionally the full-vocabulary log-sum-exp of l/T.
// The host keeps the mt19937_64 draw, so the sampled token is the reference's.
#include "common.hpp"

#include <cfloat>
#include <climits>

namespace levo_hip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kCandCap = 1024;    // LDS slots for threshold candidates
constexpr int kMaxVocab = 32768;
constexpr int kBitmapWords = kMaxVocab / 32;

// k-th largest (1 <= k <= 64) of the 64 lane keys of this wave.
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, int k) {
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        const int cnt = __popcll(__ballot(key >= cand));
        if (cnt >= k) prefix = cand;
    }
    return prefix;
}

__device__ __forceinline__ double cand_weight(float v, float m, float t) {
    if (__builtin_isinf(v) && v < 0.0f) return 0.0;
    return exp(static_cast<double>((v - m) / t));
}

template <int VEC, int NCH>
__global__ __launch_bounds__(kThreads) void cfg_sample_kernel(const levo_hip_sample_args a) {
    constexpr int ITEMS = VEC * NCH;
    constexpr int kChunk = kThreads * VEC;            // ids per chunk
    constexpr int kCPL = (NCH + 63) / 64;             // chunks per lane in the chunk scan

    __shared__ uint32_t s_pen[kBitmapWords];
    __shared__ uint32_t s_ign[kBitmapWords];
    __shared__ uint32_t s_cand[kCandCap];
    __shared__ int s_chunk_count[NCH][kWaves];
    __shared__ float s_wmax[kWaves];
    __shared__ int s_widx[kWaves];
    __shared__ int s_wnan[kWaves];
    __shared__ uint32_t s_wlow[kWaves];
    __shared__ double s_wz[kWaves];
    __shared__ float s_wlse[kWaves];
    __shared__ int s_bis[2][kWaves];
    __shared__ int s_ncand;
    __shared__ uint32_t s_tau;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const int V = static_cast<int>(a.vocab);
    const int stream = static_cast<int>(row % a.n_streams);
    int k = a.top_k[stream];
    if (k <= 0 || k >= V) k = 0;  // keep every id

    // ---- 1. load + CFG ------------------------------------------------------
    float v[ITEMS];
    const float * crow = a.cond + row * a.row_pitch;
    const float * urow = a.uncond ? a.uncond + row * a.row_pitch : nullptr;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const int base = ch * kChunk + tid * VEC;
        if constexpr (VEC == 4) {
            // pitch % 4 == 0, so a vector starting below V lies inside the row
            // pitch; its ids >= V are masked to -inf here and by idx < V below.
            if (base < V) {
                const f32x4 c = *reinterpret_cast<const f32x4 *>(crow + base);
                if (urow) {
                    const f32x4 u = *reinterpret_cast<const f32x4 *>(urow + base);
                    v[ch * 4 + 0] = u.x + a.cfg_scale * (c.x - u.x);
                    v[ch * 4 + 1] = u.y + a.cfg_scale * (c.y - u.y);
                    v[ch * 4 + 2] = u.z + a.cfg_scale * (c.z - u.z);
                    v[ch * 4 + 3] = u.w + a.cfg_scale * (c.w - u.w);
                } else {
                    v[ch * 4 + 0] = c.x;
                    v[ch * 4 + 1] = c.y;
                    v[ch * 4 + 2] = c.z;
                    v[ch * 4 + 3] = c.w;
                }
#pragma unroll
                for (int q = 1; q < 4; ++q)
                    if (base + q >= V) v[ch * 4 + q] = -INFINITY;
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[ch * 4 + q] = -INFINITY;
            }
        } else {
            if (base < V) {
                const float c = crow[base];
                v[ch] = urow ? urow[base] + a.cfg_scale * (c - urow[base]) : c;
            } else {
                v[ch] = -INFINITY;
            }
        }
    }

    // ---- 2. repetition penalty / ignore list ---------------------------------
    const bool use_pen = a.recent != nullptr && a.n_recent > 0;
    const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
    if (use_pen || use_ign) {  // uniform per workgroup
        const int words = (V + 31) / 32;
        for (int i = tid; i < words; i += kThreads) {
            s_pen[i] = 0u;
            s_ign[i] = 0u;
        }
        __syncthreads();
        if (use_pen) {
            const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
            const int64_t * rec = a.recent + row * a.n_recent;
            for (int i = tid; i < a.n_recent; i += kThreads) {
                const int64_t t = rec[i];
                if (t >= 0 && t < limit) atomicOr(&s_pen[t >> 5], 1u << (t & 31));
            }
        }
        if (use_ign) {
            for (int i = tid; i < a.n_ignore; i += kThreads) {
                const int64_t t = a.ignore[i];
                if (t >= 0 && t < V) atomicOr(&s_ign[t >> 5], 1u << (t & 31));
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
            if (idx < V) {
                const uint32_t bit = 1u << (idx & 31);
                if (s_pen[idx >> 5] & bit) v[i] = v[i] / a.repetition_penalty;
                if (s_ign[idx >> 5] & bit) v[i] = -INFINITY;
            }
        }
    }

    // ---- 3. NaN check, thread max / first argmax ----------------------------
    bool has_nan = false;
    float tmax = -INFINITY;
    int targ = INT_MAX;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) {
        const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
        if (idx < V) {
            if (__builtin_isnan(v[i])) has_nan = true;
            else if (targ == INT_MAX || v[i] > tmax) {
                tmax = v[i];
                targ = idx;
            }
        }
    }
    // wave reduction: larger value, ties -> smaller id
    float wm = tmax;
    int wi = targ;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float om = __shfl_xor(wm, o, 64);
        const int oi = __shfl_xor(wi, o, 64);
        if (oi != INT_MAX && (wi == INT_MAX || om > wm || (om == wm && oi < wi))) {
            wm = om;
            wi = oi;
        }
    }
    const bool wave_nan = __ballot(has_nan) != 0;
    // per-wave lower bound of the row's k-th largest value (k <= 64)
    uint32_t wlow = 0;
    if (k > 1 && k <= 64) wlow = wave_kth_key(targ == INT_MAX ? 0u : float_key(tmax), k);
    if (lane == 0) {
        s_wmax[wave] = wm;
        s_widx[wave] = wi;
        s_wnan[wave] = wave_nan ? 1 : 0;
        s_wlow[wave] = wlow;
    }
    if (tid == 0) s_ncand = 0;
    __syncthreads();

    float m = s_wmax[0];
    int best = s_widx[0];
    bool row_nan = s_wnan[0] != 0;
    uint32_t low = s_wlow[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        const float om = s_wmax[w];
        const int oi = s_widx[w];
        if (oi != INT_MAX && (best == INT_MAX || om > m || (om == m && oi < best))) {
            m = om;
            best = oi;
        }
        row_nan = row_nan || s_wnan[w] != 0;
        low = max(low, s_wlow[w]);
    }
    if (row_nan) {  // uniform: the reference throws "logits contain NaN"
        if (tid == 0) {
            a.best[row] = -1;
            a.count[row] = -1;
            if (a.row_max) a.row_max[row] = NAN;
            if (a.row_lse) a.row_lse[row] = NAN;
        }
        return;
    }

    // ---- optional full-vocabulary log-sum-exp of l / T ----------------------
    if (a.row_lse) {
        float s = 0.0f;
        const float inv_t = 1.0f / a.temperature;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
            if (idx < V) s += __expf((v[i] - m) * inv_t);
        }
        s = wave_sum_f32(s);
        if (lane == 0) s_wlse[wave] = s;
    }

    // ---- 4. exact threshold key tau ------------------------------------------
    uint32_t tau;
    if (k == 0) {
        tau = 0u;  // every valid id (all keys of non-NaN floats are > 0)
    } else if (k == 1) {
        tau = float_key(m);
    } else {
        bool done = false;
        tau = 0u;
        if (k <= 64) {
            // gather the keys >= low (contains every id above the k-th value)
#pragma unroll
            for (int i = 0; i < ITEMS; ++i) {
                const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
                const uint32_t key = float_key(v[i]);
                const bool p = idx < V && key >= low;
                const uint64_t mask = __ballot(p);
                if (mask) {
                    int base = 0;
                    if (lane == 0) base = atomicAdd(&s_ncand, __popcll(mask));
                    base = __builtin_amdgcn_readfirstlane(base);
                    const int pos = base + rank_in_mask(mask);
                    if (p && pos < kCandCap) s_cand[pos] = key;
                }
            }
            __syncthreads();
            const int c = s_ncand;
            if (c <= kCandCap) {
                if (wave == 0) {
                    constexpr int kSlots = kCandCap / 64;
                    uint32_t keys[kSlots];
#pragma unroll
                    for (int s = 0; s < kSlots; ++s) {
                        const int p = lane + 64 * s;
                        keys[s] = p < c ? s_cand[p] : 0u;
                    }
                    const int nslots = (c + 63) / 64;
                    uint32_t prefix = 0;
                    for (int bit = 31; bit >= 0; --bit) {
                        const uint32_t cand = prefix | (1u << bit);
                        int cnt = 0;
#pragma unroll
                        for (int s = 0; s < kSlots; ++s)
                            if (s < nslots) cnt += __popcll(__ballot(keys[s] >= cand));
                        if (cnt >= k) prefix = cand;
                    }
                    if (lane == 0) s_tau = prefix;
                }
                __syncthreads();
                tau = s_tau;
                done = true;
            }
        }
        if (!done) {
            // general path: bisection over the whole register-resident row
            uint32_t prefix = 0;
            int buf = 0;
            for (int bit = 31; bit >= 0; --bit) {
                const uint32_t cand = prefix | (1u << bit);
                int cnt = 0;
#pragma unroll
                for (int i = 0; i < ITEMS; ++i) {
                    const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
                    cnt += (idx < V && float_key(v[i]) >= cand) ? 1 : 0;
                }
                cnt = wave_sum_i32(cnt);
                if (lane == 0) s_bis[buf][wave] = cnt;
                __syncthreads();
                int total = 0;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) total += s_bis[buf][w];
                if (total >= k) prefix = cand;
                buf ^= 1;
            }
            tau = prefix;
        }
    }

    // ---- 5. candidates in ascending id order -----------------------------------
    const float temp = a.temperature;
    double z = 0.0;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        int cnt = 0;
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
            const int i = ch * VEC + q;
            const int idx = ch * kChunk + tid * VEC + q;
            const bool sel = idx < V && float_key(v[i]) >= tau;
            const uint64_t mask = __ballot(sel);
            cnt += __popcll(mask);
            if (a.cand_probs && mask && sel) z += cand_weight(v[i], m, temp);
        }
        if (lane == 0) s_chunk_count[ch][wave] = cnt;
    }
    if (a.cand_probs) {
        z = wave_sum_f64(z);
        if (lane == 0) s_wz[wave] = z;
    }
    __syncthreads();
    if (a.cand_probs) z = s_wz[0] + s_wz[1] + s_wz[2] + s_wz[3];
    const bool z_ok = z > 0.0 && __builtin_isfinite(z);

    // exclusive scan of chunk totals across the wave's lanes
    int lane_tot[kCPL];
    int lane_sum = 0;
#pragma unroll
    for (int j = 0; j < kCPL; ++j) {
        const int ch = lane * kCPL + j;
        int t = 0;
        if (ch < NCH) {
#pragma unroll
            for (int w = 0; w < kWaves; ++w) t += s_chunk_count[ch][w];
        }
        lane_tot[j] = t;
        lane_sum += t;
    }
    int incl = lane_sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
    }
    const int total = __shfl(incl, 63, 64);
    int lane_start[kCPL];
    {
        int run = incl - lane_sum;
#pragma unroll
        for (int j = 0; j < kCPL; ++j) {
            lane_start[j] = run;
            run += lane_tot[j];
        }
    }

    const int cap = a.capacity;
    int32_t * out_ids = a.cand_ids + row * cap;
    float * out_logits = a.cand_logits ? a.cand_logits + row * cap : nullptr;
    float * out_probs = a.cand_probs ? a.cand_probs + row * cap : nullptr;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        int start = 0;
#pragma unroll
        for (int j = 0; j < kCPL; ++j)
            if ((ch % kCPL) == j) start = __builtin_amdgcn_readlane(lane_start[j], ch / kCPL);
        if (start >= cap) break;  // uniform: later chunks only add later ids
        int before = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
            if (w < wave) before += s_chunk_count[ch][w];
        uint64_t masks[VEC];
        bool sels[VEC];
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
            const int idx = ch * kChunk + tid * VEC + q;
            sels[q] = idx < V && float_key(v[ch * VEC + q]) >= tau;
            masks[q] = __ballot(sels[q]);
        }
        int lower = 0;  // selected ids of lower lanes in this wave
#pragma unroll
        for (int q = 0; q < VEC; ++q) lower += rank_in_mask(masks[q]);
        int mine = 0;
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
            if (sels[q]) {
                const int pos = start + before + lower + mine;
                if (pos < cap) {
                    const int idx = ch * kChunk + tid * VEC + q;
                    const float lv = v[ch * VEC + q];
                    out_ids[pos] = idx;
                    if (out_logits) out_logits[pos] = lv;
                    if (out_probs) {
                        float p;
                        if (z_ok) p = static_cast<float>(cand_weight(lv, m, temp) / z);
                        else p = idx == best ? 1.0f : 0.0f;  // the reference falls back to best
                        out_probs[pos] = p;
                    }
                }
                ++mine;
            }
        }
    }

    if (tid == 0) {
        a.best[row] = best;
        a.count[row] = total;
        if (a.row_max) a.row_max[row] = m;
        if (a.row_lse) {
            const float s = s_wlse[0] + s_wlse[1] + s_wlse[2] + s_wlse[3];
            float lse;
            if (m == -INFINITY) lse = -INFINITY;
            else if (m == INFINITY) lse = INFINITY;
            else lse = m / a.temperature + logf(s);
            a.row_lse[row] = lse;
        }
    }
}

template <int VEC, int NCH>
int launch_sample(const levo_hip_sample_args & a, hipStream_t stream) {
    cfg_sample_kernel<VEC, NCH><<<static_cast<uint32_t>(a.rows), kThreads, 0, stream>>>(a);
    return launch_status("levo_hip_cfg_sample");
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

extern "C" int levo_hip_cfg_sample(const levo_hip_sample_args * args, levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "cfg_sample: null argument block");
    const levo_hip_sample_args & a = *args;
    LEVO_REQUIRE(a.rows >= 0, "cfg_sample: negative row count");
    if (a.rows == 0) return LEVO_HIP_OK;
    LEVO_REQUIRE(a.vocab >= 1, "cannot sample an empty vocabulary");
    LEVO_REQUIRE(a.vocab <= kMaxVocab, "cfg_sample: vocabulary exceeds %d", kMaxVocab);
    LEVO_REQUIRE(a.row_pitch >= a.vocab, "cfg_sample: row pitch is smaller than the vocabulary");
    LEVO_REQUIRE(a.rows < (int64_t{1} << 31), "cfg_sample: too many rows");
    LEVO_REQUIRE(a.cond != nullptr, "cfg_sample: conditional logits are null");
    LEVO_REQUIRE(a.n_streams >= 1 && a.n_streams <= LEVO_HIP_MAX_STREAMS, "cfg_sample: stream count out of range");
    for (int s = 0; s < a.n_streams; ++s) LEVO_REQUIRE(a.top_k[s] >= 0, "cfg_sample: negative top_k");
    LEVO_REQUIRE(a.best != nullptr && a.count != nullptr && a.cand_ids != nullptr,
                 "cfg_sample: null output");
    LEVO_REQUIRE(a.capacity >= 1, "cfg_sample: candidate capacity must be positive");
    LEVO_REQUIRE(!(a.recent != nullptr && a.n_recent > 0) ||
                     (a.repetition_penalty > 0.0f && __builtin_isfinite(a.repetition_penalty)),
                 "repetition penalty must be finite and positive");
    LEVO_REQUIRE(a.n_recent >= 0 && a.n_ignore >= 0, "cfg_sample: negative list length");
    LEVO_REQUIRE((a.cand_probs == nullptr && a.row_lse == nullptr) ||
                     (a.temperature > 0.0f && __builtin_isfinite(a.temperature)),
                 "temperature must be finite and positive for softmax outputs");
    const hipStream_t st = as_hip(stream);
    const bool vec = a.row_pitch % 4 == 0 && aligned16(a.cond) && (a.uncond == nullptr || aligned16(a.uncond));
    const int64_t V = a.vocab;
    if (vec) {
        if (V <= 1024) return launch_sample<4, 1>(a, st);
        if (V <= 2048) return launch_sample<4, 2>(a, st);
        if (V <= 4096) return launch_sample<4, 4>(a, st);
        if (V <= 8192) return launch_sample<4, 8>(a, st);
        if (V <= 16384) return launch_sample<4, 16>(a, st);
        if (V <= 17408) return launch_sample<4, 17>(a, st);
        return launch_sample<4, 32>(a, st);
    }
    if (V <= 256) return launch_sample<1, 1>(a, st);
    if (V <= 1024) return launch_sample<1, 4>(a, st);
    if (V <= 4096) return launch_sample<1, 16>(a, st);
    if (V <= 16384) return launch_sample<1, 64>(a, st);
    if (V <= 16640) return launch_sample<1, 65>(a, st);
    return launch_sample<1, 128>(a, st);
}
