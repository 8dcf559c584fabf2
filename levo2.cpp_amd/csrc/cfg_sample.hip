// CFG combine + temperature softmax + argmax / top-k over codebook logits.
//
// One workgroup (8 wave64s, 32 logits per thread at V = 16384) per logit row. The row is read once from HBM
// (cond and uncond, dwordx4), combined l = u + s*(c - u) in registers and
// never written back. Everything the sampler needs comes from the
// register-resident row, touching each value only with cheap compares:
//   A. while the loads of later chunks are still in flight, each chunk is
//      combined and folded into per-thread softmax statistics: the running
//      maximum and a sum of exp2((l - shift) * log2(e) / T) with a fixed
//      shift (the thread's first group maximum), one FMA and one exp2 per
//      value; a NaN, +inf or overflowed sum is summed again from the thread
//      maximum, and a NaN or +inf logit then leaves it NaN, which sends the row
//      to an exact re-check.
//      The unique-token repetition penalty and stream-0 ignore list are applied
//      through LDS bitmaps (src/levo-sampling.cpp:39-47, :137-147); such rows
//      recompute their statistics after the adjustment;
//   B. a lower bound of the k-th largest value: each wave bisects the
//      order-preserving keys of its 64 lane maxima with ballots (no barrier)
//      for its ceil(k/8)-th largest; at least k ids lie at or above the
//      smallest of the eight bounds;
//   C. the first maximum (std::max_element, :94-96), the optional
//      full-vocabulary log-sum-exp of l/T from the streamed statistics, and a
//      gather of the few ids at or above the bound (value and id, one compare
//      per id) into per-wave LDS segments; the row's registers are dead after
//      this point, and waves 1-7 leave (wave 1 writes the row's max, first
//      maximum and log-sum-exp), so a new row can start in their registers;
//   D. the exact k-th value of the stable descending sort (:84-89): wave 0
//      bisects the gathered keys (starting below the common high bits of the
//      bound and the maximum);
//   E. every gathered id >= that value (ties kept, as the reference keeps
//      them) is marked in an LDS bitmap; a popcount prefix scan over the
//      bitmap gives each candidate its slot in ascending id order, and its
//      logit and probability exp((l - max)/T) / sum (:98-107; F32 weights,
//      double sum) are written there. D and E are one wave's work, with no
//      workgroup barrier.
// k == 0 (keep all), k > 256, or more tied candidates than the segments hold
// take select_general (the whole workgroup), which re-reads the row instead
// of holding it.
// The host keeps the mt19937_64 draw, so the sampled token is the reference's.
#include "common.hpp"
#include "sample_draw.hpp"

#include <cfloat>
#include <climits>
#include <mutex>

namespace levo_hip {
namespace {

// 512 threads: at 72 VGPRs three rows share a CU; against 256 threads (four
// rows at 98 VGPRs) each wave's serial work after the row has arrived halves,
// which measured 4% faster on 750 x 3 rows of 16384.
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kSegCap = 256;   // gathered candidates per wave segment
constexpr int kBisCap = 256;   // candidates the one-wave bisection holds (4 per lane)
constexpr int kMaxVocab = 32768;

// The penalty and ignore lists enter a row's bitmaps through one entry per
// thread: entry i < n_pen of the row's recent ids, then entry i - n_pen of the
// ignore list. The decode step's segment kernel requests the first kThreads
// entries before its logits, so the two memory round trips overlap; the load
// takes no branch (a lane without an entry reads kNoListEntry), which keeps
// the compiler from waiting for it before the logits' loads are issued.
__device__ const int64_t kNoListEntry = -1;

__device__ __forceinline__ int64_t list_entry(const int64_t * rec, int n_pen, const int64_t * ign, int n_ign,
                                              int i) {
    const int64_t * p = i < n_pen ? rec + i : i < n_pen + n_ign ? ign + (i - n_pen) : &kNoListEntry;
    return *p;
}

__device__ __forceinline__ float float_of_key(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// k-th largest (1 <= k <= 64) of the 64 lane keys of this wave; 0 when fewer
// than k lanes hold a non-zero key. The answer lies between the smallest
// non-zero key and the largest, so the bisection starts below their common
// high bits (about 24 steps instead of 32 for logits of one magnitude).
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, int k) {
    if (static_cast<int>(__popcll(__ballot(key != 0u))) < k) return 0u;
    const uint32_t hi = dpp::allreduce(key, [](uint32_t a, uint32_t b) { return a > b ? a : b; });
    const uint32_t lo = dpp::allreduce(key == 0u ? ~0u : key, [](uint32_t a, uint32_t b) { return a < b ? a : b; });
    const uint32_t diff = lo ^ hi;
    if (diff == 0u) return lo;
    const int top = 31 - __builtin_clz(diff);
    uint32_t prefix = lo & ~((2u << top) - 1u);
    for (int bit = top; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        if (static_cast<int>(__popcll(__ballot(key >= cand))) >= k) prefix = cand;
    }
    return prefix;
}

// exp((l - max) / T) for the F32 probability output; -inf logits give 0.
__device__ __forceinline__ float cand_weight(float v, float m, float inv_t) {
    return __expf((v - m) * inv_t);
}

// Per-thread softmax statistics over groups of four items: tmax is the
// running maximum (fmaxf skips NaN); sh is a fixed shift, the largest value of
// the thread's first group (or -FLT_MAX if it is all -inf), and
// s = sum of exp2((v - sh) * c2), each term one FMA and one exp2 (no
// rescaling while the row streams in). A NaN value makes s NaN, +inf makes it
// +inf; so does a value so far above the shift that its term overflows, which
// finish_stats then resolves by summing again from the thread maximum.
struct row_stats {
    float tmax = -INFINITY;
    float sh = -FLT_MAX;
    float nsc = 0.0f;  // -sh * c2
    float s = 0.0f;
};

template <bool kFirst>
__device__ __forceinline__ void stats_add4(row_stats & st, float r0, float r1, float r2, float r3, float c2) {
    const float gm = fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
    if constexpr (kFirst) {
        st.sh = fmaxf(gm, -FLT_MAX);
        st.nsc = -st.sh * c2;
    }
    st.tmax = fmaxf(st.tmax, gm);
    float acc = st.s;
    acc += __builtin_amdgcn_exp2f(__builtin_fmaf(r0, c2, st.nsc));
    acc += __builtin_amdgcn_exp2f(__builtin_fmaf(r1, c2, st.nsc));
    acc += __builtin_amdgcn_exp2f(__builtin_fmaf(r2, c2, st.nsc));
    acc += __builtin_amdgcn_exp2f(__builtin_fmaf(r3, c2, st.nsc));
    st.s = acc;
}

// A sum that is not finite, or whose shift lies more than 2^64 (in terms)
// below the thread maximum, is summed again from the thread maximum. That
// either makes it finite (an overflow of the fixed shift) or shows a NaN or
// +inf value (the sum is then NaN); and the thread's largest term can then
// only vanish in the rescale to the row maximum when it is below 2^-85 of it.
template <int ITEMS>
__device__ __forceinline__ void finish_stats(row_stats & st, const float (&v)[ITEMS], float c2) {
    if (__builtin_isfinite(st.s) && (st.tmax - st.sh) * c2 <= 64.0f) return;
    st.sh = fmaxf(st.tmax, -FLT_MAX);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < ITEMS; ++i) acc += __builtin_amdgcn_exp2f((v[i] - st.sh) * c2);
    st.s = acc;
}

// l = u + s * (c - u) for every id this thread owns: id of item i is
// (i / VEC) * kThreads * VEC + tid * VEC + i % VEC. Every load is issued before the
// first is consumed; each chunk is folded into the statistics as it arrives.
// The logits are read once, with streaming (nontemporal) loads.
// kFull: the row fills every item (V == 256 * VEC * NCH), no masking.
template <int VEC, int NCH, bool kCfg, bool kFull>
__device__ __forceinline__ void load_row(float (&v)[VEC * NCH], row_stats & st, const float * __restrict__ crow,
                                         const float * __restrict__ urow, int V, int tid, float s, float c2) {
    constexpr int kChunk = kThreads * VEC;
    if constexpr (VEC == 4) {
        f32x4 c[NCH], u[NCH];
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = ch * kChunk + tid * 4;
            const int off = kFull || base < V ? base : 0;  // row_pitch % 4 == 0: in bounds
            c[ch] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(crow + off));
            if constexpr (kCfg) u[ch] = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(urow + off));
        }
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = ch * kChunk + tid * 4;
            float r[4] = {c[ch].x, c[ch].y, c[ch].z, c[ch].w};
            if constexpr (kCfg) {
                const float w[4] = {u[ch].x, u[ch].y, u[ch].z, u[ch].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) r[q] = w[q] + s * (r[q] - w[q]);
            }
            if constexpr (!kFull) {
#pragma unroll
                for (int q = 0; q < 4; ++q) r[q] = base + q < V ? r[q] : -INFINITY;
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) v[ch * 4 + q] = r[q];
            if (ch == 0) stats_add4<true>(st, r[0], r[1], r[2], r[3], c2);
            else stats_add4<false>(st, r[0], r[1], r[2], r[3], c2);
        }
        finish_stats(st, v, c2);
    } else {
        float c[NCH], u[NCH];
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = ch * kChunk + tid;
            const int off = base < V ? base : 0;
            c[ch] = __builtin_nontemporal_load(crow + off);
            if constexpr (kCfg) u[ch] = __builtin_nontemporal_load(urow + off);
        }
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int base = ch * kChunk + tid;
            const float r = kCfg ? u[ch] + s * (c[ch] - u[ch]) : c[ch];
            v[ch] = base < V ? r : -INFINITY;
        }
#pragma unroll
        for (int g = 0; g < NCH; g += 4) {
            const float r1 = g + 1 < NCH ? v[g + 1] : -INFINITY;
            const float r2 = g + 2 < NCH ? v[g + 2] : -INFINITY;
            const float r3 = g + 3 < NCH ? v[g + 3] : -INFINITY;
            if (g == 0) stats_add4<true>(st, v[g], r1, r2, r3, c2);
            else stats_add4<false>(st, v[g], r1, r2, r3, c2);
        }
    }
    finish_stats(st, v, c2);
}

// Shared-memory layout of one row's workgroup.
template <int kWords>
struct row_lds {
    // the bitmap and its prefix padded to a whole number of words per lane,
    // so that one wave reads and writes them without a branch per word
    static constexpr int kPadWords = (kWords + 63) / 64 * 64;
    uint32_t sel[kPadWords];     // selected-id bitmap
    uint32_t prefix[kPadWords];  // exclusive popcount prefix per bitmap word
    uint32_t pen[kWords];     // repetition-penalty ids
    uint32_t ign[kWords];     // ignored ids (stream 0)
    float cv[kWaves][kSegCap];  // gathered candidate values, one segment per wave
    int ci[kWaves][kSegCap];    // and their ids
    uint32_t hist[256];         // digit histogram of the one-wave radix select
    float wmax[kWaves];
    float wbv[kWaves];   // each wave's value at its first maximum
    float wlow[kWaves];
    int wnan[kWaves];
    int wbest[kWaves];
    int wcnt[kWaves];
    float wlse[kWaves];
    double wz[kWaves];
    int bis[2][kWaves];
    uint32_t tau;
    int total;
};

template <int kWords>
__device__ __forceinline__ float adjusted_logit(const levo_hip_sample_args & a, const row_lds<kWords> & L,
                                                const float * crow, const float * urow, bool pen, bool ign,
                                                int idx) {
    const float c = crow[idx];
    float v = urow ? urow[idx] + a.cfg_scale * (c - urow[idx]) : c;
    const uint32_t bit = 1u << (idx & 31);
    if (pen && (L.pen[idx >> 5] & bit)) v = v / a.repetition_penalty;
    if (ign && (L.ign[idx >> 5] & bit)) v = -INFINITY;
    return v;
}

// One wave's LDS operations complete in issue order; the fence keeps the
// compiler from moving them across each other and waits for their results.
__device__ __forceinline__ void wave_lds_order() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The k-th largest of the valid keys (k >= 1), all of which share `prefix`'s
// bits above bit `top`, by one wave: a radix select over digits of up to 8
// bits from bit `top` down. Each pass histograms the digit of the keys that
// match the digits chosen so far (LDS atomics), scans the 256 bins from the
// top (four per lane), and keeps the largest digit d whose keys at or above
// it number at least the still-needed count. This is the largest t with
// #{keys >= t} >= k, the same value a bit-by-bit bisection finds; when fewer
// than k keys exist the remaining digits are 0 (every key is kept).
template <int NS>
__device__ __forceinline__ uint32_t radix_kth_key(uint32_t * hist, const uint32_t (&keys)[NS],
                                                  const bool (&valid)[NS], int k, uint32_t prefix, int top) {
    const int lane = threadIdx.x & 63;
    int need = k;
    for (int hi = top; hi >= 0;) {  // uniform
        const int width = hi + 1 < 8 ? hi + 1 : 8;
        const int lo = hi + 1 - width;
        const uint32_t mask = (1u << width) - 1u;
        reinterpret_cast<u32x4 *>(hist)[lane] = u32x4{0u, 0u, 0u, 0u};
        wave_lds_order();
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const bool match = hi == 31 || ((keys[s] ^ prefix) >> (hi + 1)) == 0u;
            if (valid[s] && match) atomicAdd(&hist[(keys[s] >> lo) & mask], 1u);
        }
        wave_lds_order();
        const u32x4 b = reinterpret_cast<const u32x4 *>(hist)[lane];
        const int local = static_cast<int>(b[0] + b[1] + b[2] + b[3]);
        const int incl = wave_inclusive_scan_i32(local);
        const int above = dpp::lane(incl, 63) - incl;  // keys in the bins of higher lanes
        const int s3 = above + static_cast<int>(b[3]);
        const int s2 = s3 + static_cast<int>(b[2]);
        const int s1 = s2 + static_cast<int>(b[1]);
        const int s0 = s1 + static_cast<int>(b[0]);
        const uint64_t q = __ballot(s0 >= need);
        uint32_t digit = 0u;
        if (q != 0u) {
            const int owner = 63 - __builtin_clzll(q);
            const int j = s3 >= need ? 3 : s2 >= need ? 2 : s1 >= need ? 1 : 0;
            const int higher = j == 3 ? above : j == 2 ? s3 : j == 1 ? s2 : s1;  // keys in bins above the digit
            digit = static_cast<uint32_t>(__builtin_amdgcn_readlane(4 * lane + j, owner));
            need -= __builtin_amdgcn_readlane(higher, owner);
        }
        prefix = (prefix & ~(mask << lo)) | (digit << lo);
        hi = lo - 1;
        wave_lds_order();  // every lane has read the bins before the next pass clears them
    }
    return prefix;
}

// Exclusive prefix of the bitmap popcounts into L.prefix; returns the total
// candidate count (also stored in L.total). Called by one whole wave; the
// fences keep its LDS accesses in program order around the cross-lane reads.
template <int kWords>
__device__ __forceinline__ int wave_bitmap_prefix(row_lds<kWords> & L, int words) {
    constexpr int kWPL = row_lds<kWords>::kPadWords / 64;  // words per lane
    const int lane = threadIdx.x & 63;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // Every word of the padded bitmap is read and every prefix word written
    // with no branch around them, so the reads are issued together and waited
    // for once (a read under a per-word condition waits for each in turn);
    // words from `words` on (not cleared) count as empty.
    uint32_t bits[kWPL];
#pragma unroll
    for (int j = 0; j < kWPL; ++j) bits[j] = L.sel[lane * kWPL + j];
    int cnt[kWPL];
    int local = 0;
#pragma unroll
    for (int j = 0; j < kWPL; ++j) {
        cnt[j] = lane * kWPL + j < words ? __popc(bits[j]) : 0;
        local += cnt[j];
    }
    const int incl = wave_inclusive_scan_i32(local);
    int run = incl - local;
#pragma unroll
    for (int j = 0; j < kWPL; ++j) {
        L.prefix[lane * kWPL + j] = static_cast<uint32_t>(run);
        run += cnt[j];
    }
    const int total = dpp::lane(incl, 63);
    if (lane == 63) L.total = total;
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    return total;
}

// The same, by wave 0 of a workgroup that synchronizes afterwards.
template <int kWords>
__device__ __forceinline__ void bitmap_prefix(row_lds<kWords> & L, int words) {
    if (threadIdx.x < 64) wave_bitmap_prefix(L, words);
}

// log sum_v exp(l_v / T) of the row from the per-wave sums of exp((l - m) / T).
template <int kWords>
__device__ __forceinline__ float row_log_sum_exp(const row_lds<kWords> & L, float m, float temperature) {
    float s = L.wlse[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) s += L.wlse[w];
    if (m == -INFINITY) return -INFINITY;
    if (m == INFINITY) return INFINITY;
    return m / temperature + logf(s);
}

// Slot of a selected id in ascending id order.
template <int kWords>
__device__ __forceinline__ int slot_of(const row_lds<kWords> & L, int idx) {
    const uint32_t below = (1u << (idx & 31)) - 1u;
    return static_cast<int>(L.prefix[idx >> 5]) + __popc(L.sel[idx >> 5] & below);
}

__device__ __forceinline__ void write_candidate(const levo_hip_sample_args & a, int64_t row, int pos, int idx, float v,
                                                int best, float m, float inv_t, bool z_ok, float inv_z) {
    if (pos >= a.capacity) return;
    const int64_t o = row * a.capacity + pos;
    a.cand_ids[o] = idx;
    if (a.cand_logits) a.cand_logits[o] = v;
    if (a.cand_probs) {
        float p;
        if (z_ok) p = cand_weight(v, m, inv_t) * inv_z;
        else p = idx == best ? 1.0f : 0.0f;  // the reference falls back to best
        a.cand_probs[o] = p;
    }
}

// General selection (k == 0 keeps every id, k > 64, or more tied candidates
// than the gather segments hold): loops over the row again from L2/HBM with
// a block-wide bisection per key bit. Rare; kept out of line so that it does
// not add register pressure to the common path.
template <int kWords>
__device__ __noinline__ void select_general(const levo_hip_sample_args a, row_lds<kWords> & L, int64_t row,
                                            int V, int k, float m, int best, bool pen, bool ign) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float * crow = a.cond + row * a.row_pitch;
    const float * urow = a.uncond ? a.uncond + row * a.row_pitch : nullptr;
    uint32_t tau = 0u;  // k == 0: every valid (non-NaN) id
    if (k == 1) {
        tau = float_key(m);
    } else if (k > 1) {
        int buf = 0;
        for (int bit = 31; bit >= 0; --bit) {
            const uint32_t cand = tau | (1u << bit);
            int cnt = 0;
            for (int idx = tid; idx < V; idx += kThreads)
                cnt += float_key(adjusted_logit(a, L, crow, urow, pen, ign, idx)) >= cand ? 1 : 0;
            cnt = wave_sum_i32(cnt);
            if (lane == 0) L.bis[buf][wave] = cnt;
            __syncthreads();
            int total = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) total += L.bis[buf][w];
            if (total >= k) tau = cand;
            buf ^= 1;
        }
    }
    const bool want_probs = a.cand_probs != nullptr;
    const float inv_t = want_probs ? 1.0f / a.temperature : 0.0f;
    double z = 0.0;
    for (int idx = tid; idx < V; idx += kThreads) {
        const float v = adjusted_logit(a, L, crow, urow, pen, ign, idx);
        if (float_key(v) >= tau) {
            atomicOr(&L.sel[idx >> 5], 1u << (idx & 31));
            if (want_probs) z += static_cast<double>(cand_weight(v, m, inv_t));
        }
    }
    z = wave_sum_f64(z);
    if (lane == 0) L.wz[wave] = z;
    __syncthreads();
    bitmap_prefix(L, (V + 31) / 32);
    z = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) z += L.wz[w];
    const bool z_ok = z > 0.0 && __builtin_isfinite(z);
    const float inv_z = z_ok ? static_cast<float>(1.0 / z) : 0.0f;
    __syncthreads();
    for (int idx = tid; idx < V; idx += kThreads) {
        const float v = adjusted_logit(a, L, crow, urow, pen, ign, idx);
        if (float_key(v) >= tau) write_candidate(a, row, slot_of(L, idx), idx, v, best, m, inv_t, z_ok, inv_z);
    }
}

template <int VEC, int NCH, bool kFull>
// Seven waves per SIMD (72 VGPRs: three rows per CU) up to 36 logits per
// thread; the 64-logit rows of the longest vocabularies take four.
__global__ __launch_bounds__(kThreads, VEC * NCH <= 36 ? 7 : 4) void cfg_sample_kernel(const levo_hip_sample_args a) {
    constexpr int ITEMS = VEC * NCH;
    constexpr int kChunk = kThreads * VEC;                // ids per chunk
    constexpr int kWords = (ITEMS * kThreads + 31) / 32;  // bitmap words covering the row
    constexpr float kLog2e = 1.44269504088896340736f;
    __shared__ row_lds<kWords> L;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const int V = static_cast<int>(a.vocab);
    const int stream = static_cast<int>(row % a.n_streams);
    int k = a.top_k[stream];
    if (k <= 0 || k >= V) k = 0;  // keep every id
    const int words = (V + 31) / 32;
    // exp2 scale of the streamed sum: log2(e) / T when the log-sum-exp is
    // wanted (the temperature is then validated), log2(e) otherwise (the sum
    // then only detects NaN / +inf)
    const float c2 = a.row_lse ? (1.0f / a.temperature) * kLog2e : kLog2e;

    // ---- A. load + CFG + streamed statistics -----------------------------------------
    // All loads of the row are issued before any is consumed (no branch
    // between them: ids past V read a clamped, valid address and are masked
    // to -inf). The penalty / ignore lists are read after the row (requesting
    // them ahead of it measured slower: one more load in every row's queue).
    const bool use_pen = a.recent != nullptr && a.n_recent > 0;
    const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
    const bool adjusted = use_pen || use_ign;  // uniform per workgroup
    const int n_pen = use_pen ? a.n_recent : 0;
    const int n_ign = use_ign ? a.n_ignore : 0;
    const int64_t * rec = use_pen ? a.recent + row * a.n_recent : &kNoListEntry;
    const int64_t * ign = use_ign ? a.ignore : &kNoListEntry;
    float v[ITEMS];
    row_stats st;
    const float * crow = a.cond + row * a.row_pitch;
    if (a.uncond) load_row<VEC, NCH, true, kFull>(v, st, crow, a.uncond + row * a.row_pitch, V, tid, a.cfg_scale, c2);
    else load_row<VEC, NCH, false, kFull>(v, st, crow, crow, V, tid, a.cfg_scale, c2);
    for (int i = tid; i < words; i += kThreads) L.sel[i] = 0u;

    bool has_nan;  // a NaN (exact), or in the streamed case possibly a +inf
    float tmax;
    if (adjusted) {
        for (int i = tid; i < words; i += kThreads) {
            L.pen[i] = 0u;
            L.ign[i] = 0u;
        }
        __syncthreads();
        const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
        for (int i = tid; i < n_pen + n_ign; i += kThreads) {
            const int64_t t = list_entry(rec, n_pen, ign, n_ign, i);
            if (i < n_pen) {
                if (t >= 0 && t < limit) atomicOr(&L.pen[t >> 5], 1u << (t & 31));
            } else {
                if (t >= 0 && t < V) atomicOr(&L.ign[t >> 5], 1u << (t & 31));
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
            if (idx < V) {
                const uint32_t bit = 1u << (idx & 31);
                if (L.pen[idx >> 5] & bit) v[i] = v[i] / a.repetition_penalty;
                if (L.ign[idx >> 5] & bit) v[i] = -INFINITY;
            }
        }
        // the streamed statistics predate the adjustment: exact NaN check and
        // thread maximum (fmaxf skips NaN); the log-sum-exp is recomputed below
        has_nan = false;
        tmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            has_nan = has_nan || __builtin_isnan(v[i]);
            tmax = fmaxf(tmax, v[i]);
        }
    } else {
        tmax = st.tmax;
        has_nan = __builtin_isnan(st.s);
    }
    const bool tvalid = tid * VEC < V;

    // ---- B. wave maximum and the per-wave lower bound of the k-th value ----------
    const float wm = wave_max_f32(tmax);
    const bool wnan = __ballot(has_nan) != 0;
    // Each wave bounds its own ceil(k/8)-th largest lane maximum; the row
    // bound is the smallest of the eight, so at least 8 * ceil(k/8) >= k ids
    // lie at or above it (lanes without valid ids contribute key 0 = -inf).
    const int kw = (k + kWaves - 1) / kWaves;
    float wlow = -INFINITY;
    if (k > 1 && kw <= 64) {
        const uint32_t kk = wave_kth_key(tvalid ? float_key(tmax) : 0u, kw);
        wlow = kk == 0u ? -INFINITY : float_of_key(kk);
    }
    if (lane == 0) {
        L.wmax[wave] = wm;
        L.wlow[wave] = wlow;
        L.wnan[wave] = wnan ? 1 : 0;
    }
    __syncthreads();  // barrier 1

    float m = L.wmax[0];
    float low = L.wlow[0];
    bool row_nan = L.wnan[0] != 0;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        m = fmaxf(m, L.wmax[w]);
        low = fminf(low, L.wlow[w]);
        row_nan = row_nan || L.wnan[w] != 0;
    }
    if (row_nan && !adjusted) {  // uniform: a streamed sum went NaN; NaN or +inf?
        bool hn = false;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) hn = hn || __builtin_isnan(v[i]);
        hn = __ballot(hn) != 0;
        __syncthreads();  // every wave has read the flags above
        if (lane == 0) L.wnan[wave] = hn ? 1 : 0;
        __syncthreads();
        row_nan = false;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) row_nan = row_nan || L.wnan[w] != 0;
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
    if (k == 1) low = m;  // the candidates are the ties with the maximum

    // ---- C. first maximum, log-sum-exp, candidate gather ---------------------------
    // first id equal to the maximum; its own value is the reference's max_logit
    // (std::max keeps the first of equal values, so a -0 / +0 tie keeps its sign)
    int tbest = INT_MAX;
    float tbest_v = m;
    if (tvalid && tmax == m) {
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
            if (tbest == INT_MAX && idx < V && v[i] == m) {
                tbest = idx;
                tbest_v = v[i];
            }
        }
    }
    const int my_best = tbest;
    tbest = wave_min_i32(tbest);
    if (lane == 0) L.wbest[wave] = tbest;
    if (my_best == tbest && my_best != INT_MAX) L.wbv[wave] = tbest_v;

    if (a.row_lse) {
        float s;
        if (adjusted) {
            const float inv_t = 1.0f / a.temperature;
            s = 0.0f;
#pragma unroll
            for (int i = 0; i < ITEMS; ++i) s += __expf((v[i] - m) * inv_t);  // padding: exp(-inf) = 0
        } else {
            // streamed sum, rescaled from the thread's shift to the row maximum
            // (only a finite m reaches the log-sum-exp below)
            s = st.s * __builtin_amdgcn_exp2f((st.sh - fmaxf(m, -FLT_MAX)) * c2);
        }
        s = wave_sum_f32(s);
        if (lane == 0) L.wlse[wave] = s;
    }

    // Gather the ids >= low into this wave's segment, in item order. The
    // running count is wave-uniform, so slots need no atomics. Padding ids hold
    // -inf: a row whose bound is -inf takes the general path unless it is full.
    const bool gather = k >= 1 && kw <= 64 && (kFull || low > -INFINITY);
    if (gather) {
        int base = 0;
#pragma unroll
        for (int i = 0; i < ITEMS; ++i) {
            const int idx = (i / VEC) * kChunk + tid * VEC + (i % VEC);
            const bool p = v[i] >= low;
            const uint64_t mask = __ballot(p);
            if (mask) {
                const int pos = base + rank_in_mask(mask);
                if (p && pos < kSegCap) {
                    L.cv[wave][pos] = v[i];
                    L.ci[wave][pos] = idx;
                }
                base += static_cast<int>(__popcll(mask));
            }
        }
        if (lane == 0) L.wcnt[wave] = base;
    }
    __syncthreads();  // barrier 2

    int best = L.wbest[0];
    int best_wave = 0;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        if (L.wbest[w] < best) {
            best = L.wbest[w];
            best_wave = w;
        }
    }
    int seg_start[kWaves + 1];
    seg_start[0] = 0;
    bool fits = gather;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int c = fits ? L.wcnt[w] : 0;
        fits = fits && c <= kSegCap;
        seg_start[w + 1] = seg_start[w] + c;
    }
    const int ncand = seg_start[kWaves];
    fits = fits && ncand <= kBisCap;

    if (!fits) {  // uniform: every wave takes the general path
        select_general(a, L, row, V, k, m, best, use_pen, use_ign);
        if (my_best == best && a.row_max) a.row_max[row] = tbest_v;
        if (tid == 0) {
            a.best[row] = best;
            a.count[row] = L.total;
            if (a.row_lse) a.row_lse[row] = row_log_sum_exp(L, m, a.temperature);
        }
        return;
    }

    // The candidates are in LDS: the other waves leave, so that their
    // registers take the next row's loads while wave 0 finishes this one
    // (no workgroup barrier after this point). Wave 1 writes the row's
    // scalars on its way out.
    if (wave != 0) {
        if (wave == 1 && lane == 0) {
            a.best[row] = best;
            if (a.row_max) a.row_max[row] = L.wbv[best_wave];
            if (a.row_lse) a.row_lse[row] = row_log_sum_exp(L, m, a.temperature);
        }
        return;
    }

    // ---- D. exact k-th value (key) among the gathered candidates ------------------
    // Candidate j = lane + 64 * s in segment order sits at flat index
    // j + delta[w] of the segment array (delta[w] = w * kSegCap - seg_start[w]);
    // every load is issued before any is used, with no branch between them.
    constexpr int kSlots = kBisCap / 64;
    float cval[kSlots];
    int cidx[kSlots];
    uint32_t keys[kSlots];
    bool valid[kSlots];
    {
        const float * cv = &L.cv[0][0];
        const int * ci = &L.ci[0][0];
        int flat[kSlots];
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const int j = lane + 64 * s;
            int delta = -seg_start[0];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) delta = j >= seg_start[q] ? q * kSegCap - seg_start[q] : delta;
            valid[s] = j < ncand;
            flat[s] = valid[s] ? j + delta : 0;
        }
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            cval[s] = cv[flat[s]];
            cidx[s] = ci[flat[s]];
        }
#pragma unroll
        for (int s = 0; s < kSlots; ++s) keys[s] = valid[s] ? float_key(cval[s]) : 0u;
    }
    uint32_t tau;
    if (k == 1) {
        tau = float_key(m);
    } else {
        // tau lies in [low, m]: it shares the common high bits of their keys
        const uint32_t lo_key = low == -INFINITY ? 0u : float_key(low);
        const uint32_t hi_key = float_key(m);
        const uint32_t diff = lo_key ^ hi_key;
        const int top = diff == 0u ? -1 : 31 - __builtin_clz(diff);
        const uint32_t prefix = top < 0 ? lo_key : (lo_key & ~((2u << top) - 1u));
        tau = radix_kth_key<kSlots>(L.hist, keys, valid, k, prefix, top);
    }

    // ---- E. mark the candidates >= tau in the id bitmap; weight sum ---------------
    const bool want_probs = a.cand_probs != nullptr;
    const float inv_t = want_probs ? 1.0f / a.temperature : 0.0f;
    bool take[kSlots];
    float wgt[kSlots];
    double z = 0.0;
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        take[s] = keys[s] >= tau && valid[s];
        wgt[s] = want_probs && take[s] ? cand_weight(cval[s], m, inv_t) : 0.0f;
        if (take[s]) atomicOr(&L.sel[cidx[s] >> 5], 1u << (cidx[s] & 31));
        z += static_cast<double>(wgt[s]);
    }
    z = wave_sum_f64(z);
    const bool z_ok = z > 0.0 && __builtin_isfinite(z);
    const float inv_z = z_ok ? static_cast<float>(1.0 / z) : 0.0f;
    // one wave: its LDS operations complete in issue order, so the prefix
    // pass below reads every bit marked above
    const int total = wave_bitmap_prefix(L, words);

    // ---- write the candidates in ascending id order --------------------------------
    // every slot's lookup is read (id 0 for slots not taken), then waited for once
    int slot[kSlots];
#pragma unroll
    for (int s = 0; s < kSlots; ++s) slot[s] = slot_of(L, take[s] ? cidx[s] : 0);
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
        const int pos = take[s] ? slot[s] : a.capacity;
        if (pos < a.capacity) {
            const int64_t o = row * a.capacity + pos;
            a.cand_ids[o] = cidx[s];
            if (a.cand_logits) a.cand_logits[o] = cval[s];
            if (want_probs) a.cand_probs[o] = z_ok ? wgt[s] * inv_z : (cidx[s] == best ? 1.0f : 0.0f);
        }
    }
    if (lane == 0) a.count[row] = total;
}

template <int VEC, int NCH>
int launch_sample(const levo_hip_sample_args & a, hipStream_t stream) {
    const uint32_t grid = static_cast<uint32_t>(a.rows);
    if (VEC == 4 && a.vocab == int64_t{kThreads} * VEC * NCH)
        cfg_sample_kernel<VEC, NCH, true><<<grid, kThreads, 0, stream>>>(a);
    else
        cfg_sample_kernel<VEC, NCH, false><<<grid, kThreads, 0, stream>>>(a);
    return launch_status("levo_hip_cfg_sample");
}

// ---------------------------------------------------------------------------------------
// Decode-step sampling in two launches (levo_hip_sample_step).
//
// A decode step samples a handful of rows. One workgroup per row pulls each
// row (two 16385-logit inputs under CFG: 131 KB) through one CU, at that CU's
// share of the HBM bandwidth: about 5 us before any selection starts. Here
// every row is split into segments of 4096 ids:
//   1. segment launch, one 512-thread workgroup per (row, segment), 8 ids per
//      thread: loads, CFG, the repetition penalty and the ignore list (the
//      list ids inside the segment); the segment's maximum, first maximum,
//      NaN flag and softmax sum; and the segment's own top-k candidate set,
//      found as the row kernel finds a row's (gather above a per-wave bound,
//      the exact k-th key by a one-wave radix select, ties kept), written to
//      the workspace in ascending id order with the segment's head. The
//      row's k-th largest value is at least every segment's k-th largest, so
//      the union of the segment sets holds every candidate of the row.
//   2. merge launch, one wave per row, 8 rows per workgroup: the row's
//      maximum, first maximum and log-sum-exp from the heads; its k-th key by
//      a radix select over the handed-over candidates (at most 64 per
//      segment, read with the heads in one round trip); and the candidates
//      at or above it, whose ascending id order is the segments' order and
//      each list's own. When every row fits one workgroup it then makes
//      every row's draw, as levo_hip_sample_draw does, after a workgroup
//      barrier; with more rows the draw is a third launch.
// No workgroup waits for another. A row that does not fit (k = 0, k > 512,
// more than 64 candidates in a segment, as with heavy ties) takes
// select_general over the whole row in the merge launch.
constexpr int kStepPer = 8;                       // ids per thread
constexpr int kStepSegIds = kThreads * kStepPer;  // ids per segment
constexpr int kStepSegWords = kStepSegIds / 32;   // bitmap words of a segment
constexpr int kStepCandCap = 256;                 // candidate slots of a segment in the workspace
constexpr int kStepHandCap = 64;                  // candidates per segment the merging wave reads
constexpr int kStepWords = kMaxVocab / 32;        // bitmap words of the longest row
constexpr int kStepMaxSegs = kMaxVocab / kStepSegIds;

struct step_head {
    float max;      // segment maximum (NaN skipped)
    float bv;       // value at its first maximum
    int32_t best;   // first id holding the maximum
    int32_t nan;    // the segment holds a NaN
    uint32_t tau;   // key of the segment's k-th largest value (0: fewer than k ids)
    int32_t count;  // candidates handed over in ascending id order; -1: none (general path)
    float sum;      // sum over the segment of exp((l - max) / T)
    int32_t pad;
};

struct step_seg {
    step_head h;
    float val[kStepCandCap];
    int32_t id[kStepCandCap];
};

// The workspace starts with a reserved region of fixed size, the same for
// every row count and vocabulary; the segment records follow.
constexpr int kStepCounters = 4096;
constexpr int64_t kStepCounterBytes = kStepCounters * 4;
constexpr int64_t kStepMaxRows = kStepCounters - 1;

// Id of item q of thread tid in a segment starting at lo: dwordx4 chunks of
// 4 ids per thread (VEC 4) or single ids kThreads apart (VEC 1); coalesced
// either way.
template <int VEC>
__device__ __forceinline__ int step_id(int lo, int tid, int q) {
    return VEC == 4 ? lo + (q / 4) * kThreads * 4 + tid * 4 + (q % 4) : lo + tid + kThreads * q;
}

template <int VEC>
__global__ __launch_bounds__(kThreads) void step_segment_kernel(const levo_hip_sample_args a, uint8_t * ws, int segs) {
    __shared__ row_lds<kStepSegWords> L;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x / segs;
    const int seg = static_cast<int>(blockIdx.x % segs);
    const int V = static_cast<int>(a.vocab);
    const int lo = seg * kStepSegIds;
    const int hi = lo + kStepSegIds < V ? lo + kStepSegIds : V;
    const int stream = static_cast<int>(row % a.n_streams);
    int k = a.top_k[stream];
    if (k <= 0 || k >= V) k = 0;  // keep every id
    const int kw = (k + kWaves - 1) / kWaves;
    step_seg & out = reinterpret_cast<step_seg *>(ws + kStepCounterBytes)[row * segs + seg];

    // ---- 1. loads, CFG, penalty, ignore list, reductions ------------------------------
    // the list entries first (see list_entry), then the segment's logits
    const bool use_pen = a.recent != nullptr && a.n_recent > 0;
    const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
    const int n_pen = use_pen ? a.n_recent : 0;
    const int n_ign = use_ign ? a.n_ignore : 0;
    const int64_t * rec = use_pen ? a.recent + row * a.n_recent : &kNoListEntry;
    const int64_t * ign = use_ign ? a.ignore : &kNoListEntry;
    const int64_t entry = list_entry(rec, n_pen, ign, n_ign, tid);
    const float * crow = a.cond + row * a.row_pitch;
    const float * urow = a.uncond ? a.uncond + row * a.row_pitch : nullptr;
    float c[kStepPer], u[kStepPer];
    if constexpr (VEC == 4) {
#pragma unroll
        for (int ch = 0; ch < kStepPer / 4; ++ch) {
            const int base = step_id<VEC>(lo, tid, ch * 4);
            const int off = base < V ? base : lo;  // row_pitch % 4 == 0: in bounds
            const f32x4 cv = *reinterpret_cast<const f32x4 *>(crow + off);
            const f32x4 uv = urow ? *reinterpret_cast<const f32x4 *>(urow + off) : cv;
            c[ch * 4] = cv.x; c[ch * 4 + 1] = cv.y; c[ch * 4 + 2] = cv.z; c[ch * 4 + 3] = cv.w;
            u[ch * 4] = uv.x; u[ch * 4 + 1] = uv.y; u[ch * 4 + 2] = uv.z; u[ch * 4 + 3] = uv.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < kStepPer; ++q) {
            const int id = step_id<VEC>(lo, tid, q);
            const int off = id < V ? id : lo;
            c[q] = crow[off];
            u[q] = urow ? urow[off] : c[q];
        }
    }
    if (tid < kStepSegWords) L.sel[tid] = 0u;

    // Penalty and ignore ids inside this segment, as bitmaps of its 4096 ids
    // (128 words each).
    int pen = 0, ign_bits = 0;  // item bits
    if (use_pen || use_ign) {
        if (tid < kStepSegIds / 32) {
            L.pen[tid] = 0u;
            L.ign[tid] = 0u;
        }
        __syncthreads();
        const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
        const int64_t top = hi < limit ? hi : limit;
        for (int i = tid; i < n_pen + n_ign; i += kThreads) {
            const int64_t t = i < kThreads ? entry : list_entry(rec, n_pen, ign, n_ign, i);
            if (i < n_pen) {
                if (t >= lo && t < top) atomicOr(&L.pen[(t - lo) >> 5], 1u << ((t - lo) & 31));
            } else {
                if (t >= lo && t < hi) atomicOr(&L.ign[(t - lo) >> 5], 1u << ((t - lo) & 31));
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kStepPer; ++q) {
            const int rel = step_id<VEC>(lo, tid, q) - lo;
            pen |= (L.pen[rel >> 5] >> (rel & 31)) & 1u ? 1 << q : 0;
            ign_bits |= (L.ign[rel >> 5] >> (rel & 31)) & 1u ? 1 << q : 0;
        }
    }
    float v[kStepPer];
    bool has_nan = false;
    float tmax = -INFINITY;
#pragma unroll
    for (int q = 0; q < kStepPer; ++q) {
        float x = urow ? u[q] + a.cfg_scale * (c[q] - u[q]) : c[q];
        if (pen & (1 << q)) x = x / a.repetition_penalty;
        if (ign_bits & (1 << q)) x = -INFINITY;
        v[q] = step_id<VEC>(lo, tid, q) < hi ? x : -INFINITY;
        has_nan = has_nan || __builtin_isnan(v[q]);
        tmax = fmaxf(tmax, v[q]);
    }
    const bool tvalid = step_id<VEC>(lo, tid, 0) < hi;

    // ---- 2. segment reductions and the per-wave bound of the k-th value -------------------
    const float wm = wave_max_f32(tmax);
    const bool wnan = __ballot(has_nan) != 0;
    float wlow = -INFINITY;
    if (k > 1 && kw <= 64) {
        const uint32_t kk = wave_kth_key(tvalid ? float_key(tmax) : 0u, kw);
        wlow = kk == 0u ? -INFINITY : float_of_key(kk);
    }
    if (lane == 0) {
        L.wmax[wave] = wm;
        L.wlow[wave] = wlow;
        L.wnan[wave] = wnan ? 1 : 0;
    }
    __syncthreads();
    float m = L.wmax[0];
    float low = L.wlow[0];
    bool seg_nan = L.wnan[0] != 0;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        m = fmaxf(m, L.wmax[w]);
        low = fminf(low, L.wlow[w]);
        seg_nan = seg_nan || L.wnan[w] != 0;
    }
    if (k == 1) low = m;
    int tbest = INT_MAX;
    float tbest_v = m;
#pragma unroll
    for (int q = 0; q < kStepPer; ++q) {
        const int id = step_id<VEC>(lo, tid, q);
        if (id < hi && v[q] == m && id < tbest) {
            tbest = id;
            tbest_v = v[q];
        }
    }
    const int my_best = tbest;
    tbest = wave_min_i32(tbest);
    if (lane == 0) L.wbest[wave] = tbest;
    if (my_best == tbest && my_best != INT_MAX) L.wbv[wave] = tbest_v;
    if (a.row_lse) {
        const float inv_t = 1.0f / a.temperature;
        const float mm = fmaxf(m, -FLT_MAX);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < kStepPer; ++q) s += __expf((v[q] - mm) * inv_t);  // -inf and padding add 0
        s = wave_sum_f32(s);
        if (lane == 0) L.wlse[wave] = s;
    }
    // gather the ids >= low (k >= 1), padding excluded, into the wave's
    // kSegCap slots; a longer count only marks the segment as not fitting
    const bool gather = k >= 1 && kw <= 64 && !seg_nan;
    if (gather) {
        int base = 0;
#pragma unroll
        for (int q = 0; q < kStepPer; ++q) {
            const int id = step_id<VEC>(lo, tid, q);
            const bool p = id < hi && v[q] >= low;
            const uint64_t mask = __ballot(p);
            if (mask) {
                const int pos = base + rank_in_mask(mask);
                if (p && pos < kSegCap) {
                    L.cv[wave][pos] = v[q];
                    L.ci[wave][pos] = id;
                }
                base += static_cast<int>(__popcll(mask));
            }
        }
        if (lane == 0) L.wcnt[wave] = base;
    }
    __syncthreads();
    if (wave != 0) return;

    // ---- 3. wave 0: the segment's exact k-th key and its candidates in id order ------------
    int best = L.wbest[0], bw = 0;
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
        if (L.wbest[w] < best) {
            best = L.wbest[w];
            bw = w;
        }
    }
    float sum = 0.0f;
    if (a.row_lse) {
        sum = L.wlse[0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) sum += L.wlse[w];
    }
    int seg_start[kWaves + 1];
    seg_start[0] = 0;
    bool fits = gather;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        const int c = fits ? L.wcnt[w] : 0;
        fits = fits && c <= kSegCap;
        seg_start[w + 1] = seg_start[w] + c;
    }
    const int ncand = seg_start[kWaves];
    fits = fits && ncand <= kBisCap;
    int count = -1;
    uint32_t tau = 0u;
    if (fits) {  // uniform
        constexpr int kSlots = kBisCap / 64;
        float cval[kSlots];
        int cidx[kSlots];
        uint32_t keys[kSlots];
        bool valid[kSlots];
        const float * cv = &L.cv[0][0];
        const int * ci = &L.ci[0][0];
        int flat[kSlots];
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            const int j = lane + 64 * s;
            int delta = -seg_start[0];
#pragma unroll
            for (int q = 1; q < kWaves; ++q) delta = j >= seg_start[q] ? q * kSegCap - seg_start[q] : delta;
            valid[s] = j < ncand;
            flat[s] = valid[s] ? j + delta : 0;
        }
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            cval[s] = cv[flat[s]];
            cidx[s] = ci[flat[s]];
        }
#pragma unroll
        for (int s = 0; s < kSlots; ++s) keys[s] = valid[s] ? float_key(cval[s]) : 0u;
        if (k == 1) {
            tau = float_key(m);
        } else {
            const uint32_t lo_key = low == -INFINITY ? 0u : float_key(low);
            const uint32_t hi_key = float_key(m);
            const uint32_t diff = lo_key ^ hi_key;
            const int top = diff == 0u ? -1 : 31 - __builtin_clz(diff);
            const uint32_t prefix = top < 0 ? lo_key : (lo_key & ~((2u << top) - 1u));
            tau = radix_kth_key<kSlots>(L.hist, keys, valid, k, prefix, top);
        }
        bool take[kSlots];
#pragma unroll
        for (int s = 0; s < kSlots; ++s) {
            take[s] = valid[s] && keys[s] >= tau;
            if (take[s]) atomicOr(&L.sel[(cidx[s] - lo) >> 5], 1u << ((cidx[s] - lo) & 31));
        }
        const int total = wave_bitmap_prefix(L, kStepSegWords);
        if (total <= kStepCandCap) {
            count = total;
            int slot[kSlots];  // every lookup issued, then waited for once
#pragma unroll
            for (int s = 0; s < kSlots; ++s) slot[s] = slot_of(L, take[s] ? cidx[s] - lo : 0);
#pragma unroll
            for (int s = 0; s < kSlots; ++s) {
                if (take[s]) {
                    out.val[slot[s]] = cval[s];
                    out.id[slot[s]] = cidx[s];
                }
            }
        }
    }
    if (lane == 0) {
        step_head h;
        h.max = m;
        h.bv = best == INT_MAX ? m : L.wbv[bw];
        h.best = best;
        h.nan = seg_nan ? 1 : 0;
        h.tau = tau;
        h.count = count;
        h.sum = sum;
        h.pad = 0;
        out.h = h;
    }
}

struct merge_lds {
    row_lds<kStepWords> L;                           // the general path
    __attribute__((aligned(16))) uint32_t hist[kWaves][256];  // one radix-select histogram per wave
    int slow[kWaves];                                // rows that take the general path
    float rm[kWaves];
    int best[kWaves];
    float bv[kWaves];
    float lse[kWaves];
};

__global__ __launch_bounds__(kThreads) void step_merge_kernel(const levo_hip_sample_args a, const levo_hip_draw_args d,
                                                               const uint8_t * ws, int segs) {
    __shared__ merge_lds S;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kWaves + wave;
    const bool live = row < a.rows;  // uniform per wave
    const int V = static_cast<int>(a.vocab);
    if (live) {
        const int stream = static_cast<int>(row % a.n_streams);
        int k = a.top_k[stream];
        if (k <= 0 || k >= V) k = 0;
        const int kw = (k + kWaves - 1) / kWaves;
        const step_seg * segv = reinterpret_cast<const step_seg *>(ws + kStepCounterBytes) + row * segs;
        // every load first: lane g < segs takes head g, and every lane the
        // first kStepHandCap candidate slots of each segment
        const step_head h = segv[lane < segs ? lane : 0].h;
        float cval[kStepMaxSegs];
        int cidx[kStepMaxSegs];
#pragma unroll
        for (int s = 0; s < kStepMaxSegs; ++s) {
            const int g = s < segs ? s : 0;
            cval[s] = segv[g].val[lane];
            cidx[s] = segv[g].id[lane];
        }
        const bool mine = lane < segs;
        const bool row_nan = __ballot(mine && h.nan != 0) != 0;
        const float rm = wave_max_f32(mine ? h.max : -INFINITY);
        // the first maximum lies in the first segment whose maximum is the row's
        const uint64_t at_max = __ballot(mine && h.max == rm && h.best != INT_MAX);
        const int bseg = at_max != 0 ? __builtin_ctzll(at_max) : 0;
        const int best = at_max != 0 ? dpp::lane(h.best, bseg) : -1;
        const float bv = dpp::lane(h.bv, bseg);
        float lse = NAN;
        if (!row_nan && a.row_lse) {
            if (rm == -INFINITY) {
                lse = -INFINITY;
            } else if (rm == INFINITY) {
                lse = INFINITY;
            } else {
                const float inv_t = 1.0f / a.temperature;
                float z = 0.0f;
                for (int g = 0; g < segs; ++g)
                    z += dpp::lane(h.sum, g) * __expf((fmaxf(dpp::lane(h.max, g), -FLT_MAX) - rm) * inv_t);
                lse = rm / a.temperature + logf(z);
            }
        }
        const bool counts_ok = __ballot(mine && (h.count < 0 || h.count > kStepHandCap)) == 0;
        const bool fast = !row_nan && k >= 1 && kw <= 64 && counts_ok;
        if (row_nan) {  // the reference throws "logits contain NaN"
            if (lane == 0) {
                a.best[row] = -1;
                a.count[row] = -1;
                if (a.row_max) a.row_max[row] = NAN;
                if (a.row_lse) a.row_lse[row] = NAN;
            }
        } else if (fast) {
            // The row's k-th key is at least every segment's (a segment with
            // fewer than k ids reports 0): candidates below the largest of
            // them cannot be selected and are left out, so the rest lie
            // between it and the maximum's key.
            const uint32_t lo_key =
                k == 1 ? 0u : dpp::allreduce(mine ? h.tau : 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
            uint32_t keys[kStepMaxSegs];
            bool valid[kStepMaxSegs];
#pragma unroll
            for (int s = 0; s < kStepMaxSegs; ++s) {
                const int c = s < segs ? dpp::lane(h.count, s) : 0;
                keys[s] = float_key(cval[s]);
                valid[s] = lane < c && keys[s] >= lo_key;
                keys[s] = valid[s] ? keys[s] : 0u;
            }
            uint32_t tau;
            if (k == 1) {
                tau = float_key(rm);
            } else {
                // it shares the common high bits of lo_key and the maximum's key
                const uint32_t hi_key = float_key(rm);
                const uint32_t diff = lo_key ^ hi_key;
                const int top = diff == 0u ? -1 : 31 - __builtin_clz(diff);
                const uint32_t prefix = top < 0 ? lo_key : (lo_key & ~((2u << top) - 1u));
                tau = radix_kth_key<kStepMaxSegs>(S.hist[wave], keys, valid, k, prefix, top);
            }
            // slot = candidates taken in earlier segments + rank within this one
            const bool want_probs = a.cand_probs != nullptr;
            const float inv_t = want_probs ? 1.0f / a.temperature : 0.0f;
            bool take[kStepMaxSegs];
            int pos[kStepMaxSegs];
            float wgt[kStepMaxSegs];
            int total = 0;
            double z = 0.0;
#pragma unroll
            for (int s = 0; s < kStepMaxSegs; ++s) {
                take[s] = valid[s] && keys[s] >= tau;
                const uint64_t mask = __ballot(take[s]);
                pos[s] = total + rank_in_mask(mask);
                total += static_cast<int>(__popcll(mask));
                wgt[s] = want_probs && take[s] ? cand_weight(cval[s], rm, inv_t) : 0.0f;
                z += static_cast<double>(wgt[s]);
            }
            z = wave_sum_f64(z);
            const bool z_ok = z > 0.0 && __builtin_isfinite(z);
            const float inv_z = z_ok ? static_cast<float>(1.0 / z) : 0.0f;
#pragma unroll
            for (int s = 0; s < kStepMaxSegs; ++s) {
                if (take[s] && pos[s] < a.capacity) {
                    const int64_t o = row * a.capacity + pos[s];
                    a.cand_ids[o] = cidx[s];
                    if (a.cand_logits) a.cand_logits[o] = cval[s];
                    if (want_probs) a.cand_probs[o] = z_ok ? wgt[s] * inv_z : (cidx[s] == best ? 1.0f : 0.0f);
                }
            }
            if (lane == 0) {
                a.best[row] = best;
                a.count[row] = total;
                if (a.row_max) a.row_max[row] = bv;
                if (a.row_lse) a.row_lse[row] = lse;
            }
        }
        if (lane == 0) {
            S.slow[wave] = !row_nan && !fast ? 1 : 0;
            S.rm[wave] = rm;
            S.best[wave] = best;
            S.bv[wave] = bv;
            S.lse[wave] = lse;
        }
    } else if (lane == 0) {
        S.slow[wave] = 0;
    }
    __syncthreads();

    // ---- rows that do not fit: the whole row again, by the whole workgroup ------------------
    const int words = (V + 31) / 32;
    for (int w = 0; w < kWaves; ++w) {
        if (!S.slow[w]) continue;  // uniform
        const int64_t r = static_cast<int64_t>(blockIdx.x) * kWaves + w;
        const int stream = static_cast<int>(r % a.n_streams);
        int k = a.top_k[stream];
        if (k <= 0 || k >= V) k = 0;
        const bool use_pen = a.recent != nullptr && a.n_recent > 0;
        const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
        row_lds<kStepWords> & L = S.L;
        for (int i = tid; i < words; i += kThreads) {
            L.sel[i] = 0u;
            L.pen[i] = 0u;
            L.ign[i] = 0u;
        }
        __syncthreads();
        if (use_pen) {
            const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
            const int64_t * rec = a.recent + r * a.n_recent;
            for (int i = tid; i < a.n_recent; i += kThreads) {
                const int64_t t = rec[i];
                if (t >= 0 && t < limit) atomicOr(&L.pen[t >> 5], 1u << (t & 31));
            }
        }
        if (use_ign) {
            for (int i = tid; i < a.n_ignore; i += kThreads) {
                const int64_t t = a.ignore[i];
                if (t >= 0 && t < V) atomicOr(&L.ign[t >> 5], 1u << (t & 31));
            }
        }
        __syncthreads();
        select_general(a, L, r, V, k, S.rm[w], S.best[w], use_pen, use_ign);
        if (tid == 0) {
            a.best[r] = S.best[w];
            a.count[r] = L.total;
            if (a.row_max) a.row_max[r] = S.bv[w];
            if (a.row_lse) a.row_lse[r] = S.lse[w];
        }
        __syncthreads();  // the next row reuses the bitmaps
    }

    // ---- the draw of every row (all rows are in this workgroup) ----------------------------
    if (d.tokens == nullptr) return;
    __syncthreads();  // every row's outputs are written and visible to the workgroup
    if (live) draw_row(d, row);
}

int64_t step_segments(int64_t vocab) { return (vocab + kStepSegIds - 1) / kStepSegIds; }

int64_t step_workspace_bytes(int64_t rows, int64_t vocab) {
    return kStepCounterBytes + rows * step_segments(vocab) * static_cast<int64_t>(sizeof(step_seg));
}

}  // namespace
}  // namespace levo_hip

using namespace levo_hip;

namespace {

// The checks of levo_hip_cfg_sample (the reference's messages where it has one).
int check_sample_args(const levo_hip_sample_args & a) {
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
    LEVO_REQUIRE(a.n_recent <= (1 << 30) && a.n_ignore <= (1 << 30), "cfg_sample: list longer than 2^30 ids");
    LEVO_REQUIRE((a.cand_probs == nullptr && a.row_lse == nullptr) ||
                     (a.temperature > 0.0f && __builtin_isfinite(a.temperature)),
                 "temperature must be finite and positive for softmax outputs");
    return LEVO_HIP_OK;
}

// The checks of levo_hip_sample_draw.
int check_draw_args(const levo_hip_draw_args & a) {
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
    return LEVO_HIP_OK;
}

// Validates a sample_step call and launches it on `ws` (counters zero).
int launch_step(const levo_hip_sample_args * args, const levo_hip_draw_args * draw, void * ws, int64_t ws_bytes,
                hipStream_t stream) {
    LEVO_REQUIRE(args != nullptr, "sample_step: null argument block");
    const levo_hip_sample_args & a = *args;
    const int st = check_sample_args(a);
    if (st != LEVO_HIP_OK || a.rows == 0) return st;
    levo_hip_draw_args d{};
    if (draw != nullptr) {
        d = *draw;
        const int sd = check_draw_args(d);
        if (sd != LEVO_HIP_OK) return sd;
        LEVO_REQUIRE(d.rows == a.rows && d.capacity == a.capacity && d.best == a.best && d.count == a.count &&
                         d.cand_ids == a.cand_ids && d.cand_logits == a.cand_logits && d.row_max == a.row_max,
                     "sample_step: the draw must read the rows' own candidate outputs");
    }
    const int64_t segs = step_segments(a.vocab);
    LEVO_REQUIRE(a.rows <= kStepMaxRows, "sample_step: more than %lld rows", static_cast<long long>(kStepMaxRows));
    LEVO_REQUIRE(ws != nullptr && aligned16(ws), "sample_step: workspace must be 16-byte aligned device memory");
    LEVO_REQUIRE(ws_bytes >= step_workspace_bytes(a.rows, a.vocab),
                 "sample_step: workspace smaller than levo_hip_sample_step_workspace_bytes");
    const uint32_t grid = static_cast<uint32_t>(a.rows * segs);
    const bool vec = a.row_pitch % 4 == 0 && aligned16(a.cond) && (a.uncond == nullptr || aligned16(a.uncond));
    uint8_t * w = static_cast<uint8_t *>(ws);
    if (vec) step_segment_kernel<4><<<grid, kThreads, 0, stream>>>(a, w, static_cast<int>(segs));
    else step_segment_kernel<1><<<grid, kThreads, 0, stream>>>(a, w, static_cast<int>(segs));
    const int sa = launch_status("levo_hip_sample_step");
    if (sa != LEVO_HIP_OK) return sa;
    // the merge launch draws when every row is in its one workgroup; otherwise
    // the draw is a launch of its own
    const uint32_t merge_groups = static_cast<uint32_t>(ceil_div(a.rows, kWaves));
    levo_hip_draw_args dm = d;
    if (merge_groups > 1) dm.tokens = nullptr;
    step_merge_kernel<<<merge_groups, kThreads, 0, stream>>>(a, dm, w, static_cast<int>(segs));
    const int sb = launch_status("levo_hip_sample_step");
    if (sb != LEVO_HIP_OK || draw == nullptr || merge_groups == 1) return sb;
    return levo_hip_sample_draw(&d, reinterpret_cast<levo_hip_stream_t>(stream));
}

}  // namespace

// ---- levo_hip_sample_step_static: the step on library-held scratch ----------------------
// Callers that cannot allocate (graph capture, serving loops) get the
// workspace from this array: one copy per GPU, held until the process ends.
// Every call writes the segment records it reads, so nothing needs clearing.
// Calls that overlap on one GPU share the array and race.
constexpr int64_t kStaticScratchBytes = int64_t{2} << 20;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

namespace {

// The device address of `scratch` on the current device, found once per
// device (with that device current) and kept; the host-side name is only a
// stand-in.
int scratch_address(void ** out) {
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static void * ptrs[kMaxDevices] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        set_error("sample_step_static: cannot query the current device");
        return LEVO_HIP_ERR_RUNTIME;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[device] == nullptr) {
        void * p = nullptr;
        const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || p == nullptr) {
            set_error("sample_step_static: cannot find the scratch array on device %d: %s", device,
                      hipGetErrorString(err));
            return LEVO_HIP_ERR_RUNTIME;
        }
        ptrs[device] = p;
    }
    *out = ptrs[device];
    return LEVO_HIP_OK;
}

}  // namespace

extern "C" int levo_hip_cfg_sample(const levo_hip_sample_args * args, levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "cfg_sample: null argument block");
    const levo_hip_sample_args & a = *args;
    const int checked = check_sample_args(a);
    if (checked != LEVO_HIP_OK || a.rows == 0) return checked;
    const hipStream_t st = as_hip(stream);
    const bool vec = a.row_pitch % 4 == 0 && aligned16(a.cond) && (a.uncond == nullptr || aligned16(a.uncond));
    const int64_t V = a.vocab;
    if (vec) {
        if (V <= 2048) return launch_sample<4, 1>(a, st);
        if (V <= 4096) return launch_sample<4, 2>(a, st);
        if (V <= 8192) return launch_sample<4, 4>(a, st);
        if (V <= 16384) return launch_sample<4, 8>(a, st);
        if (V <= 18432) return launch_sample<4, 9>(a, st);
        return launch_sample<4, 16>(a, st);
    }
    if (V <= 512) return launch_sample<1, 1>(a, st);
    if (V <= 2048) return launch_sample<1, 4>(a, st);
    if (V <= 8192) return launch_sample<1, 16>(a, st);
    if (V <= 16384) return launch_sample<1, 32>(a, st);
    if (V <= 16896) return launch_sample<1, 33>(a, st);
    return launch_sample<1, 64>(a, st);
}

extern "C" int64_t levo_hip_sample_step_workspace_bytes(int64_t rows, int64_t vocab) {
    if (rows < 1 || rows > kStepMaxRows || vocab < 1 || vocab > kMaxVocab) return LEVO_HIP_ERR_INVALID;
    return step_workspace_bytes(rows, vocab);
}

extern "C" int levo_hip_sample_step(const levo_hip_sample_args * args, const levo_hip_draw_args * draw,
                                    void * workspace, int64_t workspace_bytes, levo_hip_stream_t stream) {
    return launch_step(args, draw, workspace, workspace_bytes, as_hip(stream));
}

extern "C" int levo_hip_sample_step_static(const levo_hip_sample_args * args, const levo_hip_draw_args * draw,
                                           levo_hip_stream_t stream) {
    LEVO_REQUIRE(args != nullptr, "sample_step: null argument block");
    const int checked = check_sample_args(*args);
    if (checked != LEVO_HIP_OK || args->rows == 0) return checked;
    LEVO_REQUIRE(args->rows <= kStepMaxRows, "sample_step: more than %lld rows", static_cast<long long>(kStepMaxRows));
    const int64_t need = step_workspace_bytes(args->rows, args->vocab);
    LEVO_REQUIRE(need <= kStaticScratchBytes,
                 "sample_step_static: %lld rows of %lld logits need %lld bytes of scratch; the library holds %lld "
                 "per GPU (use levo_hip_sample_step with a workspace)",
                 static_cast<long long>(args->rows), static_cast<long long>(args->vocab),
                 static_cast<long long>(need), static_cast<long long>(kStaticScratchBytes));
    void * ws = nullptr;
    const int st = scratch_address(&ws);
    if (st != LEVO_HIP_OK) return st;
    return launch_step(args, draw, ws, kStaticScratchBytes, as_hip(stream));
}
