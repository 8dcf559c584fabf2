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
__device__ int64_t kNoListEntry = -1;  // read only; global, so that the pointer choice stays a global load

__device__ __forceinline__ int64_t list_entry(const int64_t * rec, int n_pen, const int64_t * ign, int n_ign,
                                              int i) {
    const int64_t * p = i < n_pen ? rec + i : i < n_pen + n_ign ? ign + (i - n_pen) : &kNoListEntry;
    return *p;
}

__device__ __forceinline__ float float_of_key(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// k-th largest (1 <= k <= 64) of the 64 lane keys of this wave; 0 when fewer
// than k lanes hold a non-zero key. A bisection from the top bit, unrolled
// without branches: each step is one compare, one ballot popcount and one
// scalar select, so the 32 steps cost less than the dependent reductions a
// narrower starting range would need.
__device__ __forceinline__ uint32_t wave_kth_key(uint32_t key, int k) {
    if (static_cast<int>(__popcll(__ballot(key != 0u))) < k) return 0u;
    uint32_t prefix = 0u;
#pragma unroll
    for (int bit = 31; bit >= 0; --bit) {
        const uint32_t cand = prefix | (1u << bit);
        prefix = static_cast<int>(__popcll(__ballot(key >= cand))) >= k ? cand : prefix;
    }
    return prefix;
}

// The same over NS keys per lane (invalid keys 0): the largest t with at least
// k keys >= t, or 0 when fewer than k keys are non-zero. Every valid key lies
// in [lo, hi]: the bits above their highest differing bit are lo's, and the
// bisection starts below them.
template <int NS>
__device__ __forceinline__ uint32_t wave_kth_key_slots(const uint32_t (&key)[NS], int k, uint32_t lo, uint32_t hi) {
    int nz = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) nz += static_cast<int>(__popcll(__ballot(key[s] != 0u)));
    if (nz < k) return 0u;
    const uint32_t diff = lo ^ hi;
    const int top = diff == 0u ? -1 : 31 - __builtin_clz(diff);
    uint32_t prefix = top < 0 ? lo : lo & ~((2u << top) - 1u);
#pragma unroll
    for (int bit = 31; bit >= 0; --bit) {
        if (bit > top) continue;  // uniform
        const uint32_t cand = prefix | (1u << bit);
        uint64_t m[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) m[s] = __ballot(key[s] >= cand);
        int c = 0;
#pragma unroll
        for (int s = 0; s < NS; ++s) c += static_cast<int>(__popcll(m[s]));
        prefix = c >= k ? cand : prefix;
        // the NS compares back to back, each into its own register pair, then
        // the scalar counts: one compare-to-count latency per step, not NS
        __builtin_amdgcn_sched_group_barrier(0x2, NS, 0);
        __builtin_amdgcn_sched_group_barrier(0x4, 2 * NS + 2, 0);
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
// A decode step samples a handful of rows of ~16K logits. Through one
// workgroup per row, a row's 131 KB (cond and uncond) arrive at the miss
// concurrency of one CU, several microseconds, and every selection phase
// then runs at one wave's serial latency. Here the loads are spread over many
// CUs and the row's exact selection runs once:
//   1. part launch, one wave per 512 ids of a row: the list ids first (the
//      repetition penalty and the ignore list enter LDS bitmaps of the
//      part), then the logits, CFG; the part's NaN flag, maximum, first
//      maximum and softmax sum; and a bound, the G-th largest of the 64 lane
//      maxima, so that at least G ids lie at or above it. Every id at or
//      above the bound is handed to the workspace (value and id, ascending
//      ids) with the part's head.
//   2. join launch, one workgroup per row, whose first wave reads every
//      part's head and handed-over ids in one round trip. Let L be the
//      largest part bound. The row's k-th largest value (the stable sort's
//      threshold, :84-89) is found among the handed-over ids at or above L,
//      the survivors, whenever there are at least k of them: if t is the k-th
//      largest survivor, t >= L, and a row id at or above t is at or above
//      its own part's bound, so it was handed over and survived; the row then
//      holds exactly the survivors' ids at or above t, and t is the row's
//      k-th largest. A bisection over the survivors' keys gives t; the
//      candidates at or above it are written in ascending id order, followed
//      by the draw of levo_hip_sample_draw when the rows are few.
// G = min(k, 64, ceil(2.5 k * 512 / V) + 6): two and a half times the
// candidates a part holds on average, plus six. With G >= k every part hands
// over at least its own top k and the survivors always suffice; LeVo's k = 50
// over 16384-16385 ids takes G = 10: in 20000 simulated Gaussian rows no row
// fell short and none had more than 251 survivors (G = 9: 0.05% short; G = 11:
// 0.22% above 256).
// A row with fewer than k survivors or more than the joining wave holds (512), a
// part with more than kPartCap ids at or above its bound (heavy ties), or
// k = 0 takes select_general over the whole row in the join launch.
constexpr int kPartIds = 512;                          // ids per part (one wave)
constexpr int kPartPer = kPartIds / 64;                // ids per lane
constexpr int kPartCap = 32;                           // handed-over ids per part
constexpr int kMaxParts = kMaxVocab / kPartIds;        // parts of the longest row
constexpr int kJoinCap = 512;                          // survivors the joining wave selects from
constexpr int kJoinFirst = 16;                         // slots per part the join reads before the heads arrive
constexpr int kJoinDrawRows = 8;                       // rows whose draws the join launch makes
constexpr int kEarlyChunks = (kJoinDrawRows - 1) * kMaxParts / 64;  // earlier rows' heads, 64 per chunk
constexpr int kStepWords = kMaxVocab / 32;             // bitmap words of the longest row
constexpr int64_t kStepMaxRows = 4095;
constexpr int32_t kPartOverflow = -1;
constexpr int32_t kPartNaN = -2;

struct alignas(16) part_head {
    float max;       // value at the part's first maximum (NaN skipped)
    int32_t best;    // the part's first id holding its maximum
    uint32_t bound;  // key of the part's bound (0: every id of the part handed over)
    int32_t count;   // ids handed over, or kPartOverflow / kPartNaN
};

struct alignas(8) part_cand {
    float v;
    int32_t id;
};

// The workspace: every (row, part) head, then the softmax sums, then the
// handed-over ids, kPartCap slots per part.
struct step_ws {
    part_head * heads;
    float * sums;
    part_cand * cands;
};

int64_t step_parts(int64_t vocab) { return (vocab + kPartIds - 1) / kPartIds; }

int64_t step_workspace_bytes(int64_t rows, int64_t vocab) {
    const int64_t n = rows * step_parts(vocab);
    return n * static_cast<int64_t>(sizeof(part_head)) + (n * 4 + 15) / 16 * 16 +
           n * kPartCap * static_cast<int64_t>(sizeof(part_cand));
}

step_ws carve_step_ws(void * ws, int64_t rows, int64_t vocab) {
    const int64_t n = rows * step_parts(vocab);
    uint8_t * p = static_cast<uint8_t *>(ws);
    step_ws w;
    w.heads = reinterpret_cast<part_head *>(p);
    p += n * static_cast<int64_t>(sizeof(part_head));
    w.sums = reinterpret_cast<float *>(p);
    p += (n * 4 + 15) / 16 * 16;
    w.cands = reinterpret_cast<part_cand *>(p);
    return w;
}

// Lane maxima at or above a part's bound (see above).
__device__ __forceinline__ int part_groups(int k, int V) {
    const int g = (5 * k * kPartIds + 2 * V - 1) / (2 * V) + 6;
    const int m = g < k ? g : k;
    return m < 64 ? m : 64;
}

// Id of item q of a lane in the part starting at lo, ascending in (q, lane)
// for VEC 1 (64 consecutive ids per item) and in (q / 4, lane, q % 4) for
// VEC 4 (two chunks of 256, four consecutive ids per lane).
template <int VEC>
__device__ __forceinline__ int part_item_id(int lo, int lane, int q) {
    return VEC == 4 ? lo + (q >> 2) * 256 + lane * 4 + (q & 3) : lo + q * 64 + lane;
}

template <int VEC>
__global__ __launch_bounds__(64) void step_part_kernel(const levo_hip_sample_args a, const step_ws w, int parts) {
    __shared__ uint32_t pen_map[kPartIds / 32];
    __shared__ uint32_t ign_map[kPartIds / 32];
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x / static_cast<uint32_t>(parts);
    const int part = static_cast<int>(blockIdx.x % static_cast<uint32_t>(parts));
    const int V = static_cast<int>(a.vocab);
    const int lo = part * kPartIds;
    const int hi = lo + kPartIds < V ? lo + kPartIds : V;
    const int stream = static_cast<int>(row % a.n_streams);
    int k = a.top_k[stream];
    if (k <= 0 || k >= V) k = 0;  // keep every id: the general path
    const int64_t rp = row * parts + part;

    // ---- the list entries first (see list_entry), then the part's logits ----------------
    const bool use_pen = a.recent != nullptr && a.n_recent > 0;
    const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
    const int n_pen = use_pen ? a.n_recent : 0;
    const int n_ign = use_ign ? a.n_ignore : 0;
    const int64_t * rec = use_pen ? a.recent + row * a.n_recent : &kNoListEntry;
    const int64_t * ign = use_ign ? a.ignore : &kNoListEntry;
    const int64_t entry = list_entry(rec, n_pen, ign, n_ign, lane);
    __builtin_amdgcn_sched_barrier(0);  // the entry's load is issued before the logits'
    // Without CFG the second input is the first again: every load is issued
    // unconditionally, so none waits for another (a per-item choice of source
    // would make each pair of loads a round trip of its own).
    const bool cfg = a.uncond != nullptr;
    const float * crow = a.cond + row * a.row_pitch;
    const float * urow = cfg ? a.uncond + row * a.row_pitch : crow;
    float c[kPartPer], u[kPartPer];
    if constexpr (VEC == 4) {
#pragma unroll
        for (int ch = 0; ch < kPartPer / 4; ++ch) {
            const int base = part_item_id<VEC>(lo, lane, ch * 4);
            const int off = base < V ? base : lo;  // row_pitch % 4 == 0: in bounds
            const f32x4 cv = *reinterpret_cast<const f32x4 *>(crow + off);
            const f32x4 uv = *reinterpret_cast<const f32x4 *>(urow + off);
            c[ch * 4] = cv.x; c[ch * 4 + 1] = cv.y; c[ch * 4 + 2] = cv.z; c[ch * 4 + 3] = cv.w;
            u[ch * 4] = uv.x; u[ch * 4 + 1] = uv.y; u[ch * 4 + 2] = uv.z; u[ch * 4 + 3] = uv.w;
        }
    } else {
#pragma unroll
        for (int q = 0; q < kPartPer; ++q) {
            const int id = part_item_id<VEC>(lo, lane, q);
            const int off = id < V ? id : lo;
            c[q] = crow[off];
            u[q] = urow[off];
        }
    }

    // Penalty and ignore ids inside this part, as bitmaps of its 512 ids.
    int pen = 0, ign_bits = 0;  // item bits
    if (use_pen || use_ign) {
        if (lane < kPartIds / 32) {
            pen_map[lane] = 0u;
            ign_map[lane] = 0u;
        }
        wave_lds_order();
        const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
        const int64_t top = hi < limit ? hi : limit;
        // the first 64 entries outside any loop: only their own load is waited
        // for, and the bitmaps fill while the logits are still in flight
        const auto mark = [&](int i, int64_t t) {
            if (i < n_pen) {
                if (t >= lo && t < top) atomicOr(&pen_map[(t - lo) >> 5], 1u << ((t - lo) & 31));
            } else if (i < n_pen + n_ign) {
                if (t >= lo && t < hi) atomicOr(&ign_map[(t - lo) >> 5], 1u << ((t - lo) & 31));
            }
        };
        mark(lane, entry);
        for (int i = lane + 64; i < n_pen + n_ign; i += 64) mark(i, list_entry(rec, n_pen, ign, n_ign, i));
        wave_lds_order();
#pragma unroll
        for (int q = 0; q < kPartPer; ++q) {
            const int rel = part_item_id<VEC>(lo, lane, q) - lo;
            pen |= (pen_map[rel >> 5] >> (rel & 31)) & 1u ? 1 << q : 0;
            ign_bits |= (ign_map[rel >> 5] >> (rel & 31)) & 1u ? 1 << q : 0;
        }
    }
    float v[kPartPer];
    bool has_nan = false;
    float tmax = -INFINITY;
#pragma unroll
    for (int q = 0; q < kPartPer; ++q) {
        float x = cfg ? u[q] + a.cfg_scale * (c[q] - u[q]) : c[q];
        if (pen & (1 << q)) x = x / a.repetition_penalty;
        if (ign_bits & (1 << q)) x = -INFINITY;
        v[q] = part_item_id<VEC>(lo, lane, q) < hi ? x : -INFINITY;
        has_nan = has_nan || __builtin_isnan(v[q]);
        tmax = fmaxf(tmax, v[q]);
    }

    // ---- maximum, first maximum, bound --------------------------------------------------
    // One all-reduce of (key << 32 | ~id): the largest value and, among its
    // ties (+-0 alike), the smallest id, the first maximum of std::max_element
    // (:94-96); the value itself comes from the lane that holds it.
    const bool part_nan = __ballot(has_nan) != 0;
    uint64_t lk = 0u;
    float fv = -INFINITY;
#pragma unroll
    for (int q = 0; q < kPartPer; ++q) {
        const int id = part_item_id<VEC>(lo, lane, q);
        const uint64_t c = (static_cast<uint64_t>(float_key(v[q])) << 32) | static_cast<uint32_t>(~id);
        if (id < hi && c > lk) {
            lk = c;
            fv = v[q];
        }
    }
    const uint64_t top = dpp::allreduce(lk, [](uint64_t x, uint64_t y) { return x > y ? x : y; });
    const int best = static_cast<int>(~static_cast<uint32_t>(top));
    const int owner = VEC == 4 ? ((best - lo) & 255) >> 2 : (best - lo) & 63;
    const float bv = dpp::lane(fv, owner);
    const float m = bv;  // the part's maximum (when it holds no NaN)
    uint32_t bkey = 0u;
    if (k == 1) {
        bkey = float_key(m);  // the ties of the maximum
    } else if (k > 1 && !part_nan) {
        const bool lane_valid = part_item_id<VEC>(lo, lane, 0) < hi;
        bkey = wave_kth_key(lane_valid ? float_key(tmax) : 0u, part_groups(k, V));
    }

    // ---- hand over every id at or above the bound, ascending ---------------------------
    int32_t count;
    if (part_nan) {
        count = kPartNaN;
    } else if (k == 0) {
        count = kPartOverflow;
    } else {
        bool take[kPartPer];
        int pos[kPartPer];
        int total = 0;
#pragma unroll
        for (int q = 0; q < kPartPer; ++q) take[q] = part_item_id<VEC>(lo, lane, q) < hi && float_key(v[q]) >= bkey;
        if constexpr (VEC == 4) {
#pragma unroll
            for (int ch = 0; ch < kPartPer / 4; ++ch) {
                // (lane, e) order: the takes of lower lanes, then this lane's lower e
                int below = 0, in_chunk = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint64_t mask = __ballot(take[ch * 4 + e]);
                    below += rank_in_mask(mask);
                    in_chunk += static_cast<int>(__popcll(mask));
                }
                int run = total + below;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    pos[ch * 4 + e] = run;
                    run += take[ch * 4 + e] ? 1 : 0;
                }
                total += in_chunk;
            }
        } else {
#pragma unroll
            for (int q = 0; q < kPartPer; ++q) {
                const uint64_t mask = __ballot(take[q]);
                pos[q] = total + rank_in_mask(mask);
                total += static_cast<int>(__popcll(mask));
            }
        }
        count = total <= kPartCap ? total : kPartOverflow;
        if (total <= kPartCap) {
            part_cand * out = w.cands + rp * kPartCap;
#pragma unroll
            for (int q = 0; q < kPartPer; ++q)
                if (take[q]) out[pos[q]] = part_cand{v[q], part_item_id<VEC>(lo, lane, q)};
        }
    }
    float sum = 0.0f;
    if (a.row_lse && !part_nan) {
        const float inv_t = 1.0f / a.temperature;
        const float mm = fmaxf(m, -FLT_MAX);
#pragma unroll
        for (int q = 0; q < kPartPer; ++q) sum += __expf((v[q] - mm) * inv_t);  // -inf and padding add 0
        sum = wave_sum_f32(sum);
    }
    if (lane == 0) {
        w.heads[rp] = part_head{bv, best, bkey, count};
        if (a.row_lse) w.sums[rp] = sum;
    }
}

// Slots [0, SPP) of every part into NS slots per lane: slot s of lane l is
// slot (l + 64 s) % SPP of part (l + 64 s) / SPP, ascending ids within a part
// and across parts. Every load is issued before any is used.
template <int SPP, int NS>
__device__ __forceinline__ void load_slots(part_cand (&sl)[NS], const part_cand * cand, int parts, int lane) {
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int j = lane + 64 * s;
        const int g = j / SPP < parts ? j / SPP : parts - 1;
        sl[s] = cand[g * kPartCap + j % SPP];
    }
}

// The handed-over ids at or above lo_v, in ascending id order, into
// sv / si[0, kJoinCap); returns their number (which may exceed kJoinCap).
// count: this lane's part count (lane g holds part g's).
template <int SPP, int NS>
__device__ __forceinline__ int collect_survivors(const part_cand (&sl)[NS], int count, int parts, float lo_v, float * sv,
                                                 int32_t * si, int lane) {
    // each slot's part count, fetched for every slot row at once (lane shuffles
    // issued back to back); parts past the row's last count 0
    int cnt[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const int g = (lane + 64 * s) / SPP;
        cnt[s] = __shfl(count, g < 64 ? g : 0);
        cnt[s] = g < parts ? cnt[s] : 0;
    }
    int n = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        const bool surv = (lane + 64 * s) % SPP < cnt[s] && sl[s].v >= lo_v;
        const uint64_t mask = __ballot(surv);
        const int p = n + rank_in_mask(mask);
        if (surv && p < kJoinCap) {
            sv[p] = sl[s].v;
            si[p] = sl[s].id;
        }
        n += static_cast<int>(__popcll(mask));
    }
    return n;
}

// The exact k-th value of the nsurv survivors (sv / si, ascending ids; KT per
// lane) and the candidates at or above it: their ids, logits and
// probabilities written to the row's outputs, and to cv / ci in ascending id
// order for the draw. Returns the candidate count.
template <int KT>
__device__ __forceinline__ int join_select(const levo_hip_sample_args & a, const float * sv, const int32_t * si,
                                           float * cv, int32_t * ci, int nsurv, int k, uint32_t lo_key,
                                           uint32_t hi_key, int64_t row, float rm, int best, int lane) {
    uint32_t keys[KT];
    bool valid[KT];
    float cval[KT];
    int32_t cid[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        const int idx = lane + 64 * t;
        valid[t] = idx < nsurv;
        const int at = valid[t] ? idx : 0;
        cval[t] = sv[at];
        cid[t] = si[at];
        keys[t] = valid[t] ? float_key(cval[t]) : 0u;
    }
    const uint32_t tau = k > 1 ? wave_kth_key_slots<KT>(keys, k, lo_key, hi_key) : hi_key;
    const bool want_probs = a.cand_probs != nullptr;
    const float inv_t = want_probs ? 1.0f / a.temperature : 0.0f;
    bool take[KT];
    int pos[KT];
    float wgt[KT];
    double z = 0.0;
    int n = 0;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        take[t] = valid[t] && keys[t] >= tau;
        const uint64_t mask = __ballot(take[t]);
        pos[t] = n + rank_in_mask(mask);
        n += static_cast<int>(__popcll(mask));
        wgt[t] = want_probs && take[t] ? cand_weight(cval[t], rm, inv_t) : 0.0f;
        z += static_cast<double>(wgt[t]);
        if (take[t]) {
            cv[pos[t]] = cval[t];
            ci[pos[t]] = cid[t];
        }
    }
    if (want_probs) z = wave_sum_f64(z);
    const bool z_ok = z > 0.0 && __builtin_isfinite(z);
    const float inv_z = z_ok ? static_cast<float>(1.0 / z) : 0.0f;
#pragma unroll
    for (int t = 0; t < KT; ++t) {
        if (take[t] && pos[t] < a.capacity) {
            const int64_t o = row * a.capacity + pos[t];
            a.cand_ids[o] = cid[t];
            if (a.cand_logits) a.cand_logits[o] = cval[t];
            if (want_probs) a.cand_probs[o] = z_ok ? wgt[t] * inv_z : (cid[t] == best ? 1.0f : 0.0f);
        }
    }
    return n;
}

struct join_lds {
    row_lds<kStepWords> L;                                   // the general path
    float sv[kJoinCap];                                      // survivors, ascending ids: values
    int32_t si[kJoinCap];                                    // and ids
    float cv[kJoinCap];                                      // the row's candidates, ascending ids
    int32_t ci[kJoinCap];
    int slow;
    float rm;
    int best;
    float bv;
    float lse;
};

// Bits [lo, hi) of a 64-lane mask, the bounds clamped to [0, 64].
__device__ __forceinline__ uint64_t lane_range(int lo, int hi) {
    lo = lo < 0 ? 0 : lo > 64 ? 64 : lo;
    hi = hi < 0 ? 0 : hi > 64 ? 64 : hi;
    const uint64_t below_hi = hi == 64 ? ~uint64_t{0} : (uint64_t{1} << hi) - 1u;
    const uint64_t below_lo = lo == 64 ? ~uint64_t{0} : (uint64_t{1} << lo) - 1u;
    return below_hi & ~below_lo;
}

// NS: handed-over slots per lane of the joining wave, ceil(parts / 2); every
// slot load is issued before the first is used.
template <int NS>
__global__ __launch_bounds__(kThreads) void step_join_kernel(const levo_hip_sample_args a, const levo_hip_draw_args d,
                                                              const step_ws w, int parts) {
    __shared__ join_lds S;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const int V = static_cast<int>(a.vocab);
    const int stream = static_cast<int>(row % a.n_streams);
    int k = a.top_k[stream];
    if (k <= 0 || k >= V) k = 0;
    const bool drawing = d.tokens != nullptr;
    const bool sampling = drawing && d.use_sampling != 0 && d.temperature != 0.0f;
    int before = 0;            // draws taken by the rows before this one (wave 0)
    uint64_t raw_at_r = 0;     // the raw value at the row index (wave 0)

    if (wave == 0) {
        // ---- every load first: the heads, the handed-over ids, the draw inputs ------------
        const int64_t rp0 = row * parts;
        const bool mine = lane < parts;
        const part_head h = w.heads[rp0 + (mine ? lane : 0)];
        const float hsum = a.row_lse != nullptr ? w.sums[rp0 + (mine ? lane : 0)] : 0.0f;
        // the first kJoinFirst slots of every part (most parts hand over fewer)
        const part_cand * cand = w.cands + rp0 * kPartCap;
        constexpr int NF = (NS + 1) / 2;
        part_cand sl[NF];
        load_slots<kJoinFirst, NF>(sl, cand, parts, lane);
        if (sampling) raw_at_r = d.bits[row];
        // the heads of the earlier rows (at most kJoinDrawRows - 1 of them)
        const int nearly = sampling ? static_cast<int>(row) * parts : 0;
        part_head eh[kEarlyChunks];
#pragma unroll
        for (int i = 0; i < kEarlyChunks; ++i) {
            const int f = lane + 64 * i;
            eh[i] = w.heads[f < nearly ? f : 0];
        }

        // ---- the row's maximum, first maximum, NaN flag and log-sum-exp ---------------------
        const bool row_nan = __ballot(mine && h.count == kPartNaN) != 0;
        const bool overflow = __ballot(mine && h.count == kPartOverflow) != 0;
        const float rm = wave_max_f32(mine ? h.max : -INFINITY);
        // the first maximum lies in the first part whose maximum is the row's
        const uint64_t at_max = __ballot(mine && h.max == rm);
        const int bpart = at_max != 0 ? __builtin_ctzll(at_max) : 0;
        const int best = row_nan ? -1 : dpp::lane(h.best, bpart);
        const float bv = dpp::lane(h.max, bpart);
        float lse = NAN;
        if (!row_nan && a.row_lse) {
            if (rm == -INFINITY) {
                lse = -INFINITY;
            } else if (rm == INFINITY) {
                lse = INFINITY;
            } else {
                const float inv_t = 1.0f / a.temperature;
                const float term = mine ? hsum * __expf((fmaxf(h.max, -FLT_MAX) - rm) * inv_t) : 0.0f;
                lse = rm / a.temperature + logf(wave_sum_f32(term));
            }
        }

        // ---- survivors: handed-over ids at or above the largest part bound ------------------
        const uint32_t hi_key = float_key(rm);
        const uint32_t lo_key =
            k == 1 ? hi_key : dpp::allreduce(mine ? h.bound : 0u, [](uint32_t x, uint32_t y) { return x > y ? x : y; });
        bool fast = !row_nan && !overflow && k >= 1;
        int nsurv = 0;
        if (fast) {
            // lo_key as a value (every lo_key is some value's key; 0 admits every
            // handed-over id): a value is at or above it exactly when its key is
            const float lo_v = lo_key == 0u ? -INFINITY : float_of_key(lo_key);
            if (__ballot(mine && h.count > kJoinFirst) == 0) {
                nsurv = collect_survivors<kJoinFirst, NF>(sl, h.count, parts, lo_v, S.sv, S.si, lane);
            } else {  // a part handed over more: read every slot of every part again
                part_cand all[NS];
                load_slots<kPartCap, NS>(all, cand, parts, lane);
                nsurv = collect_survivors<kPartCap, NS>(all, h.count, parts, lo_v, S.sv, S.si, lane);
            }
            fast = nsurv >= k && nsurv <= kJoinCap;
        }

        // ---- the exact k-th value and the candidates at or above it, ascending ids ----------
        int n = 0;
        if (fast) {
            wave_lds_order();
            // 4 survivors per lane, or 8 for the rare rows with more than 256
            n = nsurv <= kJoinCap / 2
                    ? join_select<kJoinCap / 128>(a, S.sv, S.si, S.cv, S.ci, nsurv, k, lo_key, hi_key, row, rm, best, lane)
                    : join_select<kJoinCap / 64>(a, S.sv, S.si, S.cv, S.ci, nsurv, k, lo_key, hi_key, row, rm, best, lane);
            if (lane == 0) {
                a.best[row] = best;
                a.count[row] = n;
                if (a.row_max) a.row_max[row] = bv;
                if (a.row_lse) a.row_lse[row] = lse;
            }
        } else if (row_nan && lane == 0) {  // the reference throws "logits contain NaN"
            a.best[row] = -1;
            a.count[row] = -1;
            if (a.row_max) a.row_max[row] = NAN;
            if (a.row_lse) a.row_lse[row] = NAN;
        }

        // ---- the draw index: earlier rows draw unless they hold a NaN or a +-inf maximum ----
        if (sampling && row > 0) {
            uint64_t kill[kEarlyChunks], live[kEarlyChunks];
#pragma unroll
            for (int i = 0; i < kEarlyChunks; ++i) {
                if (i * 64 >= nearly) break;  // uniform
                const bool in = lane + 64 * i < nearly;
                kill[i] = __ballot(in && (eh[i].count == kPartNaN || eh[i].max == INFINITY));
                live[i] = __ballot(in && eh[i].max > -INFINITY);
            }
            for (int r = 0; r < static_cast<int>(row); ++r) {
                bool killed = false, alive = false;
#pragma unroll
                for (int i = 0; i < kEarlyChunks; ++i) {
                    if (i * 64 >= nearly) break;  // uniform
                    const uint64_t range = lane_range(r * parts - 64 * i, (r + 1) * parts - 64 * i);
                    killed = killed || (kill[i] & range) != 0;
                    alive = alive || (live[i] & range) != 0;
                }
                before += !killed && alive ? 1 : 0;
            }
        }
        const bool slow = !row_nan && !fast;
        if (drawing && !slow) {
            wave_lds_order();
            const bool draws = sampling && !row_nan && __builtin_isfinite(bv);
            int64_t token;
            if (row_nan) token = LEVO_HIP_TOKEN_NAN;
            else if (!draws) token = best;
            else if (n > d.capacity) token = LEVO_HIP_TOKEN_OVERFLOW;
            else {
                const int first = lane < n ? lane : 0;
                const uint64_t raw = before == row ? raw_at_r : d.bits[before];
                token = draw_token(S.cv, S.ci, S.cv[first], S.ci[first], n, bv, d.temperature, raw);
            }
            if (lane == 0) {
                d.draws[row] = before + (draws ? 1 : 0);
                d.tokens[row] = token;
            }
        }
        if (lane == 0) {
            S.slow = slow ? 1 : 0;
            S.rm = rm;
            S.best = best;
            S.bv = bv;
            S.lse = lse;
        }
    }
    __syncthreads();
    if (!S.slow) return;  // uniform

    // ---- a row the fast path does not cover: the whole row again, by the whole workgroup ----
    const bool use_pen = a.recent != nullptr && a.n_recent > 0;
    const bool use_ign = a.ignore != nullptr && a.n_ignore > 0 && stream == 0;
    row_lds<kStepWords> & L = S.L;
    const int words = (V + 31) / 32;
    for (int i = tid; i < words; i += kThreads) {
        L.sel[i] = 0u;
        L.pen[i] = 0u;
        L.ign[i] = 0u;
    }
    __syncthreads();
    if (use_pen) {
        const int64_t limit = a.penalty_limit > 0 && a.penalty_limit < V ? a.penalty_limit : V;
        const int64_t * rec = a.recent + row * a.n_recent;
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
    select_general(a, L, row, V, k, S.rm, S.best, use_pen, use_ign);
    if (tid == 0) {
        a.best[row] = S.best;
        a.count[row] = L.total;
        if (a.row_max) a.row_max[row] = S.bv;
        if (a.row_lse) a.row_lse[row] = S.lse;
    }
    if (!drawing) return;
    __syncthreads();  // the row's candidates are written and visible to the workgroup
    if (wave != 0) return;
    const int n = L.total;
    const bool draws = sampling && __builtin_isfinite(S.bv);
    int64_t token;
    if (!draws) token = S.best;
    else if (n > d.capacity) token = LEVO_HIP_TOKEN_OVERFLOW;
    else {
        const float * vals = a.cand_logits + row * a.capacity;
        const int32_t * ids = a.cand_ids + row * a.capacity;
        const int first = lane < n ? lane : 0;
        const uint64_t raw = before == row ? raw_at_r : d.bits[before];
        token = draw_token(vals, ids, vals[first], ids[first], n, S.bv, d.temperature, raw);
    }
    if (lane == 0) {
        d.draws[row] = before + (draws ? 1 : 0);
        d.tokens[row] = token;
    }
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
    const int64_t parts = step_parts(a.vocab);
    LEVO_REQUIRE(a.rows <= kStepMaxRows, "sample_step: more than %lld rows", static_cast<long long>(kStepMaxRows));
    LEVO_REQUIRE(ws != nullptr && aligned16(ws), "sample_step: workspace must be 16-byte aligned device memory");
    LEVO_REQUIRE(ws_bytes >= step_workspace_bytes(a.rows, a.vocab),
                 "sample_step: workspace smaller than levo_hip_sample_step_workspace_bytes");
    const step_ws w = carve_step_ws(ws, a.rows, a.vocab);
    const uint32_t grid = static_cast<uint32_t>(a.rows * parts);
    const bool vec = a.row_pitch % 4 == 0 && aligned16(a.cond) && (a.uncond == nullptr || aligned16(a.uncond));
    if (vec) step_part_kernel<4><<<grid, 64, 0, stream>>>(a, w, static_cast<int>(parts));
    else step_part_kernel<1><<<grid, 64, 0, stream>>>(a, w, static_cast<int>(parts));
    const int sa = launch_status("levo_hip_sample_step");
    if (sa != LEVO_HIP_OK) return sa;
    // the join launch draws when the rows are few; otherwise the draw is a
    // launch of its own
    const bool join_draws = a.rows <= kJoinDrawRows;
    levo_hip_draw_args dm = d;
    if (!join_draws) dm.tokens = nullptr;
    const uint32_t jg = static_cast<uint32_t>(a.rows);
    const int np = static_cast<int>(parts);
    if (parts <= 8) step_join_kernel<4><<<jg, kThreads, 0, stream>>>(a, dm, w, np);
    else if (parts <= 16) step_join_kernel<8><<<jg, kThreads, 0, stream>>>(a, dm, w, np);
    else if (parts <= 34) step_join_kernel<17><<<jg, kThreads, 0, stream>>>(a, dm, w, np);
    else step_join_kernel<32><<<jg, kThreads, 0, stream>>>(a, dm, w, np);
    const int sb = launch_status("levo_hip_sample_step");
    if (sb != LEVO_HIP_OK || draw == nullptr || join_draws) return sb;
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
