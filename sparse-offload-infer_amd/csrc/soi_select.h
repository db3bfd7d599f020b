// Threshold top-k building blocks shared by the top-k kernels and the fused
// DIP select + down-projection kernel (gfx950, wave64).
//
// Rule A of the reference's topk_threshold_select
// (csrc/kernels/topk_select.cu:19-95) depends on the values only through
// v_(k), the k-th largest value: count(v >= mid) >= k exactly when
// v_(k) >= mid. A workgroup finds v_(k) by a radix select on
// order-preserving keys (radix_pass), replays the 24 fp32 bisection steps on
// it (rule_a_tau) and compacts the elements with v >= tau in ascending index
// order (rule_a_compact).
#pragma once

#include "soi_device.h"

namespace soi {

constexpr int kBisectionSteps = 24;

__device__ __forceinline__ uint32_t popc64(uint64_t m) { return static_cast<uint32_t>(__builtin_popcountll(m)); }

// Inclusive prefix sum over the 64 lanes (DPP, fixed order).
__device__ __forceinline__ uint32_t wave_prefix_u32(uint32_t x) {
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x111, 0xf, 0xf, false));  // row_shr:1
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x112, 0xf, 0xf, false));  // row_shr:2
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x114, 0xf, 0xf, false));  // row_shr:4
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x118, 0xf, 0xf, false));  // row_shr:8
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x142, 0xa, 0xf, false));  // row_bcast:15
    x += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x143, 0xc, 0xf, false));  // row_bcast:31
    return x;
}

// Value sources: fp32 values as given, or |x| of binary16 values (the fp32
// conversion and the absolute value are exact, so selecting over F16Abs(g)
// equals selecting over g.float().abs()).
// Each source also defines an order-preserving radix key (0 = NaN / padding,
// never counted), the value of a key, and the digits of the radix passes.
struct F32Values {
    // Every bisection midpoint is > 0 (lo >= 0, hi >= 1e-3 / 2^24), so all values <= 0 compare alike: they share
    // key 1, a positive value v has key bits(v) + 1 (<= 0x7f800001), NaN 0. 31-bit keys, digits of 11, 10, 10
    // bits (8 bins per octave in the first pass).
    static constexpr int kPasses = 3;
    const float* p;
    __device__ __forceinline__ float operator[](int i) const { return ldg(p + i); }
    __device__ __forceinline__ float load(int i) const { return ldg(p + i); }
    __device__ __forceinline__ static uint32_t key_of(float v) {
        const uint32_t kp = __builtin_bit_cast(uint32_t, v) + 1u;
        const uint32_t k1 = v > 0.0f ? kp : 1u;
        return v == v ? k1 : 0u;
    }
    __device__ __forceinline__ static float value_of(uint32_t key) {
        return key >= 2u ? __builtin_bit_cast(float, key - 1u) : 0.0f;
    }
    __host__ __device__ static constexpr int shift(int pass) { return pass == 0 ? 20 : (pass == 1 ? 10 : 0); }
    __host__ __device__ static constexpr int bits(int pass) { return pass == 0 ? 11 : 10; }
};
struct F16AbsValues {
    // |binary16| orders like its 15-bit pattern (exponent, mantissa): key = 0x8000 | pattern, NaN -> 0;
    // digits of 9 and 6 bits (16 bins per octave in the first pass). A 12-bit first digit (128 bins per octave,
    // fewer same-word LDS atomics) measured slower: its 64-bin-per-lane scan costs more than the conflicts save.
    static constexpr int kPasses = 2;
    const uint16_t* p;
    __device__ __forceinline__ float operator[](int i) const { return fabsf(f16_bits_to_f32(ldg(p + i))); }
    __device__ __forceinline__ float load(int i) const {
        return f16_bits_to_f32(static_cast<uint16_t>(ldg(p + i) & 0x7fffu));
    }
    __device__ __forceinline__ static uint32_t key_of(float v) {  // v = |h|: its binary16 pattern back, exactly
        const uint32_t m = __builtin_bit_cast(uint16_t, static_cast<f16>(v));
        return v == v ? (m | 0x8000u) : 0u;
    }
    __device__ __forceinline__ static float value_of(uint32_t key) {
        return f16_bits_to_f32(static_cast<uint16_t>(key & 0x7fffu));
    }
    __host__ __device__ static constexpr int shift(int pass) { return pass == 0 ? 6 : 0; }
    __host__ __device__ static constexpr int bits(int pass) { return pass == 0 ? 9 : 6; }
};

__device__ __forceinline__ int hist_slot(int bin) { return bin + (bin >> 5); }
__host__ __device__ constexpr int hist_words(int nb) { return nb + nb / 32; }

template <class Values>
__host__ __device__ constexpr int radix_hist_offset(int p) {
    int w = 0;
    for (int q = 0; q < p; ++q) w += hist_words(1 << Values::bits(q)) + kWave;  // + one dummy word per lane
    return w;
}

// One radix pass over digit (key >> SHIFT) & (2^BITS - 1) of the candidate keys
// (key & pmask == prefix): histogram, barrier, then every wave finds the digit
// holding the rank on its own. Lane l reads its B = 2^BITS / 64 contiguous bins
// (counted from the top) into registers; the lane prefix over lanes is then a
// suffix count over bins. Returns false if fewer than `rank` candidates exist
// (only possible in the first pass: fewer than k valid values).
template <int SHIFT, int BITS, int E>
__device__ __forceinline__ bool radix_pass(const uint32_t (&key)[E], uint32_t* hist, uint32_t& prefix, uint32_t& pmask,
                                           uint32_t& rank, int lane) {
    constexpr int NB = 1 << BITS;
    constexpr int B = NB / kWave;
    // branch-free: a non-candidate adds to its lane's private dummy word after the histogram instead
    // (a branch per element costs more than the extra conflict-free LDS add)
    const int dummy = hist_words(NB) + lane;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const uint32_t kk = key[j];
        const bool cand = kk != 0u && (kk & pmask) == prefix;
        atomicAdd(&hist[cand ? hist_slot(static_cast<int>((kk >> SHIFT) & (NB - 1))) : dummy], 1u);
    }
    __syncthreads();
    const int top = NB - B * lane - 1;
    uint32_t c[B];
#pragma unroll
    for (int b = 0; b < B; ++b) c[b] = hist[hist_slot(top - b)];
#pragma unroll
    for (int w = 1; w < B; w *= 2)  // pairwise tree: c[0] ends with the lane's total
#pragma unroll
        for (int b = 0; b + w < B; b += 2 * w) c[b] += c[b + w];
    const uint32_t t = c[0];
    const uint32_t incl = wave_prefix_u32(t);
    const uint32_t reach = popc64(ballot(incl >= rank));  // lanes [64 - reach, 63] reach the rank
    if (reach == 0u) return false;
    const int L = kWave - static_cast<int>(reach);
    // the bin inside lane L's range: lane b < B takes bin topL - b, a lane prefix over those gives the running
    // count from the top, and the first lane whose running count reaches the rank holds the digit
    const int topL = NB - B * L - 1;
    const uint32_t base = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl - t), L));
    const uint32_t cb_all = hist[hist_slot(topL - (lane < B ? lane : 0))];
    const uint32_t cb = lane < B ? cb_all : 0u;
    const uint32_t run = base + wave_prefix_u32(cb);
    const uint64_t hitm = ballot(lane < B && run >= rank);
    const int hb = static_cast<int>(__builtin_ctzll(hitm));
    const uint32_t d = static_cast<uint32_t>(topL - hb);
    const uint32_t above = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(run - cb), hb));
    prefix |= d << SHIFT;
    pmask |= static_cast<uint32_t>(NB - 1) << SHIFT;
    rank -= above;
    return true;
}

// Zero the histograms rule_a_tau uses (its ZEROED = true form expects this done before its call, e.g. while
// the keys' loads are in flight).
template <int NW, class Values>
__device__ __forceinline__ void rule_a_zero_hist(uint32_t* s_hist, int tid) {
    constexpr int kWords = radix_hist_offset<Values>(Values::kPasses);
    for (int i = tid; i < kWords; i += NW * kWave) s_hist[i] = 0u;
}

struct NoMid {
    __device__ __forceinline__ void operator()() const {}
};

// tau of rule A over the workgroup's keys: NW waves, E keys per lane (0 = NaN
// or padding), local_max = this lane's fmaxf over its values starting from
// 0.0f. Zeroes s_hist (radix_hist_offset<Values>(kPasses) words) itself
// unless ZEROED; with SYNCED the caller zeroed it and ran a barrier after, so
// the first radix pass's barrier also publishes s_max (no barrier of its own
// between the keys and the first pass); s_max holds NW floats. mid() runs in every thread after the
// first radix pass and before the second pass's barrier, which publishes its
// LDS stores (a barrier of its own replaces that pass when it does not run):
// work that does not feed the selection, done while its first pass waits.
// Returns tau = lo after the 24 steps, or, for binary16
// values, a threshold that selects exactly the same values (see below);
// `found` is false when fewer than k keys are nonzero (then every step goes
// left, as the reference's counts do).
template <int E, int NW, class Values, bool ZEROED = false, class Mid = NoMid, bool SYNCED = false>
__device__ __forceinline__ float rule_a_tau(const uint32_t (&key)[E], float local_max, uint32_t* s_hist, float* s_max,
                                            int k, int tid, const Mid& mid = Mid{}) {
    constexpr int NPASS = Values::kPasses;
    const int wave = tid >> 6, lane = tid & 63;
    if (!ZEROED && !SYNCED) rule_a_zero_hist<NW, Values>(s_hist, tid);
    const float wmax = wave_max_bcast(local_max);
    if (lane == 0) s_max[wave] = wmax;
    if (!SYNCED) __syncthreads();

    uint32_t prefix = 0u, pmask = 0u, rank = static_cast<uint32_t>(k);
    bool found = radix_pass<Values::shift(0), Values::bits(0)>(key, s_hist, prefix, pmask, rank, lane);
    mid();
    if (found)
        found = radix_pass<Values::shift(1), Values::bits(1)>(key, s_hist + radix_hist_offset<Values>(1), prefix,
                                                              pmask, rank, lane);
    else if (!__is_same(Mid, NoMid))
        __syncthreads();  // found is the same in every wave (all read one histogram)
    if (NPASS == 3 && found)
        found = radix_pass<Values::shift(NPASS == 3 ? 2 : 1), Values::bits(NPASS == 3 ? 2 : 1)>(
            key, s_hist + radix_hist_offset<Values>(NPASS == 3 ? 2 : 1), prefix, pmask, rank, lane);

    float total_max = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) total_max = fmaxf(total_max, s_max[w]);
    const float vk = Values::value_of(prefix | (NPASS == 2 ? 0x8000u : 0u));
    float lo = 0.0f;
    float hi = total_max + 1e-3f;
    if constexpr (NPASS == 2) {
        // binary16 values: the 24 steps below keep lo <= v_(k) <= hi, and each halves hi - lo and adds at most
        // hi0 * 2^-24 of rounding (mid = fl(0.5 * fl(lo + hi)), lo + hi <= 2 hi0), so at the end
        // v_(k) - lo <= 3 * hi0 * 2^-24. When v_(k) is a normal binary16 >= hi0 * 2^-11, every smaller binary16
        // lies at least v_(k) * 2^-11 > 3 * hi0 * 2^-24 below it, none lies in [lo, v_(k)), and "v >= tau" selects
        // exactly the values "v >= v_(k)" selects: v_(k) stands for tau without the replay.
        if (found && vk >= 0x1p-14f && vk >= hi * 0x1p-11f) return vk;
    }
    // 24 steps of mid = fl(0.5f * fl(lo + hi)), lo = mid if v_(k) >= mid else hi = mid. Both possible next
    // sums are formed while the comparison resolves (the same fp32 operations, fewer dependent steps).
    float sum = lo + hi;
#pragma unroll
    for (int it = 0; it < kBisectionSteps; ++it) {
        const float mid = 0.5f * sum;
        const bool right = found && vk >= mid;
        const float s_right = mid + hi, s_left = lo + mid;
        lo = right ? mid : lo;
        hi = right ? hi : mid;
        sum = right ? s_right : s_left;
    }
    return lo;
}

// Ordered compaction of the elements with val >= tau (element (j, lane) of
// wave w = w*64E + 64j + lane): its position is (selected elements of earlier
// waves) + (selected elements of earlier j of this wave) + (earlier lanes of
// this j), i.e. ascending index order. emit(pos, j) runs in every lane whose
// element is selected and whose position lies in [lo, hi); the return value
// is the total number selected. The first pass keeps each j's count (wave-
// uniform), so the second pass ballots again only for the j whose positions
// reach into the window: a workgroup that needs one chunk of the positions
// walks the rest with a few scalar instructions per j. s_tot holds NW words;
// one barrier.
template <int E, int NW, class Emit>
__device__ __forceinline__ uint32_t rule_a_compact(const float (&val)[E], float tau, uint32_t* s_tot, int tid,
                                                   uint32_t lo, uint32_t hi, Emit&& emit) {
    const int wave = tid >> 6, lane = tid & 63;
    uint32_t cnt[E];
    uint32_t wave_total = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        cnt[j] = popc64(ballot(val[j] >= tau));
        wave_total += cnt[j];
    }
    if (lane == 0) s_tot[wave] = wave_total;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const uint32_t c = s_tot[w];
        before += (w < wave) ? c : 0u;
        total += c;
    }
    uint32_t running = before;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        if (running < hi && running + cnt[j] > lo) {  // wave-uniform
            const bool sel = val[j] >= tau;
            const uint64_t mk = ballot(sel);
            const uint32_t pos = running + mask_prefix(mk);
            if (sel && pos >= lo && pos < hi) emit(pos, j);
        }
        running += cnt[j];
    }
    return total;
}

template <int E, int NW, class Emit>
__device__ __forceinline__ uint32_t rule_a_compact(const float (&val)[E], float tau, uint32_t* s_tot, int tid,
                                                   Emit&& emit) {
    return rule_a_compact<E, NW>(val, tau, s_tot, tid, 0u, 0xffffffffu, static_cast<Emit&&>(emit));
}

}  // namespace soi
