// Deterministic threshold top-k (Dynamic Input Pruning channel selection).
//
// Semantics are exactly the reference's topk_threshold_select
// (csrc/kernels/topk_select.cu:10-96):
//   total_max = max(0, max_i v_i);  lo = 0;  hi = fl(total_max + 1e-3f)
//   24 times: mid = fl(0.5f * fl(lo + hi));
//             if count(v_i >= mid) >= k  lo = mid  else  hi = mid
//   out = the first k indices, ascending, with v_i >= lo;  count = #written.
// Counts are integers, so the decisions (and hence tau = lo) do not depend on
// how the counting is parallelised.
//
// gfx950 design: ONE workgroup of 16 waves holds all values in registers.
// The 24 bisection steps are replayed 8 at a time from one LDS histogram of
// the values against the exact node values of the next 8 levels (three
// rounds, two barriers each, instead of one barrier round per step); see
// topk_rule_a_regs_kernel. The final compaction is an ordered ballot prefix
// scan: position = (elements of earlier waves) + (earlier rows of this wave)
// + (earlier lanes in this row), so the output is in ascending index order
// by construction and identical on every call.
#include "soi_device.h"
#include "soi_host.h"
#include "soi_select.h"

namespace soi {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;

// Block-wide fp32 max of per-thread values (initial value 0.0f, as the reference).
__device__ __forceinline__ float block_max_from(float local, float* s_max, int wave, int lane) {
    const float wm = wave_max_bcast(local);
    if (lane == 0) s_max[wave] = wm;
    __syncthreads();
    float m = 0.0f;
#pragma unroll
    for (int w = 0; w < kTopkWaves; ++w) m = fmaxf(m, s_max[w]);
    return m;
}

// Value of bisection node `i` (in-order index 1..255 of the next 8 levels)
// reached from state (lo, hi) by the reference recurrence: at each level
// mid = fl(0.5f * fl(lo + hi)), going right sets lo = mid, left sets hi = mid.
__device__ __forceinline__ float bisection_node(float lo, float hi, int i) {
    int c = 128, step = 64;
    float m = 0.0f;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
        m = 0.5f * (lo + hi);
        if (i == c) break;
        if (i > c) {
            lo = m;
            c += step;
        } else {
            hi = m;
            c -= step;
        }
        step >>= 1;
    }
    return m;
}


// E values per thread held in registers: n <= 1024*E. Wave w owns elements
// [w*64E, (w+1)*64E), element (j, lane) = w*64E + 64j + lane, so each load is
// 64 contiguous floats and the ascending-index order is (wave, j, lane).
//
// The 24 bisection steps are replayed 8 at a time. For the current (lo, hi)
// the 255 node values T_1 <= ... <= T_255 of the next 8 levels are computed
// with the reference's fp32 recurrence (thread t computes T_{t+1}). With
// pos(v) = #{i : T_i <= v}, count(v >= T_c) = S(c) = #{pos >= c} + #{v >= hi},
// non-increasing in c, so the 8 sequential decisions "S(mid) >= k" of a
// binary search over the nodes end exactly at c* = #{c : S(c) >= k}: the
// new state is lo = T_{c*} (unchanged if c* = 0), hi = T_{c*+1} (unchanged if
// c* = 255). One histogram of pos over the candidates lo <= v < hi gives all
// S(c); pos is estimated from the even node spacing and verified against the
// exact node values (an exact search runs only when the estimate is off).
// Node and histogram buffers are double-buffered by round: two barriers per
// round, three rounds.

template <int E, class Values>
__global__ __launch_bounds__(kTopkThreads) void topk_rule_a_regs_kernel(const Values v, int n, int k,
                                                                         int32_t* __restrict__ out_idx,
                                                                         int32_t* __restrict__ out_count) {
    __shared__ float s_max[kTopkWaves];
    __shared__ float s_T[2][256];     // s_T[b][i] = T_i, i in 1..255
    __shared__ uint32_t s_hist[2][256];  // pos histogram of candidates
    __shared__ uint32_t s_above[2];      // count of v >= hi
    __shared__ __attribute__((aligned(16))) uint32_t s_tot[kTopkWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int base_i = wave * kWave * E + lane;

    float val[E];
    float local_max = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {  // clamped index: every load is issued unconditionally, no branch per load
        const int i = base_i + j * kWave;
        const float x = v[i < n ? i : n - 1];
        val[j] = (i < n) ? x : -__builtin_inff();
        local_max = fmaxf(local_max, val[j]);
    }
    const float total_max = block_max_from(local_max, s_max, wave, lane);

    float lo = 0.0f;
    float hi = total_max + 1e-3f;
#pragma unroll 1
    for (int round = 0; round < 3; ++round) {
        const int b = round & 1;
        if (tid < 255) s_T[b][tid + 1] = bisection_node(lo, hi, tid + 1);
        if (tid < 256) s_hist[b][tid] = 0u;
        if (tid == 0) s_above[b] = 0u;
        __syncthreads();

        const float est = 256.0f / (hi - lo);
        uint32_t above = 0;
        int p[E];
        float ta[E], tb[E];
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float x = val[j];
            above += popc64(ballot(x >= hi));
            int q = static_cast<int>((x - lo) * est);
            q = q < 0 ? 0 : (q > 255 ? 255 : q);
            p[j] = q;
            ta[j] = s_T[b][q > 0 ? q : 1];
            tb[j] = s_T[b][q < 255 ? q + 1 : 255];
        }
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float x = val[j];
            if (x >= lo && x < hi) {
                int q = p[j];
                const bool ok = (q == 0 || x >= ta[j]) && (q == 255 || x < tb[j]);
                if (!ok) {  // exact search from the estimate (rare)
                    while (q < 255 && x >= s_T[b][q + 1]) ++q;
                    while (q > 0 && x < s_T[b][q]) --q;
                }
                atomicAdd(&s_hist[b][q], 1u);
            }
        }
        if (lane == 0 && above) atomicAdd(&s_above[b], above);
        __syncthreads();

        // lane l holds buckets c = 255-4l-jj (jj = 0..3): a lane prefix in that order is a suffix over c
        uint32_t a[4];
        uint32_t run = 0;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            run += s_hist[b][255 - 4 * lane - jj];
            a[jj] = run;
        }
        const uint32_t excl = wave_prefix_u32(run) - run + s_above[b];
        uint32_t cstar = 0;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const int c = 255 - 4 * lane - jj;
            cstar += popc64(ballot(c >= 1 && excl + a[jj] >= static_cast<uint32_t>(k)));
        }
        const float new_lo = cstar >= 1 ? s_T[b][cstar >= 1 ? cstar : 1] : lo;
        const float new_hi = cstar <= 254 ? s_T[b][cstar <= 254 ? cstar + 1 : 255] : hi;
        lo = new_lo;
        hi = new_hi;
    }
    const float tau = lo;

    uint64_t m[E];
    uint32_t cnt[E];
    uint32_t wave_total = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        m[j] = ballot(val[j] >= tau);
        cnt[j] = popc64(m[j]);
        wave_total += cnt[j];
    }
    if (lane == 0) s_tot[wave] = wave_total;
    __syncthreads();
    uint32_t before = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kTopkWaves; ++w) {
        const uint32_t c = s_tot[w];
        before += (w < wave) ? c : 0u;
        total += c;
    }
    uint32_t running = before;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const uint32_t pos = running + mask_prefix(m[j]);
        if (val[j] >= tau && pos < static_cast<uint32_t>(k)) out_idx[pos] = base_i + j * kWave;
        running += cnt[j];
    }
    if (tid == 0) *out_count = static_cast<int32_t>(total < static_cast<uint32_t>(k) ? total : k);
}

// Radix form (n <= 512*32): rule A depends on the values only through v_(k),
// the k-th largest value: count(v >= mid) >= k exactly when v_(k) >= mid. So
// the kernel finds v_(k) exactly by a radix select on order-preserving keys
// (NaN and padding map to key 0 and never count; see the value sources),
// replays the 24 bisection steps on it in fp32 (the reference's op
// sequence), and compacts.
//
// One workgroup of 8 waves, E values per lane in registers, element
// (j, lane) of wave w = w*64E + 64j + lane. Every pass: candidates (keys that
// match the digits found so far) add 1 to an LDS histogram of their next
// digit, one barrier, then EVERY wave scans the histogram itself (lane l
// reads the contiguous bins l*B..l*B+B-1 counted from the top, a DPP prefix
// over lanes finds the lane holding the rank, then B lanes re-read that
// lane's bins and a second prefix finds the bin), so the passes need no
// further barrier. Histograms are zeroed up front and padded by one word per
// 32 bins (conflict-free lane reads); a lane whose element is not a
// candidate adds to a private dummy word instead of branching. fp32 keys take
// digits of 11, 10 and 10 bits; a binary16 magnitude's key is its 15-bit
// pattern, two digits of 9 and 6 bits (16 bins per octave in the first pass,
// so gate magnitudes spread over many bins: few same-address LDS atomics).
// Four (binary16) or five (fp32) barriers in all, against nine for the
// bisection-histogram form. Every global load is issued unconditionally
// (clamped index): a branch per load serialises them.
constexpr int kRadixThreads = 512;
constexpr int kRadixWaves = kRadixThreads / kWave;

template <int E, class Values>
__global__ __launch_bounds__(kRadixThreads) void topk_radix_kernel(const Values v, int n, int k,
                                                                   int32_t* __restrict__ out_idx,
                                                                   int32_t* __restrict__ out_count) {
    __shared__ uint32_t s_hist[radix_hist_offset<Values>(Values::kPasses)];
    __shared__ float s_max[kRadixWaves];
    __shared__ uint32_t s_tot[kRadixWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int base_i = wave * kWave * E + lane;

    float val[E];
    uint32_t key[E];
    float local_max = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {  // clamped index: every load is issued unconditionally, no branch per load
        const int i = base_i + j * kWave;
        val[j] = v.load(i < n ? i : n - 1);
    }
    // the histograms are zeroed and published while the values are in flight (rule A's SYNCED form)
    rule_a_zero_hist<kRadixWaves, Values>(s_hist, tid);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = base_i + j * kWave;
        val[j] = (i < n) ? val[j] : __builtin_nanf("");
        key[j] = Values::key_of(val[j]);
        local_max = fmaxf(local_max, val[j]);
    }
    const float tau = rule_a_tau<E, kRadixWaves, Values, true, NoMid, true>(key, local_max, s_hist, s_max, k, tid);
    const uint32_t total = rule_a_compact<E, kRadixWaves>(val, tau, s_tot, tid, [&](uint32_t pos, int j) {
        if (pos < static_cast<uint32_t>(k)) out_idx[pos] = base_i + j * kWave;
    });
    if (tid == 0) *out_count = static_cast<int32_t>(total < static_cast<uint32_t>(k) ? total : k);
}

// Any n: values streamed from global memory (L2-resident after the first
// pass) in blocks of 1024, same arithmetic and same output order.
template <class Values>
__global__ __launch_bounds__(kTopkThreads) void topk_rule_a_stream_kernel(const Values v, int n, int k,
                                                                           int32_t* __restrict__ out_idx,
                                                                           int32_t* __restrict__ out_count) {
    __shared__ float s_max[kTopkWaves];
    __shared__ uint32_t s_cnt[2][kTopkWaves];
    __shared__ uint32_t s_blk[2][kTopkWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    float local_max = 0.0f;
    for (int i = tid; i < n; i += kTopkThreads) local_max = fmaxf(local_max, v[i]);
    const float total_max = block_max_from(local_max, s_max, wave, lane);

    float lo = 0.0f;
    float hi = total_max + 1e-3f;
    for (int it = 0; it < kBisectionSteps; ++it) {
        const float mid = 0.5f * (lo + hi);
        uint32_t cnt = 0;
        for (int b = 0; b < n; b += kTopkThreads) {
            const int i = b + tid;
            cnt += popc64(ballot(i < n && v[i] >= mid));
        }
        if (lane == 0) s_cnt[it & 1][wave] = cnt;
        __syncthreads();
        uint32_t total = 0;
        for (int w = 0; w < kTopkWaves; ++w) total += s_cnt[it & 1][w];
        if (total >= static_cast<uint32_t>(k))
            lo = mid;
        else
            hi = mid;
    }
    const float tau = lo;
    uint32_t running = 0;
    int parity = 0;
    for (int b = 0; b < n && running < static_cast<uint32_t>(k); b += kTopkThreads, parity ^= 1) {
        const int i = b + tid;
        const bool flag = i < n && v[i] >= tau;
        const uint64_t mk = ballot(flag);
        if (lane == 0) s_blk[parity][wave] = popc64(mk);
        __syncthreads();
        uint32_t before = 0, blk = 0;
        for (int w = 0; w < kTopkWaves; ++w) {
            const uint32_t c = s_blk[parity][w];
            before += (w < wave) ? c : 0u;
            blk += c;
        }
        const uint32_t pos = running + before + mask_prefix(mk);
        if (flag && pos < static_cast<uint32_t>(k)) out_idx[pos] = i;
        running += blk;
    }
    if (tid == 0) *out_count = static_cast<int32_t>(running < static_cast<uint32_t>(k) ? running : k);
}

template <class Values>
static int launch_topk(const Values v, int64_t n, int64_t k, int32_t* out_indices, int32_t* out_count, void* stream,
                       const char* what) {
    SOI_REQUIRE(n >= 1 && n <= (int64_t(1) << 30), "%s: n must be in [1, 2^30]", what);
    SOI_REQUIRE(k >= 1 && k <= n, "%s: k must be in [1, n]", what);
    SOI_REQUIRE(v.p && out_indices && out_count, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    const int ni = static_cast<int>(n), ki = static_cast<int>(k);
    const int64_t er = ceil_div64(n, kRadixThreads);
    if (er <= 32) {
#define SOI_R(EE) \
    hipLaunchKernelGGL((topk_radix_kernel<EE, Values>), dim3(1), dim3(kRadixThreads), 0, st, v, ni, ki, \
                       out_indices, out_count)
        if (er <= 1) SOI_R(1);
        else if (er <= 2) SOI_R(2);
        else if (er <= 4) SOI_R(4);
        else if (er <= 8) SOI_R(8);
        else if (er <= 12) SOI_R(12);
        else if (er <= 16) SOI_R(16);
        else if (er <= 24) SOI_R(24);
        else SOI_R(32);
#undef SOI_R
        return launch_status(what);
    }
    const int64_t e = ceil_div64(n, kTopkThreads);
#define SOI_T(EE)                                                                                               \
    hipLaunchKernelGGL((topk_rule_a_regs_kernel<EE, Values>), dim3(1), dim3(kTopkThreads), 0, st, v, ni, ki, \
                       out_indices, out_count)
    if (e <= 24) SOI_T(24);  // n in (16384, 24576]
    else if (e <= 32) SOI_T(32);
    else
        hipLaunchKernelGGL((topk_rule_a_stream_kernel<Values>), dim3(1), dim3(kTopkThreads), 0, st, v, ni, ki,
                           out_indices, out_count);
#undef SOI_T
    return launch_status(what);
}

}  // namespace soi

using namespace soi;

extern "C" int soi_topk_threshold_select(const float* abs_g, int64_t n, int64_t k, int32_t* out_indices,
                                         int32_t* out_count, void* stream) {
    return launch_topk(F32Values{abs_g}, n, k, out_indices, out_count, stream, "soi_topk_threshold_select");
}

extern "C" int soi_topk_threshold_select_f16abs(const uint16_t* gate, int64_t n, int64_t k, int32_t* out_indices,
                                                int32_t* out_count, void* stream) {
    return launch_topk(F16AbsValues{gate}, n, k, out_indices, out_count, stream, "soi_topk_threshold_select_f16abs");
}
