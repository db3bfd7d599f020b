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
// gfx950 design: ONE workgroup of 16 waves holds all values in registers
// (element i = j*1024 + tid). Each bisection step is one compare per element,
// a 64-lane ballot + popcount per wave, and one LDS exchange of 16 per-wave
// counts behind a single barrier (double-buffered by step parity, so no second
// barrier is needed). Every thread replays lo/hi/mid redundantly in fp32 in
// the same order as the reference's thread 0. The final compaction is an
// ordered ballot prefix scan: position = (elements before this block) +
// (earlier waves in this block) + (earlier lanes in this wave), so the
// output order is ascending index order by construction.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

constexpr int kTopkThreads = 1024;
constexpr int kTopkWaves = kTopkThreads / kWave;
constexpr int kBisectionSteps = 24;

__device__ __forceinline__ uint32_t popc64(uint64_t m) { return static_cast<uint32_t>(__builtin_popcountll(m)); }

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

// E values per thread held in registers: n <= 1024*E.
template <int E>
__global__ __launch_bounds__(kTopkThreads) void topk_rule_a_regs_kernel(const float* __restrict__ v, int n, int k,
                                                                         int32_t* __restrict__ out_idx,
                                                                         int32_t* __restrict__ out_count) {
    __shared__ float s_max[kTopkWaves];
    __shared__ uint32_t s_cnt[2][kTopkWaves];
    __shared__ uint32_t s_blk[E][kTopkWaves];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    float val[E];
    float local_max = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = j * kTopkThreads + tid;
        val[j] = (i < n) ? v[i] : -__builtin_inff();
        local_max = fmaxf(local_max, val[j]);
    }
    const float total_max = block_max_from(local_max, s_max, wave, lane);

    float lo = 0.0f;
    float hi = total_max + 1e-3f;
#pragma unroll 1
    for (int it = 0; it < kBisectionSteps; ++it) {
        const float mid = 0.5f * (lo + hi);
        uint32_t cnt = 0;
#pragma unroll
        for (int j = 0; j < E; ++j) cnt += popc64(ballot(val[j] >= mid));
        if (lane == 0) s_cnt[it & 1][wave] = cnt;
        __syncthreads();
        uint32_t total = 0;
#pragma unroll
        for (int w = 0; w < kTopkWaves; ++w) total += s_cnt[it & 1][w];
        if (total >= static_cast<uint32_t>(k))
            lo = mid;
        else
            hi = mid;
    }
    const float tau = lo;

    uint64_t m[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        m[j] = ballot(val[j] >= tau);
        if (lane == 0) s_blk[j][wave] = popc64(m[j]);
    }
    __syncthreads();
    uint32_t running = 0;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        uint32_t before = 0, blk = 0;
#pragma unroll
        for (int w = 0; w < kTopkWaves; ++w) {
            const uint32_t c = s_blk[j][w];
            before += (w < wave) ? c : 0u;
            blk += c;
        }
        const bool flag = val[j] >= tau;
        const uint32_t pos = running + before + mask_prefix(m[j]);
        if (flag && pos < static_cast<uint32_t>(k)) out_idx[pos] = j * kTopkThreads + tid;
        running += blk;
    }
    if (tid == 0) *out_count = static_cast<int32_t>(running < static_cast<uint32_t>(k) ? running : k);
}

// Any n: values streamed from global memory (L2-resident after the first
// pass) in blocks of 1024, same arithmetic and same output order.
__global__ __launch_bounds__(kTopkThreads) void topk_rule_a_stream_kernel(const float* __restrict__ v, int n, int k,
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

}  // namespace soi

using namespace soi;

extern "C" int soi_topk_threshold_select(const float* abs_g, int64_t n, int64_t k, int32_t* out_indices,
                                         int32_t* out_count, void* stream) {
    const char* what = "soi_topk_threshold_select";
    SOI_REQUIRE(n >= 1 && n <= (int64_t(1) << 30), "%s: n must be in [1, 2^30]", what);
    SOI_REQUIRE(k >= 1 && k <= n, "%s: k must be in [1, n]", what);
    SOI_REQUIRE(abs_g && out_indices && out_count, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    const int ni = static_cast<int>(n), ki = static_cast<int>(k);
    const int64_t e = ceil_div64(n, kTopkThreads);
#define SOI_T(EE)                                                                                                   \
    hipLaunchKernelGGL((topk_rule_a_regs_kernel<EE>), dim3(1), dim3(kTopkThreads), 0, st, abs_g, ni, ki, out_indices, \
                       out_count)
    if (e <= 1) SOI_T(1);
    else if (e <= 2) SOI_T(2);
    else if (e <= 4) SOI_T(4);
    else if (e <= 6) SOI_T(6);
    else if (e <= 8) SOI_T(8);
    else if (e <= 12) SOI_T(12);
    else if (e <= 16) SOI_T(16);
    else if (e <= 24) SOI_T(24);
    else if (e <= 32) SOI_T(32);
    else
        hipLaunchKernelGGL(topk_rule_a_stream_kernel, dim3(1), dim3(kTopkThreads), 0, st, abs_g, ni, ki, out_indices,
                           out_count);
#undef SOI_T
    return launch_status(what);
}
