// Grid-wide barrier among co-resident workgroups, and the measurement of its
// cost (soi_grid_barrier_bench).
//
// A persistent decode launch (one launch per layer or per token, workgroups
// held across the layer's dependent GEMVs) replaces each launch boundary by
// a grid barrier. It pays only if the barrier costs less than a boundary of
// a captured graph (about 1.6 us between two dependent kernels on MI355X).
// This file holds the cheapest barrier found and measures it in place:
//
//  * arrival is O(P) and spread over 8 counters: workgroup b adds 1 to
//    counter b % 8 (one per XCD under the round-robin dispatch, each on its
//    own 256-byte line); the arrival that completes a counter adds 1 to a
//    global counter; the arrival that completes that one publishes the next
//    generation in 8 copies (one line per XCD). One lane per workgroup polls
//    its XCD's copy, with s_sleep between polls. Counters only grow:
//    barrier number g completes a counter of m members at (g + 1) * m
//    (mod 2^32), so nothing is reset between barriers, calls or replays;
//  * data exchanged across the barrier is written and read device-coherent
//    (st_agent / ld_agent, sc1), so neither an L2 write-back before arrival
//    nor an L2 invalidate after the wait is needed (fenced = 1 adds them, as
//    a release / acquire pair at agent scope, for comparison);
//  * every wait is bounded: a workgroup that gives up sets the error word,
//    and the other waiters see it and leave, so a launch always drains.
//
// The measurement: P workgroups of 256 threads run R rounds of (write 64
// words, barrier, read another workgroup's 64 words and count mismatches).
// Per-workgroup s_memrealtime stamps (100 MHz) around the rounds give the
// launch's span; the caller takes spans at two round counts and divides.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

constexpr int kBarThreads = 256;
constexpr int kBarSpin = 1 << 20;  // polls before a waiter gives up (each a device round trip + s_sleep)

// sync block: 8 arrival counters, the global counter, 8 generation copies, 2 error words; one line each
struct BarSync {
    uint32_t cnt[8][64];
    uint32_t gcnt[64];
    uint32_t gen[8][64];
    uint32_t err[64];  // err[0]: a wait gave up; err[1]: mismatched words read across a barrier
};

template <bool FENCED>
__device__ __forceinline__ void grid_barrier(BarSync* s, uint32_t& gen) {
    const int b = static_cast<int>(blockIdx.x), P = static_cast<int>(gridDim.x);
    arrive_coherent();
    if (threadIdx.x == 0) {
        if (FENCED) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        const int x = b & 7;
        const uint32_t members = static_cast<uint32_t>((P >> 3) + (x < (P & 7) ? 1 : 0));
        const uint32_t groups = P < 8 ? static_cast<uint32_t>(P) : 8u;
        bool last = false;
        const uint32_t o = __hip_atomic_fetch_add(&s->cnt[x][0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (o + 1u == (gen + 1u) * members) {
            const uint32_t o2 = __hip_atomic_fetch_add(&s->gcnt[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = o2 + 1u == (gen + 1u) * groups;
        }
        if (last) {
            for (int i = 0; i < 8; ++i)
                __hip_atomic_store(&s->gen[i][0], gen + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        int spins = 0;
        while (__hip_atomic_load(&s->gen[x][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gen) {
            if (++spins > kBarSpin) {
                __hip_atomic_store(&s->err[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            if ((spins & 255) == 0 &&
                __hip_atomic_load(&s->err[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u)
                break;  // another workgroup gave up: leave too, so the launch drains
            __builtin_amdgcn_s_sleep(1);
        }
        if (FENCED) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    }
    ++gen;
    __syncthreads();
}

template <bool FENCED>
__global__ __launch_bounds__(kBarThreads) void grid_barrier_bench_kernel(BarSync* __restrict__ s,
                                                                         uint64_t* __restrict__ stamps,
                                                                         uint32_t* __restrict__ data, int rounds) {
    __shared__ uint32_t s_gen;
    const int t = threadIdx.x, b = static_cast<int>(blockIdx.x), P = static_cast<int>(gridDim.x);
    if (t == 0) s_gen = __hip_atomic_load(&s->gen[0][0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    uint32_t gen = s_gen;
    if (t == 0) stamps[2 * b] = __builtin_amdgcn_s_memrealtime();
    uint32_t bad = 0;
    for (int r = 0; r < rounds; ++r) {
        uint32_t* buf = data + static_cast<int64_t>(r & 1) * P * 64;
        const uint32_t v = (gen * 2654435761u) ^ static_cast<uint32_t>(b * 64 + t);
        if (t < 64) {
            if (FENCED)
                stg(buf + b * 64 + t, v);
            else
                __hip_atomic_store(buf + b * 64 + t, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        grid_barrier<FENCED>(s, gen);
        if (t < 64) {
            const int o = (b + 1 + r % (P > 1 ? P - 1 : 1)) % P;  // a different workgroup each round
            const uint32_t want = ((gen - 1u) * 2654435761u) ^ static_cast<uint32_t>(o * 64 + t);
            const uint32_t got = FENCED ? ldg(buf + o * 64 + t)
                                        : __hip_atomic_load(buf + o * 64 + t, __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
            bad += got != want ? 1u : 0u;
        }
    }
    if (t == 0) stamps[2 * b + 1] = __builtin_amdgcn_s_memrealtime();
    if (bad) atomicAdd(&s->err[1], bad);
}

}  // namespace soi

using namespace soi;

extern "C" size_t soi_grid_barrier_bench_workspace_bytes(int64_t P) {
    if (P < 1) return 0;
    return sizeof(BarSync) + static_cast<size_t>(P) * 2 * sizeof(uint64_t) +
           static_cast<size_t>(P) * 2 * 64 * sizeof(uint32_t);
}

extern "C" int soi_grid_barrier_max_workgroups(int64_t* max_workgroups) {
    const char* what = "soi_grid_barrier_max_workgroups";
    SOI_REQUIRE(max_workgroups, "%s: null pointer", what);
    int dev = 0, cus = 0, per_cu = 0, per_cu_f = 0;
    SOI_HIP_TRY(hipGetDevice(&dev), what);
    SOI_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), what);
    SOI_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, grid_barrier_bench_kernel<false>, kBarThreads, 0),
                what);
    SOI_HIP_TRY(
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_f, grid_barrier_bench_kernel<true>, kBarThreads, 0), what);
    *max_workgroups = static_cast<int64_t>(cus) * (per_cu < per_cu_f ? per_cu : per_cu_f);
    return SOI_OK;
}

extern "C" int soi_grid_barrier_bench(int fenced, int64_t P, int64_t rounds, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    const char* what = "soi_grid_barrier_bench";
    int64_t max_p = 0;
    int s = soi_grid_barrier_max_workgroups(&max_p);
    if (s) return s;
    // every workgroup must be resident at once, or the barrier's waits would wait on workgroups not yet running
    SOI_REQUIRE(P >= 1 && P <= max_p, "%s: P = %lld workgroups, this GPU holds at most %lld at once", what,
                (long long)P, (long long)max_p);
    SOI_REQUIRE(rounds >= 1 && rounds <= 100000, "%s: rounds must be in [1, 100000]", what);
    SOI_REQUIRE(workspace && workspace_bytes >= soi_grid_barrier_bench_workspace_bytes(P) && aligned16(workspace),
                "%s: 16-byte aligned workspace of %zu bytes required (zero-filled before the first call)", what,
                soi_grid_barrier_bench_workspace_bytes(P));
    BarSync* sync = static_cast<BarSync*>(workspace);
    uint64_t* stamps = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + sizeof(BarSync));
    uint32_t* data = reinterpret_cast<uint32_t*>(stamps + 2 * P);
    const dim3 grid(static_cast<unsigned>(P)), block(kBarThreads);
    if (fenced)
        hipLaunchKernelGGL(grid_barrier_bench_kernel<true>, grid, block, 0, as_stream(stream), sync, stamps, data,
                           static_cast<int>(rounds));
    else
        hipLaunchKernelGGL(grid_barrier_bench_kernel<false>, grid, block, 0, as_stream(stream), sync, stamps, data,
                           static_cast<int>(rounds));
    return launch_status(what);
}
