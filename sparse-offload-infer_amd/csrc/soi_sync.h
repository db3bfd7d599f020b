// Grid-wide barrier for a launch whose workgroups are all resident at once
// (grid <= number of CUs, one workgroup per CU fits): the single-launch DIP
// MLP crosses two all-to-all dependencies (every gate before the selection,
// every gated up value before the down projection) inside one kernel.
//
// Flag array, no same-address atomics: workgroup b publishes a running count
// in its own word flags[b]; every workgroup waits until all P words have
// reached the barrier's target. 256 workgroups incrementing one counter
// serialise on that address; separate words do not. Targets come from a
// per-call epoch kept in device memory (read at kernel start, advanced by
// workgroup 0 after the last barrier), so no flag is ever reset and graph
// replays need no host involvement: call e uses targets 2e+1 and 2e+2.
//
// Memory ordering (agent scope = all XCDs of the GPU, whose L2s are not
// coherent with each other): before publishing, every wave waits for its
// stores and thread 0 issues a device-scope release (L2 write-back, waited
// for: release_agent); after the wait, every wave issues a device-scope
// acquire fence (L2/L1 invalidate) before reading data other workgroups wrote.
//
// Every wait is bounded: after kSpinLimit polls the waiting workgroup records
// an error in the sync block and proceeds (the call's output is then not
// valid, and the host reports it), so no wave can spin forever even if the
// co-residency assumption were broken.
#pragma once

#include "soi_device.h"

namespace soi {

// sync block (zero-filled once by the caller, then maintained by the kernels)
struct GridSync {
    uint32_t epoch;  // completed calls
    uint32_t error;  // nonzero once a barrier wait gave up
};
constexpr int kSyncHeaderBytes = 256;  // header, then flags[P] (uint32 each)
constexpr int kSpinLimit = 1 << 20;    // polls (each a device round trip plus s_sleep): about a second

__device__ __forceinline__ uint32_t* sync_flags(uint32_t* sync) {
    return sync + kSyncHeaderBytes / sizeof(uint32_t);
}

// Epoch of this call, read by thread 0 and broadcast through s_word.
__device__ __forceinline__ uint32_t grid_epoch(uint32_t* sync, uint32_t* s_word) {
    if (threadIdx.x == 0)
        *s_word = __hip_atomic_load(&reinterpret_cast<GridSync*>(sync)->epoch, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *s_word;
}

// Wave-uniform: has every one of the P flags reached `target` (wrap-safe)?
__device__ __forceinline__ bool flags_reached(const uint32_t* flags, int P, uint32_t target, int lane) {
    bool mine = true;
    for (int i = lane; i < P; i += kWave) {
        const uint32_t f = __hip_atomic_load(flags + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mine = mine && static_cast<int32_t>(f - target) >= 0;
    }
    return ballot(!mine) == 0;
}

// All workgroups of the launch (P = gridDim.x) arrive and leave together.
__device__ __forceinline__ void grid_barrier(uint32_t* sync, uint32_t target) {
    const int tid = threadIdx.x;
    uint32_t* flags = sync_flags(sync);
    const int P = static_cast<int>(gridDim.x);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have reached L2
    __syncthreads();
    if (tid == 0) {
        release_agent();
        __hip_atomic_store(flags + blockIdx.x, target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (tid < kWave) {
        int spins = 0;
        while (!flags_reached(flags, P, target, tid)) {
            if (++spins >= kSpinLimit) {
                if (tid == 0)
                    __hip_atomic_store(&reinterpret_cast<GridSync*>(sync)->error, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Workgroup 0, after the call's last barrier and its own last reads of
// barrier-protected data: advance the epoch for the next call.
__device__ __forceinline__ void grid_epoch_advance(uint32_t* sync, uint32_t epoch) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(&reinterpret_cast<GridSync*>(sync)->epoch, epoch + 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace soi
