// Split plan of the decode attention kernels (decode_attention.hip): how many
// workgroups share one KV head's timesteps. Evaluated on the host (grid sizes,
// workspace) and on the device (the device-position forms, which read the
// context length at run time, and the o projection's combine of split states),
// so both sides see one partition. Kept apart from the kernels so a host-only
// build can check its invariants over every length.
#pragma once

#include <stdint.h>

namespace soi {

constexpr int kAttnPassMax = 8;  // passes whose K/V rows a lane requests at once (8 x 32 bytes)
// Split contexts aim at this many workgroups in all: fewer, longer splits
// trade stream time per workgroup against the arrival on each KV head's
// counter and the combine, which both grow with the splits per KV head.
// Up to kAttnMidRows timestep rows in all (L * NKV) the arrival and combine
// weigh more, and half as many workgroups are faster (measured at L = 512:
// 7.3 against 8.5 us; at L = 2048 and 4096 the larger target wins or ties).
constexpr int kAttnTargetGroups = 128;
constexpr int kAttnMidGroups = 64;
constexpr int64_t kAttnMidRows = 8192;

// Plan for a context of L timesteps, `step` = timesteps one workgroup pass
// covers: one workgroup per KV head when L fits kAttnPassMax passes, else
// about kAttnMidGroups or kAttnTargetGroups workgroups, tps a multiple of step. The host and
// the device (the device-position forms, which read L at run time) use this
// same function, so both give the same partition and bit-identical results.
// ns <= ceil(kAttnTargetGroups/NKV) and ns <= ceil(L/step) for every L.
// Every quantity fits in 32 bits (L * NKV < 2^31: plan_attention takes the fast kernels only then) and step and
// both group targets are powers of two, so the device evaluates the plan with shifts, a mask and one 32-bit
// division instead of three 64-bit division sequences (on the critical path of the device-position forms and of
// the o projection's combine).
constexpr int kAttnMidGroupsLog2 = 6, kAttnTargetGroupsLog2 = 7;
static_assert((1 << kAttnMidGroupsLog2) == kAttnMidGroups && (1 << kAttnTargetGroupsLog2) == kAttnTargetGroups,
              "split targets are powers of two");
__host__ __device__ __forceinline__ void split_plan(int64_t L64, int64_t NKV64, int64_t step64, int& tps, int& ns) {
    const uint32_t L = static_cast<uint32_t>(L64), NKV = static_cast<uint32_t>(NKV64);
    const uint32_t step = static_cast<uint32_t>(step64);  // a power of two
    if (L <= kAttnPassMax * step) {
        tps = static_cast<int>(L);
        ns = 1;
        return;
    }
    const uint32_t rows = L * NKV;
    const int lg = rows <= static_cast<uint32_t>(kAttnMidRows) ? kAttnMidGroupsLog2 : kAttnTargetGroupsLog2;
    uint32_t t = (rows + (1u << lg) - 1u) >> lg;  // ceil(rows / groups)
    t = (t + step - 1u) & ~(step - 1u);           // rounded up to a multiple of step
    if (t < step) t = step;
    tps = static_cast<int>(t);
    ns = static_cast<int>((L + t - 1u) / t);
}

}  // namespace soi
