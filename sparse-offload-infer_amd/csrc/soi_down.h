// Sparse down projection over selected rows of down_proj^T: the work of one
// (column slice, row chunk) item, shared by the kernels of sparse_down.hip
// (one item per workgroup). See sparse_down.hip for the layout and the
// arithmetic.
#pragma once

#include "soi_device.h"
#include "soi_rows.h"

namespace soi {

// Coefficient sources: h_sel given (PlainH), or the SiLU gating of the
// selected channels computed on the fly (GatedH: h_j = fp16(silu(gate[c]) *
// up[c]), c = idx[j], the rounding of the indexed SiLU GEMV epilogue and of
// generate.py:304-305; a channel outside [0, n) gives NaN). As for the row
// sources, key(j) is the first load, fetch() the dependent loads and value()
// the arithmetic, so a kernel can issue every row's loads before using any.
struct PlainH {
    const uint16_t* h;
    struct Raw {
        uint16_t b;
    };
    __device__ __forceinline__ int64_t key(int64_t j) const { return j; }
    __device__ __forceinline__ Raw fetch(int64_t k) const { return {ldg(h + k)}; }
    __device__ __forceinline__ static float value(Raw r) { return f16_bits_to_f32(r.b); }
};
struct GatedH {
    const uint16_t* gate;
    const uint16_t* up;
    const int32_t* idx;
    int n;
    struct Raw {
        uint16_t g, u;
        bool ok;
    };
    __device__ __forceinline__ int64_t key(int64_t j) const { return ldg(idx + j); }
    __device__ __forceinline__ Raw fetch(int64_t c) const {
        const bool ok = c >= 0 && c < n;
        const int64_t cc = ok ? c : 0;
        return {ldg(gate + cc), ldg(up + cc), ok};
    }
    __device__ __forceinline__ static float value(Raw r) {
        const float g = f16_bits_to_f32(r.g);
        const float u = f16_bits_to_f32(r.u);
        return r.ok ? f16_bits_to_f32(f32_to_f16_bits(silu_f32(g) * u)) : __builtin_nanf("");
    }
};

constexpr int kDownWaves = 4;
constexpr int kDownThreads = kDownWaves * kWave;
constexpr int kSliceChunks = 8;                 // 16-byte chunks per slice
constexpr int kSliceCols = kSliceChunks * 32;   // 256 columns
constexpr int kGroupRows = kWave / kSliceChunks;  // 8 rows per wave-wide load
constexpr int kRedPitch = 33;                   // LDS floats per (row lane, chunk): conflict-free columns
constexpr int kDownU = 6;                       // 8-row groups per wave per batch

// U groups per wave per batch (a lane with no chunk or a row past the range
// reads g_zero16 instead, so the loads are issued unconditionally).
constexpr int kRedFloats = kDownWaves * kGroupRows * kSliceChunks * kRedPitch;

// One workgroup's share: rows [r*rpc, min((r+1)*rpc, k)) of slice `slice`
// (both from down_item), then the partial row, the arrival and (last workgroup
// of the slice) the combine. red: kRedFloats floats of LDS; s_last: one LDS word.
// The work of item (slice, r) by a group of kDownWaves waves; gtid = the
// thread's index inside its group. Every thread of the workgroup must call it
// the same number of times (it holds workgroup barriers); a group with no item
// passes active = false and only takes part in the barriers. A workgroup may run
// several groups side by side, each with its own red / s_last.
template <int U, bool VEC, bool CHUNK_SCALE, class Rows, class HS>
__device__ __forceinline__ void sparse_down_item(const Rows& rows, const HS& hs, uint16_t* __restrict__ y,
                                                 float* __restrict__ partial, uint32_t* __restrict__ counters,
                                                 int64_t k, int H, int gs, int rpc, int R, float* red, int* s_last_p,
                                                 int slice, int r, int gtid, bool active) {
    constexpr int SC = CHUNK_SCALE ? 1 : 4;
    int& s_last = *s_last_p;
    const int tid = gtid, wave = gtid >> 6, lane = gtid & 63;
    const int rs = lane >> 3, cc = lane & (kSliceChunks - 1);
    const int words = (H + 7) >> 3;
    const int chunks = (words + 3) >> 2;
    const int c = slice * kSliceChunks + cc;
    const bool cvalid = c < chunks;
    const int64_t j0 = static_cast<int64_t>(r) * rpc;
    const int64_t j1 = !active ? j0 : ((j0 + rpc < k) ? j0 + rpc : k);
    const uint32_t* z = g_zero16;
    const float* zf = reinterpret_cast<const float*>(g_zero16);

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.0f;

    constexpr int kBatchRows = kDownWaves * kGroupRows * U;
    for (int64_t jb = j0 + static_cast<int64_t>(wave) * kGroupRows; jb < j1; jb += kBatchRows) {
        uint32_t wv[U][4];
        float coef[U][SC];
        // Loads complete in order, so a lookup issued after another row's weight chunk could only be used once
        // that chunk had arrived too. Every group's loads are therefore issued level by level (keys, dependent
        // lookups, weight chunks and scales), with scheduling barriers between the levels, before any arithmetic.
        int64_t jc[U], rk[U], hk[U];
        bool in[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = jb + static_cast<int64_t>(u) * kDownWaves * kGroupRows + rs;
            in[u] = j < j1;
            jc[u] = in[u] ? j : j0;  // unconditional loads from a clamped row: no branch around a load
            rk[u] = rows.key(jc[u]);
            hk[u] = hs.key(jc[u]);
        }
        __builtin_amdgcn_sched_barrier(0);
        RowRef ref[U];
        typename HS::Raw hr[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            ref[u] = rows.resolve(rk[u], jc[u]);
            hr[u] = hs.fetch(hk[u]);
        }
        __builtin_amdgcn_sched_barrier(0);
        float sv[U][SC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool ok = in[u] && ref[u].ok && cvalid;
            if (VEC) {
                const u32x4 t = __builtin_nontemporal_load(ok ? reinterpret_cast<const u32x4*>(ref[u].w) + c
                                                              : reinterpret_cast<const u32x4*>(z));
                wv[u][0] = t.x;
                wv[u][1] = t.y;
                wv[u][2] = t.z;
                wv[u][3] = t.w;
            } else {
                const uint32_t* rw = reinterpret_cast<const uint32_t*>(ref[u].w);
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[u][i] = *((ok && 4 * c + i < words) ? rw + 4 * c + i : z);
            }
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const int wi = 4 * c + i;
                sv[u][i] = CHUNK_SCALE ? *(ok ? ref[u].s + (32 * c) / gs : zf)
                                       : *((ok && wi < words) ? ref[u].s + (8 * wi) / gs : zf);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const float hj = in[u] ? HS::value(hr[u]) : 0.0f;
            const float bad = (in[u] && !ref[u].ok) ? __builtin_nanf("") : 1.0f;  // unresolvable row -> NaN
#pragma unroll
            for (int i = 0; i < SC; ++i) coef[u][i] = (hj * sv[u][i]) * bad;
        }
        // Phase 3: the accumulation
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f16x2 q[4];
                dequant_int4x8_bitfield(wv[u][i], q);
                const float cf = coef[u][CHUNK_SCALE ? 0 : i];
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    acc[8 * i + 2 * p] = fmaf(cf, static_cast<float>(q[p].x), acc[8 * i + 2 * p]);
                    acc[8 * i + 2 * p + 1] = fmaf(cf, static_cast<float>(q[p].y), acc[8 * i + 2 * p + 1]);
                }
            }
        }
    }

    // partial row of the slice: column (cc, i) summed over (wave, rs) in ascending order
    float* red_lane = red + ((wave * kGroupRows + rs) * kSliceChunks + cc) * kRedPitch;
#pragma unroll
    for (int i = 0; i < 32; ++i) red_lane[i] = acc[i];
    __syncthreads();
    const int tc = tid >> 5, ti = tid & 31;  // thread tid <-> slice column tid = 32*tc + ti
    float part = 0.0f;
#pragma unroll
    for (int g = 0; g < kDownWaves * kGroupRows; ++g) part += red[(g * kSliceChunks + tc) * kRedPitch + ti];
    const int64_t col = static_cast<int64_t>(slice) * kSliceCols + tid;
    // the partial row goes out device-coherent (the slice's other items may run on other XCDs)
    if (active && col < H) st_agent(partial + static_cast<int64_t>(r) * H + col, part);

    // arrival: the last of the slice's R items sums the partial rows (arrive_coherent: no L2 write-back or
    // invalidate, the partial rows are written and read device-coherent)
    arrive_coherent();
    if (tid == 0) {
        bool last = false;
        if (active) {
            const uint32_t prev = atomicAdd(counters + slice, 1u);
            last = prev + 1 == static_cast<uint32_t>(R);
            if (last) atomicExch(counters + slice, 0u);
        }
        s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    if (col >= H) return;
    const float* pc = partial + col;
    float sum = 0.0f;
    int rr = 0;
    for (; rr + 8 <= R; rr += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = ld_agent(pc + static_cast<int64_t>(rr + u) * H);
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += v[u];
    }
    for (; rr < R; ++rr) sum += ld_agent(pc + static_cast<int64_t>(rr) * H);
    stg(y + col, f32_to_f16_bits(sum));
}

// Item (slice, row chunk) of the workgroup in a grid of S x R workgroups. Workgroups are dispatched to the 8
// XCDs round-robin by linear id; with R a multiple of 8, XCD x takes row chunks x, x + 8, ... of every slice
// (linear id 8i + x -> slice i % S, chunk x + 8 (i / S)), so the S workgroups reading the same rows share one
// L2: each row's scale line, index and coefficient are fetched once per chunk instead of once per slice (the
// identity order put every slice on its own XCD, each fetching every row's 64-byte scale line). Otherwise the
// identity order.
__device__ __forceinline__ void down_item(int& slice, int& r) {
    const int S = static_cast<int>(gridDim.x), R = static_cast<int>(gridDim.y);
    if (R % 8 == 0) {
        const int L = static_cast<int>(blockIdx.x) + S * static_cast<int>(blockIdx.y);
        const int x = L & 7, i = L >> 3;
        slice = i % S;
        r = x + 8 * (i / S);
    } else {
        slice = static_cast<int>(blockIdx.x);
        r = static_cast<int>(blockIdx.y);
    }
}

// Partition: S = ceil(chunks / 8) slices; each slice's k rows split into R
// chunks of rpc rows (a multiple of 32: one 8-row group per wave), R as small
// as one load batch per wave allows (rpc <= 4 waves x 8 rows x kDownU = 192),
// but at least 64 workgroups in all (at least 4 chunks per slice). Fewer,
// fuller chunks mean fewer arrivals on each slice's counter and fewer partial
// rows for the last workgroup to sum, while every wave still makes a single
// round trip for its rows (swept at H = 2048: 32 chunks of 96 rows at
// k = 3072 took 8.5 us, 16 of 192 rows 7.0 us, 8 of 384 rows (two batches)
// 8.2 us; at k = 768, 8 chunks of 96 rows 5.7 us against 7.0 us for 24 of 32).
struct DownPlan {
    int64_t S, R, rpc;
};

inline DownPlan down_plan(int64_t H, int64_t k) {
    auto ceil_div64 = [](int64_t a, int64_t b) { return (a + b - 1) / b; };
    const int64_t chunks = ceil_div64(ceil_div64(H, 8), 4);
    DownPlan p;
    p.S = ceil_div64(chunks, kSliceChunks);
    const int64_t step = static_cast<int64_t>(kDownWaves) * kGroupRows;
    const int64_t batch = step * kDownU;
    int64_t target = ceil_div64(k, batch);
    int64_t floor_chunks = ceil_div64(64, p.S);
    if (floor_chunks < 4) floor_chunks = 4;
    if (target < floor_chunks) target = floor_chunks;
    p.rpc = ceil_div64(ceil_div64(k, target), step) * step;
    p.R = ceil_div64(k, p.rpc);
    return p;
}

}  // namespace soi
