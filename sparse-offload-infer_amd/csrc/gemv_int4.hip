// INT4 group-quantized GEMV for batch-1 decode on gfx950.
//
// Restates the arithmetic of the reference's gemv_w4a16_group{,_lop3}
// (csrc/kernels/gemv_w4a16_group.cu:23-127): y[n] = sum_k s[n,k/gs]*q[n,k]*x[k],
// fp32 accumulation, binary16 output (round to nearest even).
//
// Layout of the work (one wave64 = one workgroup, R rows per wave):
//   * a row of ceil(K/8) packed words is cut into 16-byte chunks (4 words =
//     32 consecutive k); lane l owns chunk l of every 64-chunk pass, so one
//     wave-wide global_load_dwordx4 reads 1 KB of a row, fully coalesced;
//   * R rows are loaded before any arithmetic, so a wave keeps R KB in flight;
//   * dequantisation is exact (see soi_device.h) and products of two binary16
//     values are exact in binary32, so the only roundings are the fp32 sums:
//     per lane, t = ordered v_dot2 chain over the chunk's 16 pairs, then
//     acc = fma(scale, t, acc) (or one fma per word when 32 does not divide
//     group_size); finally a fixed-order DPP wave reduction.
// The bitfield and scalar dequant methods produce identical binary16 values,
// and every row source (dense / descriptor / index) feeds the same body, so
// all variants agree bit for bit.
#include "soi_device.h"
#include "soi_host.h"
#include "soi_int4_tile.h"
#include "soi_rows.h"

namespace soi {

// Side copies done by a GEMV's waves for their own rows. NoCopy: none.
// MissCopy<CH>: for each row j of the wave's tile whose channel c = sel[j] is
// not in the hot cache (slot_of[c] < 0), row c of src (row_bytes, typically
// pinned host memory read in place) is copied to row j of dst (device
// staging). The copy's loads (rows up to CH KB, read by 16 lanes of 64
// contiguous bytes per KB) are issued before the GEMV's, so both round trips
// overlap.
struct NoCopy {
    static constexpr int kChunks = 0;
};

template <int CH>
struct MissCopy {
    static constexpr int kChunks = CH;
    const int32_t* sel;
    const int32_t* slot_of;
    int64_t num_channels;
    const uint8_t* src;
    uint8_t* dst;
    int64_t row_bytes;  // multiple of 16, at most CH * 1024
    __device__ __forceinline__ int32_t miss_channel(int64_t j) const {
        const int32_t c = ldg(sel + j);
        return (c >= 0 && c < num_channels && ldg(slot_of + c) < 0) ? c : -1;
    }
};

template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool BITFIELD, bool FULL, class Rows, class EP, class CP>
__device__ __forceinline__ void gemv_int4_body(const Rows& rows, int64_t N, const uint16_t* __restrict__ x,
                                               const EP& ep, int K, int gs, const CP& cp) {
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
    if constexpr (CP::kChunks > 0) {
        // 16 lanes per row, each reading 64 contiguous bytes of every 1 KB (4 chunks): reads of pinned host
        // memory cross PCIe at ~54 GB/s this way against ~48 GB/s with 16 bytes per lane (measured on a 1 KB
        // row gather). Lane l takes rows l / 16 + 4m (m < RM) of the tile.
        constexpr int CH = CP::kChunks;
        constexpr int RM = (R + 3) / 4;
        const int lane = threadIdx.x;
        const int quarter = lane >> 4, sub = lane & 15;
        const int64_t nchunks = cp.row_bytes >> 4;
        const u32x4* z = reinterpret_cast<const u32x4*>(g_zero16);
        u32x4 buf[RM][CH][4];
        int32_t ch[RM];
#pragma unroll
        for (int m = 0; m < RM; ++m) {
            const int r = quarter + 4 * m;
            ch[m] = (r < R && row0 + r < N) ? cp.miss_channel(row0 + r) : -1;
            const u32x4* src =
                reinterpret_cast<const u32x4*>(cp.src + static_cast<int64_t>(ch[m] >= 0 ? ch[m] : 0) * cp.row_bytes);
#pragma unroll
            for (int i = 0; i < CH; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t c = 64 * i + 4 * sub + j;
                    buf[m][i][j] = ldg_stream((ch[m] >= 0 && c < nchunks) ? src + c : z);
                }
            }
        }
        gemv_int4_tile<R, PU, VEC, CHUNK_SCALE, BITFIELD, FULL>(rows, N, PlainX{x}, ep, K, gs, row0);
#pragma unroll
        for (int m = 0; m < RM; ++m) {
            if (ch[m] < 0) continue;
            u32x4* dst = reinterpret_cast<u32x4*>(cp.dst + (row0 + quarter + 4 * m) * cp.row_bytes);
#pragma unroll
            for (int i = 0; i < CH; ++i) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t c = 64 * i + 4 * sub + j;
                    if (c < nchunks) stg(dst + c, buf[m][i][j]);
                }
            }
        }
    } else {
        gemv_int4_tile<R, PU, VEC, CHUNK_SCALE, BITFIELD, FULL>(rows, N, PlainX{x}, ep, K, gs, row0);
    }
}

// Single-pass tiles: the default register budget (occupancy-driven scheduling).
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool BITFIELD, bool FULL, class Rows, class EP = StoreY,
          class CP = NoCopy>
__global__ __launch_bounds__(64) void gemv_int4_kernel(Rows rows, int64_t N, const uint16_t* __restrict__ x, EP ep,
                                                       int K, int gs, CP cp = CP{}) {
    gemv_int4_body<R, PU, VEC, CHUNK_SCALE, BITFIELD, FULL>(rows, N, x, ep, K, gs, cp);
}

// Multi-pass tiles (PU > 1: rows longer than 64 chunks, e.g. down_proj at K = 6144): at decode sizes a launch
// has about one wave per SIMD, so occupancy buys nothing, while every pass's loads must be in flight at once
// (R*PU weight chunks + PU x chunks, ~90 VGPRs). With the default budget the scheduler kept 5 waves per SIMD by
// reusing registers, which serialised the passes' loads into several round trips.
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool BITFIELD, bool FULL, class Rows, class EP = StoreY,
          class CP = NoCopy>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(1, 4))) void gemv_int4_mp_kernel(
    Rows rows, int64_t N, const uint16_t* __restrict__ x, EP ep, int K, int gs, CP cp = CP{}) {
    gemv_int4_body<R, PU, VEC, CHUNK_SCALE, BITFIELD, FULL>(rows, N, x, ep, K, gs, cp);
}

// A problem of the batched / grouped forms whose W or x is not 16-byte aligned
// while the vector path is compiled in cannot be read with dwordx4 loads: its
// rows are set to NaN, so the output is never left unwritten (the host
// wrappers reject such problems before launching).
template <int R>
__device__ __forceinline__ void misaligned_rows_nan(uint16_t* y, int64_t N, int64_t row0) {
    const int64_t r = row0 + static_cast<int64_t>(threadIdx.x);
    if (threadIdx.x < R && r < N) stg(y + r, static_cast<uint16_t>(0x7e00u));
}

// Batched form: P independent problems of one shape [N, K]; workgroup b takes
// row tile b % tiles of problem b / tiles. Pointer tables live in device
// memory; a problem with a null pointer writes nothing, a misaligned one NaN
// rows (misaligned_rows_nan).
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__device__ __forceinline__ void gemv_int4_batched_body(const uint8_t* const* __restrict__ Wp,
                                                       const float* const* __restrict__ Sp,
                                                       const uint16_t* const* __restrict__ Xp,
                                                       uint16_t* const* __restrict__ Yp, int64_t N, int K, int gs, int G,
                                                       int tiles) {
    const int p = blockIdx.x / tiles;
    const int tile = blockIdx.x - p * tiles;
    const uint8_t* W = ldg(Wp + p);
    const float* S = ldg(Sp + p);
    const uint16_t* x = ldg(Xp + p);
    uint16_t* y = ldg(Yp + p);
    if (!W || !S || !x || !y) return;
    const uintptr_t bad = reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x);
    if (VEC && (bad & 15u)) {
        misaligned_rows_nan<R>(y, N, static_cast<int64_t>(tile) * R);
        return;
    }
    const int64_t row_bytes = static_cast<int64_t>((K + 7) >> 3) * 4;
    DenseRows rows{W, S, row_bytes, G};
    gemv_int4_tile<R, PU, VEC, CHUNK_SCALE, true, FULL>(rows, N, PlainX{x}, StoreY{y}, K, gs,
                                                       static_cast<int64_t>(tile) * R);
}

#define SOI_BATCHED_PARAMS                                                                                     \
    const uint8_t* const* __restrict__ Wp, const float* const* __restrict__ Sp,                              \
        const uint16_t* const* __restrict__ Xp, uint16_t* const* __restrict__ Yp, int64_t N, int K, int gs, int G, \
        int tiles
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) void gemv_int4_batched_kernel(SOI_BATCHED_PARAMS) {
    gemv_int4_batched_body<R, PU, VEC, CHUNK_SCALE, FULL>(Wp, Sp, Xp, Yp, N, K, gs, G, tiles);
}
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) SOI_GEMV_OCCUPANCY void gemv_int4_batched_occ_kernel(SOI_BATCHED_PARAMS) {
    gemv_int4_batched_body<R, PU, VEC, CHUNK_SCALE, FULL>(Wp, Sp, Xp, Yp, N, K, gs, G, tiles);
}
#undef SOI_BATCHED_PARAMS

// Decode-step form: y = W . rmsnorm(a + d, w) with the residual add and the
// RMSNorm done on load. Every workgroup computes inv = 1/sqrt(mean((a+d)^2) +
// eps) with the same wave reduction (so all agree bit for bit); workgroup 0
// also writes x_out = a + d and h_out = rmsnorm(a + d, w) when given. a, d,
// w, x_out, h_out: fp16 [K], K % 32 == 0, 16-byte aligned; x_out and h_out
// must not alias a or d (other workgroups are still reading them). OP: 0 the
// general form, 1 the one-pass form (K == 2048) with d, 2 the one-pass form
// without d (its lanes load only a and w).
template <int R, bool CHUNK_SCALE, bool FULL, int OP, class EP>
__global__ __launch_bounds__(64) void gemv_int4_norm_kernel(DenseRows rows, int64_t N, const uint16_t* __restrict__ a,
                                                            const uint16_t* __restrict__ d,
                                                            const uint16_t* __restrict__ w, float eps,
                                                            uint16_t* __restrict__ x_out, uint16_t* __restrict__ h_out,
                                                            EP ep, int K, int gs) {
    const int lane = threadIdx.x;
    const u32x4* a4 = reinterpret_cast<const u32x4*>(a);
    const u32x4* d4 = reinterpret_cast<const u32x4*>(d);
    const u32x4* w4 = reinterpret_cast<const u32x4*>(w);
    if constexpr (OP != 0) {
        // K == 2048: lane l's 32 elements are exactly its GEMV chunk. Its a / d / w chunks are requested here, the
        // tile then issues the weight loads, and the add + RMSNorm run while those are in flight (RegNormX).
        static_assert(FULL, "the one-pass norm form needs the full tile");
        RegNormX xs;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xs.t[i] = ldg(a4 + 4 * lane + i);
            xs.g[i] = ldg(w4 + 4 * lane + i);
            if constexpr (OP == 1) xs.e[i] = ldg(d4 + 4 * lane + i);  // compile-time choice: no branch at run time
        }
        xs.has_d = OP == 1;
        xs.eps = eps;
        xs.K = K;
        xs.x_out = blockIdx.x == 0 ? x_out : nullptr;
        xs.h_out = blockIdx.x == 0 ? h_out : nullptr;
        xs.b = a;
        gemv_int4_tile<R, 1, true, CHUNK_SCALE, true, FULL>(rows, N, xs, ep, K, gs, static_cast<int64_t>(blockIdx.x) * R);
        return;
    }
    const int n8 = K >> 3;
    float ss = 0.0f;
    for (int c = lane; c < n8; c += kWave) {
        u32x4 t = ldg(a4 + c);
        if (d) {
            const u32x4 e = ldg(d4 + c);
            t.x = add_f16x2(t.x, e.x);
            t.y = add_f16x2(t.y, e.y);
            t.z = add_f16x2(t.z, e.z);
            t.w = add_f16x2(t.w, e.w);
        }
        ss += sumsq_f16x2(t.x) + sumsq_f16x2(t.y) + sumsq_f16x2(t.z) + sumsq_f16x2(t.w);
    }
    const float inv = rsqrtf(wave_sum_bcast(ss) / static_cast<float>(K) + eps);
    if (blockIdx.x == 0 && (x_out || h_out)) {
        for (int c = lane; c < n8; c += kWave) {
            u32x4 t = ldg(a4 + c);
            if (d) {
                const u32x4 e = ldg(d4 + c);
                t.x = add_f16x2(t.x, e.x);
                t.y = add_f16x2(t.y, e.y);
                t.z = add_f16x2(t.z, e.z);
                t.w = add_f16x2(t.w, e.w);
            }
            if (x_out) stg(reinterpret_cast<u32x4*>(x_out) + c, t);
            if (h_out) {
                const u32x4 g = ldg(w4 + c);
                u32x4 r;
                r.x = norm_f16x2(t.x, g.x, inv);
                r.y = norm_f16x2(t.y, g.y, inv);
                r.z = norm_f16x2(t.z, g.z, inv);
                r.w = norm_f16x2(t.w, g.w, inv);
                stg(reinterpret_cast<u32x4*>(h_out) + c, r);
            }
        }
    }
    gemv_int4_tile<R, 1, true, CHUNK_SCALE, true, FULL>(rows, N, NormX{a, d, w, inv}, ep, K, gs,
                                                       static_cast<int64_t>(blockIdx.x) * R);
}

// Grouped form: problems of up to kMaxClasses shapes in one launch. Class c
// owns workgroups [first_wg[c], first_wg[c+1]) and problems
// [first_problem[c], first_problem[c] + count[c]) of the pointer tables; the
// class of a workgroup is found by comparisons against kernel arguments
// (constant indices only, so the table stays in SGPRs).
constexpr int kMaxClasses = 8;

struct GroupClasses {
    int n;
    int first_wg[kMaxClasses];
    int tiles[kMaxClasses];
    int first_problem[kMaxClasses];
    int N[kMaxClasses];
    int K[kMaxClasses];
    int G[kMaxClasses];
};

template <int R, bool VEC, bool CHUNK_SCALE, bool FULL>
__device__ __forceinline__ void gemv_int4_grouped_body(const uint8_t* const* __restrict__ Wp,
                                                       const float* const* __restrict__ Sp,
                                                       const uint16_t* const* __restrict__ Xp,
                                                       uint16_t* const* __restrict__ Yp, const GroupClasses& cl,
                                                       int gs) {
    const int b = blockIdx.x;
    int first = cl.first_wg[0], tiles = cl.tiles[0], p0 = cl.first_problem[0];
    int N = cl.N[0], K = cl.K[0], G = cl.G[0];
#pragma unroll
    for (int i = 1; i < kMaxClasses; ++i) {
        if (i < cl.n && b >= cl.first_wg[i]) {
            first = cl.first_wg[i];
            tiles = cl.tiles[i];
            p0 = cl.first_problem[i];
            N = cl.N[i];
            K = cl.K[i];
            G = cl.G[i];
        }
    }
    const int local = b - first;
    const int pi = local / tiles;
    const int tile = local - pi * tiles;
    const int p = p0 + pi;
    const uint8_t* W = ldg(Wp + p);
    const float* S = ldg(Sp + p);
    const uint16_t* x = ldg(Xp + p);
    uint16_t* y = ldg(Yp + p);
    if (!W || !S || !x || !y) return;
    const uintptr_t bad = reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x);
    if (VEC && (bad & 15u)) {
        misaligned_rows_nan<R>(y, N, static_cast<int64_t>(tile) * R);
        return;
    }
    const int64_t row_bytes = static_cast<int64_t>((K + 7) >> 3) * 4;
    DenseRows rows{W, S, row_bytes, G};
    gemv_int4_tile<R, 1, VEC, CHUNK_SCALE, true, FULL>(rows, N, PlainX{x}, StoreY{y}, K, gs,
                                                      static_cast<int64_t>(tile) * R);
}

#define SOI_GROUPED_PARAMS                                                                                   \
    const uint8_t* const* __restrict__ Wp, const float* const* __restrict__ Sp,                            \
        const uint16_t* const* __restrict__ Xp, uint16_t* const* __restrict__ Yp, GroupClasses cl, int gs
template <int R, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) void gemv_int4_grouped_kernel(SOI_GROUPED_PARAMS) {
    gemv_int4_grouped_body<R, VEC, CHUNK_SCALE, FULL>(Wp, Sp, Xp, Yp, cl, gs);
}
template <int R, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) SOI_GEMV_OCCUPANCY void gemv_int4_grouped_occ_kernel(SOI_GROUPED_PARAMS) {
    gemv_int4_grouped_body<R, VEC, CHUNK_SCALE, FULL>(Wp, Sp, Xp, Yp, cl, gs);
}
#undef SOI_GROUPED_PARAMS

// The occupancy hint is applied where the tile fits its register budget
// without spilling (checked on the compiler's output): vector loads, one
// scale per chunk, and one pass per batch (or at most 4 row segments).
constexpr bool occ_fits(int R, int PU, bool VEC, bool CS, bool FULL) {
    return VEC && CS && (PU == 1 || (R * PU <= 4 && FULL));
}

template <int R, int PU, bool V, bool CS, bool FL>
static void launch_batched_kernel(dim3 grid, hipStream_t st, const uint8_t* const* Wp, const float* const* Sp,
                                  const uint16_t* const* Xp, uint16_t* const* Yp, int64_t N, int K, int gs, int G,
                                  int tiles) {
    if constexpr (occ_fits(R, PU, V, CS, FL))
        hipLaunchKernelGGL((gemv_int4_batched_occ_kernel<R, PU, V, CS, FL>), grid, dim3(64), 0, st, Wp, Sp, Xp, Yp,
                           N, K, gs, G, tiles);
    else
        hipLaunchKernelGGL((gemv_int4_batched_kernel<R, PU, V, CS, FL>), grid, dim3(64), 0, st, Wp, Sp, Xp, Yp, N, K,
                           gs, G, tiles);
}

template <int R, bool V, bool CS, bool FL>
static void launch_grouped_kernel(dim3 grid, hipStream_t st, const uint8_t* const* Wp, const float* const* Sp,
                                  const uint16_t* const* Xp, uint16_t* const* Yp, const GroupClasses& cl, int gs) {
    if constexpr (occ_fits(R, 1, V, CS, FL))
        hipLaunchKernelGGL((gemv_int4_grouped_occ_kernel<R, V, CS, FL>), grid, dim3(64), 0, st, Wp, Sp, Xp, Yp, cl,
                           gs);
    else
        hipLaunchKernelGGL((gemv_int4_grouped_kernel<R, V, CS, FL>), grid, dim3(64), 0, st, Wp, Sp, Xp, Yp, cl, gs);
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------

struct Int4Plan {
    int R, PU;
};

// PU: passes per batch (all of them up to 4); R: rows per wave, 8 for a
// one-pass tile over >= 4096 rows, else 2 from 2048 rows, else 1. Swept on
// single cold launches of the Qwen3-1.7B shapes: 4-row tiles were slower than
// both 8- and 2-row tiles at every shape (gate/up 6144x2048: 3.39 / 3.93 /
// 3.53 us for 8 / 4 / 2 rows), and more than 8 row segments in flight per
// wave did not pay.
static Int4Plan plan_int4(int64_t N, int64_t K, bool vec) {
    const int64_t chunks = ceil_div64(ceil_div64(K, 8), 4);
    const int64_t passes = ceil_div64(chunks, kWave);
    Int4Plan p{1, 1};
    p.PU = vec ? static_cast<int>(passes < 4 ? passes : 4) : 1;
    if (p.PU == 3 && passes > 3) p.PU = 4;
    p.R = (N >= 4 * 1024 && p.PU == 1) ? 8 : N >= 2 * 1024 ? 2 : 1;
    return p;
}

template <int RR, int PP, bool V, bool CS, bool BF, bool FL, class Rows, class EP, class CP>
static void launch_int4_kernel(dim3 grid, hipStream_t st, const Rows& rows, int64_t N, const uint16_t* x, const EP& ep,
                               int K, int gs, const CP& cp) {
    if constexpr (PP > 1)
        hipLaunchKernelGGL((gemv_int4_mp_kernel<RR, PP, V, CS, BF, FL, Rows, EP, CP>), grid, dim3(64), 0, st, rows, N,
                           x, ep, K, gs, cp);
    else
        hipLaunchKernelGGL((gemv_int4_kernel<RR, PP, V, CS, BF, FL, Rows, EP, CP>), grid, dim3(64), 0, st, rows, N, x,
                           ep, K, gs, cp);
}

template <bool BITFIELD, class Rows, class EP = StoreY, class CP = NoCopy>
static int launch_int4(const Rows& rows, int64_t N, const uint16_t* x, const EP& ep, int64_t K, int64_t gs, bool vec,
                       hipStream_t st, const char* what, const CP& cp = CP{}) {
    if (N == 0) return SOI_OK;
    Int4Plan pl = plan_int4(N, K, vec);
    // a multi-pass tile over more than 2048 rows: 4 rows per wave (2560 x 9728 7.7 against 8.1 us, 4096 x 12288
    // 9.9 against 10.6 us back to back on cold copies; 2048 x 6144 stays at 2 rows, 3.8 against 4.0 us)
    if (pl.PU > 1 && N > 2 * 1024) pl.R = 4;
    const bool cs = (gs % 32) == 0;
    const bool full = vec && cs && (N % pl.R == 0) && ((K / 32) % (64 * pl.PU) == 0);
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, pl.R)));
    const int Ki = static_cast<int>(K), gi = static_cast<int>(gs);
#define SOI_L(RR, PP, V, CS, FL) \
    launch_int4_kernel<RR, PP, V, CS, BITFIELD, FL>(grid, st, rows, N, x, ep, Ki, gi, cp)
#define SOI_CS(RR, PP, V)                    \
    if (V && full) SOI_L(RR, PP, V, true, true); \
    else if (cs) SOI_L(RR, PP, V, true, false);  \
    else SOI_L(RR, PP, V, false, false)
    const int key = pl.R * 10 + pl.PU;
    if (vec) {
        switch (key) {
            case 81: SOI_CS(8, 1, true); break;
            case 21: SOI_CS(2, 1, true); break;
            case 11: SOI_CS(1, 1, true); break;
            case 22: SOI_CS(2, 2, true); break;
            case 12: SOI_CS(1, 2, true); break;
            case 23: SOI_CS(2, 3, true); break;
            case 13: SOI_CS(1, 3, true); break;
            case 24: SOI_CS(2, 4, true); break;
            case 42: SOI_CS(4, 2, true); break;
            case 43: SOI_CS(4, 3, true); break;
            case 44: SOI_CS(4, 4, true); break;
            default: SOI_CS(1, 4, true); break;
        }
    } else {
        switch (pl.R) {
            case 8: SOI_CS(8, 1, false); break;
            case 2: SOI_CS(2, 1, false); break;
            default: SOI_CS(1, 1, false); break;
        }
    }
#undef SOI_CS
#undef SOI_L
    return launch_status(what);
}

static int launch_int4_batched(const uint8_t* const* Wp, const float* const* Sp, const uint16_t* const* Xp,
                               uint16_t* const* Yp, int64_t P, int64_t N, int64_t K, int64_t gs, int64_t G,
                               hipStream_t st, const char* what) {
    const bool vec = (K % 32) == 0;
    Int4Plan pl = plan_int4(N * P, K, vec);  // rows per wave chosen on the total row count
    if (P > 1) {  // throughput regime: one pass per batch, 8 rows per wave (measured best when streaming)
        pl.PU = 1;
        pl.R = (N * P >= 8 * 1024) ? 8 : pl.R;
    }
    const int64_t tiles = ceil_div64(N, pl.R);
    SOI_REQUIRE(tiles * P <= (int64_t(1) << 31) - 1, "%s: too many row tiles", what);
    const bool cs = (gs % 32) == 0;
    const bool full = vec && cs && (N % pl.R == 0) && ((K / 32) % (64 * pl.PU) == 0);
    const dim3 grid(static_cast<unsigned>(tiles * P));
    const int Ki = static_cast<int>(K), gi = static_cast<int>(gs), Gi = static_cast<int>(G), ti = static_cast<int>(tiles);
#define SOI_B(RR, PP, V, CS, FL) launch_batched_kernel<RR, PP, V, CS, FL>(grid, st, Wp, Sp, Xp, Yp, N, Ki, gi, Gi, ti)
#define SOI_BCS(RR, PP, V)                        \
    if (V && full) SOI_B(RR, PP, V, true, true);  \
    else if (cs) SOI_B(RR, PP, V, true, false);   \
    else SOI_B(RR, PP, V, false, false)
    const int key = pl.R * 10 + pl.PU;
    if (vec) {
        switch (key) {
            case 81: SOI_BCS(8, 1, true); break;
            case 21: SOI_BCS(2, 1, true); break;
            case 11: SOI_BCS(1, 1, true); break;
            case 22: SOI_BCS(2, 2, true); break;
            case 12: SOI_BCS(1, 2, true); break;
            case 23: SOI_BCS(2, 3, true); break;
            case 13: SOI_BCS(1, 3, true); break;
            case 24: SOI_BCS(2, 4, true); break;
            default: SOI_BCS(1, 4, true); break;
        }
    } else {
        switch (pl.R) {
            case 8: SOI_BCS(8, 1, false); break;
            case 2: SOI_BCS(2, 1, false); break;
            default: SOI_BCS(1, 1, false); break;
        }
    }
#undef SOI_BCS
#undef SOI_B
    return launch_status(what);
}

static int check_int4_common(int64_t K, int64_t gs, int64_t G, const char* what) {
    SOI_REQUIRE(K >= 1 && K <= (int64_t(1) << 30), "%s: K must be in [1, 2^30], got %lld", what, (long long)K);
    SOI_REQUIRE(gs >= 1 && gs % 8 == 0, "%s: group_size must be a positive multiple of 8, got %lld", what,
                (long long)gs);
    SOI_REQUIRE(G == ceil_div64(K, gs), "%s: num_groups must be ceil(K/group_size) = %lld, got %lld", what,
                (long long)ceil_div64(K, gs), (long long)G);
    return SOI_OK;
}

template <bool BITFIELD>
static int dense_int4(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N, int64_t K,
                      int64_t gs, int64_t G, void* stream, const char* what) {
    int st = check_int4_common(K, gs, G, what);
    if (st) return st;
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    if (N == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && x && y, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(Wq) && aligned16(x);
    DenseRows rows{Wq, scale, row_bytes, G};
    return launch_int4<BITFIELD>(rows, N, x, StoreY{y}, K, gs, vec, as_stream(stream), what);
}

}  // namespace soi

using namespace soi;

extern "C" int soi_gemv_w4a16_group(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N,
                                    int64_t K, int64_t group_size, int64_t num_groups, void* stream) {
    return dense_int4<false>(Wq, scale, x, y, N, K, group_size, num_groups, stream, "soi_gemv_w4a16_group");
}

extern "C" int soi_gemv_w4a16_group_lop3(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y,
                                         int64_t N, int64_t K, int64_t group_size, int64_t num_groups, void* stream) {
    return dense_int4<true>(Wq, scale, x, y, N, K, group_size, num_groups, stream, "soi_gemv_w4a16_group_lop3");
}

extern "C" int soi_gemv_w4a16_residual(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y,
                                       const uint16_t* res, uint16_t* res_out, int64_t N, int64_t K,
                                       int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_w4a16_residual";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    if (N == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && x && y && res && res_out, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(Wq) && aligned16(x);
    DenseRows rows{Wq, scale, row_bytes, num_groups};
    return launch_int4<true>(rows, N, x, StoreYAdd{y, res, res_out}, K, group_size, vec, as_stream(stream), what);
}

extern "C" int soi_gemv_dip_fused_up(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                     const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                                     const int32_t* desc, int64_t k, const uint16_t* x, uint16_t* y, int64_t K,
                                     int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_dip_fused_up";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1, "%s: k out of range", what);
    SOI_REQUIRE(cache_rows >= 0 && staging_rows >= 0, "%s: negative row count", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(desc && x && y, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(x) && (cache_rows == 0 || aligned16(cache_Wq)) &&
                     (staging_rows == 0 || aligned16(staging_Wq));
    DescRows rows{cache_Wq, cache_scale, cache_rows, staging_Wq, staging_scale, staging_rows, desc, row_bytes,
                  num_groups};
    return launch_int4<true>(rows, k, x, StoreY{y}, K, group_size, vec, as_stream(stream), what);
}

extern "C" int soi_gemv_w4a16_indexed(const uint8_t* Wq, const float* scale, int64_t num_rows, const int32_t* idx,
                                      int64_t k, const uint16_t* x, uint16_t* y, int64_t K, int64_t group_size,
                                      int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_w4a16_indexed";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1 && num_rows >= 0, "%s: k or num_rows out of range", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && idx && x && y, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(Wq) && aligned16(x);
    IndexRows rows{Wq, scale, num_rows, idx, row_bytes, num_groups};
    return launch_int4<true>(rows, k, x, StoreY{y}, K, group_size, vec, as_stream(stream), what);
}

extern "C" int soi_gemv_w4a16_grouped(const uint8_t* const* Wq_ptrs, const float* const* scale_ptrs,
                                      const uint16_t* const* x_ptrs, uint16_t* const* y_ptrs, int64_t num_classes,
                                      const int64_t* class_count, const int64_t* class_N, const int64_t* class_K,
                                      int64_t group_size, void* stream) {
    const char* what = "soi_gemv_w4a16_grouped";
    SOI_REQUIRE(num_classes >= 0 && num_classes <= kMaxClasses, "%s: num_classes must be in [0, %d], got %lld", what,
                kMaxClasses, (long long)num_classes);
    if (num_classes == 0) return SOI_OK;
    SOI_REQUIRE(class_count && class_N && class_K, "%s: null class array", what);
    SOI_REQUIRE(group_size >= 1 && group_size % 8 == 0, "%s: group_size must be a positive multiple of 8", what);
    constexpr int R = 8;
    GroupClasses cl{};
    int64_t wg = 0, problems = 0;
    bool vec = true, full = (group_size % 32) == 0;
    int n = 0;
    for (int64_t c = 0; c < num_classes; ++c) {
        const int64_t P = class_count[c], N = class_N[c], K = class_K[c];
        SOI_REQUIRE(P >= 0 && N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: class %lld count or N out of range", what,
                    (long long)c);
        SOI_REQUIRE(K >= 1 && K <= (int64_t(1) << 30), "%s: class %lld K must be in [1, 2^30]", what, (long long)c);
        if (P == 0 || N == 0) {
            problems += P;
            continue;
        }
        const int64_t tiles = ceil_div64(N, R);
        cl.first_wg[n] = static_cast<int>(wg);
        cl.tiles[n] = static_cast<int>(tiles);
        cl.first_problem[n] = static_cast<int>(problems);
        cl.N[n] = static_cast<int>(N);
        cl.K[n] = static_cast<int>(K);
        cl.G[n] = static_cast<int>(ceil_div64(K, group_size));
        vec = vec && (K % 32) == 0;
        full = full && (N % R) == 0 && ((K / 32) % 64) == 0;
        wg += tiles * P;
        problems += P;
        ++n;
        SOI_REQUIRE(wg <= (int64_t(1) << 31) - 1 && problems <= (int64_t(1) << 31) - 1, "%s: too many row tiles",
                    what);
    }
    if (n == 0) return SOI_OK;
    SOI_REQUIRE(Wq_ptrs && scale_ptrs && x_ptrs && y_ptrs, "%s: null pointer table", what);
    cl.n = n;
    full = full && vec;
    const dim3 grid(static_cast<unsigned>(wg));
    const int gi = static_cast<int>(group_size);
    const bool cs = (group_size % 32) == 0;
    hipStream_t st = as_stream(stream);
#define SOI_G(V, CS, FL) launch_grouped_kernel<R, V, CS, FL>(grid, st, Wq_ptrs, scale_ptrs, x_ptrs, y_ptrs, cl, gi)
    if (full) SOI_G(true, true, true);
    else if (vec && cs) SOI_G(true, true, false);
    else if (vec) SOI_G(true, false, false);
    else if (cs) SOI_G(false, true, false);
    else SOI_G(false, false, false);
#undef SOI_G
    return launch_status(what);
}

extern "C" int soi_gemv_w4a16_batched(const uint8_t* const* Wq_ptrs, const float* const* scale_ptrs,
                                      const uint16_t* const* x_ptrs, uint16_t* const* y_ptrs, int64_t P, int64_t N,
                                      int64_t K, int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_w4a16_batched";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(P >= 0 && N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: P or N out of range", what);
    if (P == 0 || N == 0) return SOI_OK;
    SOI_REQUIRE(Wq_ptrs && scale_ptrs && x_ptrs && y_ptrs, "%s: null pointer table", what);
    return launch_int4_batched(Wq_ptrs, scale_ptrs, x_ptrs, y_ptrs, P, N, K, group_size, num_groups,
                               as_stream(stream), what);
}

extern "C" int soi_gemv_w4a16_rmsnorm_gate_up(const uint8_t* Wq, const float* scale, const uint16_t* x,
                                              const uint16_t* delta, const uint16_t* norm_weight, float eps,
                                              uint16_t* x_out, uint16_t* h_out, uint16_t* gate_out, uint16_t* up_out,
                                              int64_t N, int64_t K, int64_t group_size, int64_t num_groups,
                                              void* stream) {
    const char* what = "soi_gemv_w4a16_rmsnorm_gate_up";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1 && N % 8 == 0, "%s: N must be a multiple of 8 (8-row tiles)",
                what);
    SOI_REQUIRE(K % 32 == 0, "%s: K must be a multiple of 32", what);
    SOI_REQUIRE(Wq && scale && x && norm_weight && gate_out && up_out, "%s: null pointer", what);
    SOI_REQUIRE(aligned16(Wq) && aligned16(x) && aligned16(norm_weight) && (!delta || aligned16(delta)) &&
                    (!x_out || aligned16(x_out)) && (!h_out || aligned16(h_out)),
                "%s: vectors and weights must be 16-byte aligned", what);
    const void* ins[2] = {x, delta};
    for (const void* o : {static_cast<const void*>(x_out), static_cast<const void*>(h_out)})
        for (const void* i : ins) SOI_REQUIRE(!o || o != i, "%s: x_out / h_out must not alias x or delta", what);
    if (N == 0) return SOI_OK;
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    DenseRows rows{Wq, scale, row_bytes, num_groups};
    hipStream_t s = as_stream(stream);
    const bool cs = (group_size % 32) == 0;
    const int Ki = static_cast<int>(K), gi = static_cast<int>(group_size);
    const bool full_k = (K / 32) % 64 == 0;
    const bool one = cs && K == 2048;
    const dim3 grid(static_cast<unsigned>(N / 8));
    const SplitGUY ep{gate_out, up_out};
#define SOI_N(CS, FL, OP)                                                                                          \
    hipLaunchKernelGGL((gemv_int4_norm_kernel<8, CS, FL, OP, SplitGUY>), grid, dim3(64), 0, s, rows, N, x, delta,   \
                       norm_weight, eps, x_out, h_out, ep, Ki, gi)
    if (one && delta) SOI_N(true, true, 1);
    else if (one) SOI_N(true, true, 2);
    else if (cs && full_k) SOI_N(true, true, 0);
    else if (cs) SOI_N(true, false, 0);
    else SOI_N(false, false, 0);
#undef SOI_N
    return launch_status(what);
}

static int rmsnorm_impl(const uint8_t* Wq, const float* scale, const uint16_t* x, const uint16_t* delta,
                        const uint16_t* norm_weight, float eps, uint16_t* x_out, uint16_t* h_out, uint16_t* gate_out,
                        uint16_t* y, int64_t N, int64_t K, int64_t group_size, int64_t num_groups, int swiglu,
                        void* stream, const char* what) {
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    SOI_REQUIRE(K % 32 == 0, "%s: K must be a multiple of 32", what);
    SOI_REQUIRE(Wq && scale && x && norm_weight && y, "%s: null pointer", what);
    SOI_REQUIRE(aligned16(Wq) && aligned16(x) && aligned16(norm_weight) && (!delta || aligned16(delta)) &&
                    (!x_out || aligned16(x_out)) && (!h_out || aligned16(h_out)),
                "%s: vectors and weights must be 16-byte aligned", what);
    const void* ins[2] = {x, delta};
    for (const void* o : {static_cast<const void*>(x_out), static_cast<const void*>(h_out)})
        for (const void* i : ins) SOI_REQUIRE(!o || o != i, "%s: x_out / h_out must not alias x or delta", what);
    SOI_REQUIRE(!swiglu || N % 8 == 0, "%s: the SwiGLU form needs N %% 8 == 0 (8-row gate/up tiles)", what);
    if (N == 0) return SOI_OK;
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    DenseRows rows{Wq, scale, row_bytes, num_groups};
    hipStream_t s = as_stream(stream);
    const bool cs = (group_size % 32) == 0;
    const int Ki = static_cast<int>(K), gi = static_cast<int>(group_size);
    const bool full_k = (K / 32) % 64 == 0;
    const bool one = cs && K == 2048;  // one 64-chunk pass: the lane's x chunk stays in registers
    if (swiglu) {
        const dim3 grid(static_cast<unsigned>(N / 8));
        const SwigluY ep{y, gate_out};
#define SOI_N(CS, FL, OP)                                                                                          \
    hipLaunchKernelGGL((gemv_int4_norm_kernel<8, CS, FL, OP, SwigluY>), grid, dim3(64), 0, s, rows, N, x, delta,    \
                       norm_weight, eps, x_out, h_out, ep, Ki, gi)
        if (one && delta) SOI_N(true, true, 1);
        else if (one) SOI_N(true, true, 2);
        else if (cs && full_k) SOI_N(true, true, 0);
        else if (cs) SOI_N(true, false, 0);
        else SOI_N(false, false, 0);
#undef SOI_N
        return launch_status(what);
    }
    // each wave normalises the whole vector before its rows, so larger tiles than the plain GEMV's pay here
    // (swept at K = 2048: N = 4096 / 6144 / 2048 best at 8 / 8 / 4 rows per wave)
    const int R = N >= 4 * 1024 ? 8 : N >= 2 * 1024 ? 4 : N >= 1024 ? 2 : 1;
    const bool full = cs && full_k && N % R == 0;
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, R)));
    const StoreY ep{y};
#define SOI_N(RR, CS, FL, OP)                                                                                      \
    hipLaunchKernelGGL((gemv_int4_norm_kernel<RR, CS, FL, OP, StoreY>), grid, dim3(64), 0, s, rows, N, x, delta,   \
                       norm_weight, eps, x_out, h_out, ep, Ki, gi)
#define SOI_NR(RR)                                      \
    if (full && one && delta) SOI_N(RR, true, true, 1); \
    else if (full && one) SOI_N(RR, true, true, 2);     \
    else if (full) SOI_N(RR, true, true, 0);            \
    else if (cs) SOI_N(RR, true, false, 0);             \
    else SOI_N(RR, false, false, 0)
    switch (R) {
        case 8: SOI_NR(8); break;
        case 4: SOI_NR(4); break;
        case 2: SOI_NR(2); break;
        default: SOI_NR(1); break;
    }
#undef SOI_NR
#undef SOI_N
    return launch_status(what);
}

extern "C" int soi_gemv_w4a16_rmsnorm(const uint8_t* Wq, const float* scale, const uint16_t* x, const uint16_t* delta,
                                      const uint16_t* norm_weight, float eps, uint16_t* x_out, uint16_t* h_out,
                                      uint16_t* y, int64_t N, int64_t K, int64_t group_size, int64_t num_groups,
                                      int swiglu, void* stream) {
    return rmsnorm_impl(Wq, scale, x, delta, norm_weight, eps, x_out, h_out, nullptr, y, N, K, group_size, num_groups,
                        swiglu, stream, "soi_gemv_w4a16_rmsnorm");
}

extern "C" int soi_gemv_w4a16_rmsnorm_swiglu_gate(const uint8_t* Wq, const float* scale, const uint16_t* x,
                                                  const uint16_t* delta, const uint16_t* norm_weight, float eps,
                                                  uint16_t* x_out, uint16_t* h_out, uint16_t* gate_out, uint16_t* y,
                                                  int64_t N, int64_t K, int64_t group_size, int64_t num_groups,
                                                  void* stream) {
    const char* what = "soi_gemv_w4a16_rmsnorm_swiglu_gate";
    SOI_REQUIRE(gate_out, "%s: null pointer", what);
    return rmsnorm_impl(Wq, scale, x, delta, norm_weight, eps, x_out, h_out, gate_out, y, N, K, group_size,
                        num_groups, 1, stream, what);
}

extern "C" int soi_gemv_w4a16_indexed_silu(const uint8_t* Wq, const float* scale, int64_t num_rows, const int32_t* idx,
                                           int64_t k, const uint16_t* x, const uint16_t* gate, int64_t n_gate,
                                           uint16_t* h_sel, int64_t K, int64_t group_size, int64_t num_groups,
                                           void* stream) {
    const char* what = "soi_gemv_w4a16_indexed_silu";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1 && num_rows >= 0 && n_gate >= 0 &&
                    n_gate <= (int64_t(1) << 31) - 1,
                "%s: size out of range", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && idx && x && gate && h_sel, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(Wq) && aligned16(x);
    IndexRows rows{Wq, scale, num_rows, idx, row_bytes, num_groups};
    return launch_int4<true>(rows, k, x, SiluIdxY{h_sel, gate, idx, static_cast<int>(n_gate)}, K, group_size, vec,
                             as_stream(stream), what);
}

static int check_cached(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows, const uint8_t* full_Wq,
                        const float* full_scale, int64_t num_channels, const int32_t* slot_of, const int32_t* sel,
                        int64_t k, const char* what) {
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1, "%s: k out of range", what);
    SOI_REQUIRE(cache_rows >= 0 && num_channels >= 0 && num_channels <= (int64_t(1) << 31) - 1,
                "%s: negative or too large row / channel count", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(num_channels >= 1, "%s: a selection needs at least one channel", what);
    SOI_REQUIRE(sel && slot_of && full_Wq && full_scale, "%s: null pointer", what);
    SOI_REQUIRE(cache_rows == 0 || (cache_Wq && cache_scale), "%s: null cache", what);
    return SOI_OK;
}

extern "C" int soi_gemv_dip_cached_up(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                      const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                                      const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* x,
                                      uint16_t* y, int64_t K, int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_dip_cached_up";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    st = check_cached(cache_Wq, cache_scale, cache_rows, full_Wq, full_scale, num_channels, slot_of, sel, k, what);
    if (st || k == 0) return st;
    SOI_REQUIRE(x && y, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(x) && aligned16(full_Wq) && (cache_rows == 0 || aligned16(cache_Wq));
    SlotRows rows{cache_Wq, cache_scale, cache_rows, full_Wq, full_scale, num_channels, sel, slot_of, row_bytes,
                  num_groups};
    return launch_int4<true>(rows, k, x, StoreY{y}, K, group_size, vec, as_stream(stream), what);
}

extern "C" int soi_gemv_dip_cached_up_silu(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                           const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                                           const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* x,
                                           const uint16_t* gate, uint16_t* h_sel, int64_t K, int64_t group_size,
                                           int64_t num_groups, const uint8_t* copy_src, int64_t copy_row_bytes,
                                           uint8_t* copy_dst, void* stream) {
    const char* what = "soi_gemv_dip_cached_up_silu";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    st = check_cached(cache_Wq, cache_scale, cache_rows, full_Wq, full_scale, num_channels, slot_of, sel, k, what);
    if (st || k == 0) return st;
    SOI_REQUIRE(x && gate && h_sel, "%s: null pointer", what);
    SOI_REQUIRE((copy_src == nullptr) == (copy_dst == nullptr), "%s: copy_src and copy_dst go together", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && aligned16(x) && aligned16(full_Wq) && (cache_rows == 0 || aligned16(cache_Wq));
    SlotRows rows{cache_Wq, cache_scale, cache_rows, full_Wq, full_scale, num_channels, sel, slot_of, row_bytes,
                  num_groups};
    const SiluIdxY ep{h_sel, gate, sel, static_cast<int>(num_channels)};
    hipStream_t s = as_stream(stream);
    if (!copy_src) return launch_int4<true>(rows, k, x, ep, K, group_size, vec, s, what);
    SOI_REQUIRE(copy_row_bytes > 0 && copy_row_bytes % 16 == 0 && copy_row_bytes <= 4096 && aligned16(copy_src) &&
                    aligned16(copy_dst),
                "%s: copied rows must be 16-byte aligned, a multiple of 16 bytes and at most 4096 bytes", what);
    if (copy_row_bytes <= 1024)
        return launch_int4<true>(rows, k, x, ep, K, group_size, vec, s, what,
                                 MissCopy<1>{sel, slot_of, num_channels, copy_src, copy_dst, copy_row_bytes});
    if (copy_row_bytes <= 2048)
        return launch_int4<true>(rows, k, x, ep, K, group_size, vec, s, what,
                                 MissCopy<2>{sel, slot_of, num_channels, copy_src, copy_dst, copy_row_bytes});
    return launch_int4<true>(rows, k, x, ep, K, group_size, vec, s, what,
                             MissCopy<4>{sel, slot_of, num_channels, copy_src, copy_dst, copy_row_bytes});
}

extern "C" int soi_gemv_dip_fused_up_silu(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                          const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                                          const int32_t* desc, const int32_t* sel, int64_t k, const uint16_t* x,
                                          const uint16_t* gate, int64_t n_gate, uint16_t* h_sel, int64_t K,
                                          int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_dip_fused_up_silu";
    int st = check_int4_common(K, group_size, num_groups, what);
    if (st) return st;
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1 && n_gate >= 0 && n_gate <= (int64_t(1) << 31) - 1,
                "%s: size out of range", what);
    SOI_REQUIRE(cache_rows >= 0 && staging_rows >= 0, "%s: negative row count", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(desc && sel && x && gate && h_sel, "%s: null pointer", what);
    SOI_REQUIRE((cache_rows == 0 || (cache_Wq && cache_scale)) && (staging_rows == 0 || (staging_Wq && staging_scale)),
                "%s: null row source", what);
    const int64_t row_bytes = ceil_div64(K, 8) * 4;
    const bool vec = (K % 32 == 0) && (cache_rows == 0 || aligned16(cache_Wq)) &&
                     (staging_rows == 0 || aligned16(staging_Wq)) && aligned16(x);
    DescRows rows{cache_Wq, cache_scale, cache_rows, staging_Wq, staging_scale, staging_rows, desc, row_bytes,
                  num_groups};
    return launch_int4<true>(rows, k, x, SiluIdxY{h_sel, gate, sel, static_cast<int>(n_gate)}, K, group_size, vec,
                             as_stream(stream), what);
}
