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
#include "soi_rows.h"

namespace soi {

template <bool VEC>
__device__ __forceinline__ void load_x_chunk(const uint16_t* __restrict__ x, int K, int k0, f16x2 xv[16]) {
    if (VEC && k0 + 32 <= K) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(x + k0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 t = xp[i];
            xv[4 * i + 0] = as_f16x2(t.x);
            xv[4 * i + 1] = as_f16x2(t.y);
            xv[4 * i + 2] = as_f16x2(t.z);
            xv[4 * i + 3] = as_f16x2(t.w);
        }
    } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int ka = k0 + 2 * e, kb = ka + 1;
            const uint32_t lo = (ka < K) ? x[ka] : 0u;
            const uint32_t hi = (kb < K) ? x[kb] : 0u;
            xv[e] = as_f16x2(lo | (hi << 16));
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void load_w_chunk(const uint8_t* __restrict__ row, int words, int c, uint32_t wv[4]) {
    if (VEC) {
        const u32x4 t = reinterpret_cast<const u32x4*>(row)[c];
        wv[0] = t.x;
        wv[1] = t.y;
        wv[2] = t.z;
        wv[3] = t.w;
    } else {
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int wi = 4 * c + i;
            wv[i] = (wi < words) ? rw[wi] : 0u;
        }
    }
}

template <bool BITFIELD>
__device__ __forceinline__ void dequant8(uint32_t w, f16x2 q[4]) {
    if (BITFIELD)
        dequant_int4x8_bitfield(w, q);
    else
        dequant_int4x8_scalar(w, q);
}

template <int R, bool VEC, bool CHUNK_SCALE, bool BITFIELD, class Rows>
__global__ __launch_bounds__(64) void gemv_int4_kernel(Rows rows, int64_t N, const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, int K, int gs) {
    const int lane = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
    const int words = (K + 7) >> 3;
    const int chunks = (words + 3) >> 2;

    RowRef ref[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ref[r] = (row0 + r < N) ? rows.get(row0 + r) : RowRef{nullptr, nullptr, false};

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int c0 = 0; c0 < chunks; c0 += kWave) {
        const int c = c0 + lane;
        if (c < chunks) {
            uint32_t wv[R][4];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (ref[r].ok) {
                    load_w_chunk<VEC>(ref[r].w, words, c, wv[r]);
                } else {
                    wv[r][0] = wv[r][1] = wv[r][2] = wv[r][3] = 0u;
                }
            }
            const int k0 = 32 * c;
            float sc[R][CHUNK_SCALE ? 1 : 4];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (CHUNK_SCALE) {
                    sc[r][0] = ref[r].ok ? ref[r].s[k0 / gs] : 0.0f;
                } else {
#pragma unroll
                    for (int i = 0; i < (CHUNK_SCALE ? 1 : 4); ++i) {
                        const int wi = 4 * c + i;
                        sc[r][i] = (ref[r].ok && wi < words) ? ref[r].s[(8 * wi) / gs] : 0.0f;
                    }
                }
            }
            f16x2 xv[16];
            load_x_chunk<VEC>(x, K, k0, xv);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (CHUNK_SCALE) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        f16x2 q[4];
                        dequant8<BITFIELD>(wv[r][i], q);
#pragma unroll
                        for (int p = 0; p < 4; ++p) t = dot2(q[p], xv[4 * i + p], t);
                    }
                    acc[r] = fmaf(sc[r][0], t, acc[r]);
                } else {
#pragma unroll
                    for (int i = 0; i < (CHUNK_SCALE ? 1 : 4); ++i) {
                        f16x2 q[4];
                        dequant8<BITFIELD>(wv[r][i], q);
                        float t = 0.0f;
#pragma unroll
                        for (int p = 0; p < 4; ++p) t = dot2(q[p], xv[4 * i + p], t);
                        acc[r] = fmaf(sc[r][i], t, acc[r]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float total = wave_sum_lane63(acc[r]);
        if (lane == 63 && row0 + r < N) y[row0 + r] = ref[r].ok ? f32_to_f16_bits(total) : uint16_t(0x7e00u);
    }
}

// ---------------------------------------------------------------------------
// host dispatch
// ---------------------------------------------------------------------------

// Rows per wave: keep >= ~1024 waves in flight (4 per CU on 256 CUs) while
// giving each wave as many independent 1 KB row loads as that allows.
static int pick_rows_per_wave(int64_t N) {
    if (N >= 8 * 1024) return 8;
    if (N >= 4 * 1024) return 4;
    if (N >= 2 * 1024) return 2;
    return 1;
}

template <bool BITFIELD, class Rows>
static int launch_int4(const Rows& rows, int64_t N, const uint16_t* x, uint16_t* y, int64_t K, int64_t gs, bool vec,
                       hipStream_t st, const char* what) {
    if (N == 0) return SOI_OK;
    const int R = pick_rows_per_wave(N);
    const bool chunk_scale = (gs % 32) == 0;
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, R)));
    const int Ki = static_cast<int>(K), gi = static_cast<int>(gs);
#define SOI_L(RR, V, CS) \
    hipLaunchKernelGGL((gemv_int4_kernel<RR, V, CS, BITFIELD, Rows>), grid, dim3(64), 0, st, rows, N, x, y, Ki, gi)
#define SOI_LR(V, CS)          \
    switch (R) {               \
        case 8: SOI_L(8, V, CS); break; \
        case 4: SOI_L(4, V, CS); break; \
        case 2: SOI_L(2, V, CS); break; \
        default: SOI_L(1, V, CS); break; \
    }
    if (vec) {
        if (chunk_scale) { SOI_LR(true, true) } else { SOI_LR(true, false) }
    } else {
        if (chunk_scale) { SOI_LR(false, true) } else { SOI_LR(false, false) }
    }
#undef SOI_LR
#undef SOI_L
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
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq) && aligned16(x);
    DenseRows rows{Wq, scale, row_bytes, G};
    return launch_int4<BITFIELD>(rows, N, x, y, K, gs, vec, as_stream(stream), what);
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
    const bool vec = (row_bytes % 16 == 0) && aligned16(x) && (cache_rows == 0 || aligned16(cache_Wq)) &&
                     (staging_rows == 0 || aligned16(staging_Wq));
    DescRows rows{cache_Wq, cache_scale, cache_rows, staging_Wq, staging_scale, staging_rows, desc, row_bytes,
                  num_groups};
    return launch_int4<true>(rows, k, x, y, K, group_size, vec, as_stream(stream), what);
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
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq) && aligned16(x);
    IndexRows rows{Wq, scale, num_rows, idx, row_bytes, num_groups};
    return launch_int4<true>(rows, k, x, y, K, group_size, vec, as_stream(stream), what);
}
