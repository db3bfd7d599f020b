// INT8 GEMV for batch-1 decode on gfx950.
//
// Restates the reference's gemv_w8a16 (csrc/kernels/gemv_w8a16.cu:22-62):
// y[n] = sum_k s[n*stride + k/gs] * q[n,k] * x[k], stride 0 = per-tensor
// scale, fp32 accumulation, binary16 output.
//
// One wave per workgroup, R rows per wave, PU 64-chunk passes per batch.
// Lane l owns 16-byte chunk l of each pass (16 consecutive k), so a wave-wide
// dwordx4 load reads 1 KB of a row; R*PU such loads are issued before any
// arithmetic. Loads are unconditional: a lane past the last chunk (or any
// byte past K) reads the zero word instead (address select, no branch), and
// row addresses are wave-uniform (scalar registers). Bytes become exact
// binary16 integers (soi_device.h), pairs are accumulated with an ordered
// v_dot2 chain, the scale is applied once per chunk (per word when 16 does
// not divide group_size), and the R row totals come out of one transposed
// wave reduction with a fixed order of additions.
//
// One deliberate difference: with num_groups == 1 every element uses the
// row's single scale. The reference indexes scale[row*stride + k/gs] even
// then, which reads past a [N,1] scale when the caller passes gs < K.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

// Rows row0 .. row0 + R - 1 of one problem, by the calling wave (the single and batched kernels share it, so a
// batched problem's y is bit-identical to the single launch's).
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__device__ __forceinline__ void gemv_int8_rows(const int8_t* __restrict__ W, const float* __restrict__ S,
                                               int64_t srow_stride, int64_t N, const uint16_t* __restrict__ x,
                                               uint16_t* __restrict__ y, int K, int gs, int G, int64_t row0) {
    constexpr int SC = CHUNK_SCALE ? 1 : 4;
    const int lane = threadIdx.x;
    const int chunks = (K + 15) >> 4;
    const uint32_t* zw = g_zero16;
    const float* zf = reinterpret_cast<const float*>(g_zero16);

    // rows past N read row N-1 (never stored)
    const uint8_t* wr[R];
    const float* sr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t n = (FULL || row0 + r < N) ? row0 + r : N - 1;
        wr[r] = uniform_ptr(reinterpret_cast<const uint8_t*>(W) + n * static_cast<int64_t>(K));
        sr[r] = uniform_ptr(S + n * srow_stride);
    }

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int c0 = 0; c0 < chunks; c0 += kWave * PU) {
        uint32_t wv[PU][R][4];
        float sc[PU][R][SC];
        f16x2 xv[PU][8];
#pragma unroll
        for (int p = 0; p < PU; ++p) {
            const int c = c0 + p * kWave + lane;
            const bool cv = FULL || c < chunks;
            const int k0 = 16 * c;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (VEC) {
                    const u32x4* q = reinterpret_cast<const u32x4*>(wr[r]) + c;
                    const u32x4 t = ldg_stream(cv ? q : reinterpret_cast<const u32x4*>(zw));
                    wv[p][r][0] = t.x;
                    wv[p][r][1] = t.y;
                    wv[p][r][2] = t.z;
                    wv[p][r][3] = t.w;
                } else {
                    // ragged K: bytes past K read as 0x00 -> value 0 (x there is 0 too)
                    const uint8_t* zb = reinterpret_cast<const uint8_t*>(zw);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        uint32_t word = 0;
#pragma unroll
                        for (int b = 0; b < 4; ++b) {
                            const int kk = k0 + 4 * i + b;
                            word |= static_cast<uint32_t>(ldg((cv && kk < K) ? wr[r] + kk : zb)) << (8 * b);
                        }
                        wv[p][r][i] = word;
                    }
                }
                if (CHUNK_SCALE) {
                    sc[p][r][0] = ldg(cv ? sr[r] + (G == 1 ? 0 : k0 / gs) : zf);
                } else {
#pragma unroll
                    for (int i = 0; i < SC; ++i) {
                        const int kk = k0 + 4 * i;
                        sc[p][r][i] = ldg((cv && kk < K) ? sr[r] + kk / gs : zf);
                    }
                }
            }
            if (VEC) {  // K % 16 == 0: a valid chunk is fully inside x
                const u32x4* xp = reinterpret_cast<const u32x4*>(x + k0);
                const u32x4* z4 = reinterpret_cast<const u32x4*>(zw);
                const u32x4 a = ldg(cv ? xp : z4), b = ldg(cv ? xp + 1 : z4);
                xv[p][0] = as_f16x2(a.x);
                xv[p][1] = as_f16x2(a.y);
                xv[p][2] = as_f16x2(a.z);
                xv[p][3] = as_f16x2(a.w);
                xv[p][4] = as_f16x2(b.x);
                xv[p][5] = as_f16x2(b.y);
                xv[p][6] = as_f16x2(b.z);
                xv[p][7] = as_f16x2(b.w);
            } else {
                const uint16_t* zh = reinterpret_cast<const uint16_t*>(zw);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int ka = k0 + 2 * e, kb = ka + 1;
                    const uint32_t lo = ldg((cv && ka < K) ? x + ka : zh);
                    const uint32_t hi = ldg((cv && kb < K) ? x + kb : zh);
                    xv[p][e] = as_f16x2(lo | (hi << 16));
                }
            }
        }
#pragma unroll
        for (int p = 0; p < PU; ++p) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (CHUNK_SCALE) {
                    float t = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        f16x2 q[2];
                        dequant_int8x4(wv[p][r][i], q);
                        t = dot2(q[0], xv[p][2 * i], t);
                        t = dot2(q[1], xv[p][2 * i + 1], t);
                    }
                    acc[r] = fmaf(sc[p][r][0], t, acc[r]);
                } else {
#pragma unroll
                    for (int i = 0; i < SC; ++i) {
                        f16x2 q[2];
                        dequant_int8x4(wv[p][r][i], q);
                        float t = dot2(q[0], xv[p][2 * i], 0.0f);
                        t = dot2(q[1], xv[p][2 * i + 1], t);
                        acc[r] = fmaf(sc[p][r][i], t, acc[r]);
                    }
                }
            }
        }
    }

    const float total = reduce_rows<R>(acc);
    const int r = reduce_rows_row<R>(static_cast<uint32_t>(lane));
    if ((lane & (64 / R - 1)) == 0 && (FULL || row0 + r < N)) stg(y + row0 + r, f32_to_f16_bits(total));
}

template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) void gemv_int8_kernel(const int8_t* __restrict__ W, const float* __restrict__ S,
                                                       int64_t srow_stride, int64_t N, const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, int K, int gs, int G) {
    gemv_int8_rows<R, PU, VEC, CHUNK_SCALE, FULL>(W, S, srow_stride, N, x, y, K, gs, G,
                                                  static_cast<int64_t>(blockIdx.x) * R);
}

// Batched form: P problems of one shape; workgroup b takes row tile b % tiles of problem b / tiles. The pointer
// tables live in device memory; a problem with a null pointer writes nothing, and (VEC) one whose W or x is not
// 16-byte aligned gets NaN rows instead of being read with dwordx4 loads.
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) void gemv_int8_batched_kernel(const int8_t* const* __restrict__ Wp,
                                                               const float* const* __restrict__ Sp,
                                                               const uint16_t* const* __restrict__ Xp,
                                                               uint16_t* const* __restrict__ Yp, int64_t srow_stride,
                                                               int64_t N, int K, int gs, int G, int tiles) {
    const int b = static_cast<int>(blockIdx.x);
    const int p = b / tiles;
    const int64_t row0 = static_cast<int64_t>(b - p * tiles) * R;
    const int8_t* W = ldg(Wp + p);
    const float* S = ldg(Sp + p);
    const uint16_t* x = ldg(Xp + p);
    uint16_t* y = ldg(Yp + p);
    if (!W || !S || !x || !y) return;
    if (VEC && ((reinterpret_cast<uintptr_t>(W) | reinterpret_cast<uintptr_t>(x)) & 15u)) {
        const int64_t r = row0 + static_cast<int64_t>(threadIdx.x);
        if (threadIdx.x < R && r < N) stg(y + r, static_cast<uint16_t>(0x7e00u));
        return;
    }
    gemv_int8_rows<R, PU, VEC, CHUNK_SCALE, FULL>(W, S, srow_stride, N, x, y, K, gs, G, row0);
}

struct Int8Plan {
    int R, PU;
};

// PU: passes per batch, the largest of 4, 3, 2 that divides the pass count
// (all of them when there are fewer than 4); R: the most rows per wave with
// R*PU <= 8 1 KB row segments in flight that still leaves >= 2048 waves in the
// grid (swept on the Qwen3-1.7B shapes: more waves beat more rows per wave).
static Int8Plan plan_int8(int64_t N, int64_t K, bool vec) {
    const int64_t passes = ceil_div64(ceil_div64(K, 16), kWave);
    Int8Plan p{1, 1};
    if (vec) {
        if (passes <= 4) p.PU = static_cast<int>(passes);
        else if (passes % 4 == 0) p.PU = 4;
        else if (passes % 3 == 0) p.PU = 3;
        else if (passes % 2 == 0) p.PU = 2;
        else p.PU = 4;
    }
    int R = 8;
    while (R > 1 && (R * p.PU > 8 || N / R < 2048)) R >>= 1;
    p.R = R;
    return p;
}

}  // namespace soi

using namespace soi;

static int check_int8(int64_t N, int64_t K, int64_t group_size, int64_t num_groups, int64_t scale_row_stride,
                      const char* what) {
    SOI_REQUIRE(K >= 1 && K <= (int64_t(1) << 30), "%s: K must be in [1, 2^30]", what);
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    SOI_REQUIRE(group_size >= 1, "%s: group_size must be >= 1", what);
    SOI_REQUIRE(num_groups == 1 || group_size % 4 == 0,
                "%s: group_size must be a multiple of 4 when num_groups > 1", what);
    SOI_REQUIRE(num_groups == 1 || num_groups == ceil_div64(K, group_size),
                "%s: num_groups must be 1 or ceil(K/group_size) = %lld, got %lld", what,
                (long long)ceil_div64(K, group_size), (long long)num_groups);
    SOI_REQUIRE(scale_row_stride == 0 || scale_row_stride == num_groups,
                "%s: scale_row_stride must be 0 (per-tensor) or num_groups", what);
    return SOI_OK;
}

// Picks the instantiation (R, PU, VEC, CHUNK_SCALE, FULL) of the plan and calls launch.go<...>() with it; the
// launcher (SingleInt8Launch or BatchedInt8Launch) holds the arguments of its kernel form.
template <class Launch>
static void dispatch_int8(const Int8Plan& pl, bool vec, bool full, bool chunk_scale, Launch&& launch) {
#define SOI_L(RR, PP, V, CS, FL) launch.template go<RR, PP, V, CS, FL>()
#define SOI_CS(RR, PP, V)                                     \
    if (V && full && chunk_scale) SOI_L(RR, PP, V, true, true); \
    else if (chunk_scale) SOI_L(RR, PP, V, true, false);        \
    else SOI_L(RR, PP, V, false, false)
    if (vec) {
        switch (pl.R * 10 + pl.PU) {
            case 81: SOI_CS(8, 1, true); break;
            case 41: SOI_CS(4, 1, true); break;
            case 21: SOI_CS(2, 1, true); break;
            case 11: SOI_CS(1, 1, true); break;
            case 42: SOI_CS(4, 2, true); break;
            case 22: SOI_CS(2, 2, true); break;
            case 12: SOI_CS(1, 2, true); break;
            case 23: SOI_CS(2, 3, true); break;
            case 13: SOI_CS(1, 3, true); break;
            case 24: SOI_CS(2, 4, true); break;
            default: SOI_CS(1, 4, true); break;
        }
    } else {
        switch (pl.R) {
            case 8: SOI_CS(8, 1, false); break;
            case 4: SOI_CS(4, 1, false); break;
            case 2: SOI_CS(2, 1, false); break;
            default: SOI_CS(1, 1, false); break;
        }
    }
#undef SOI_CS
#undef SOI_L
}

struct SingleInt8Launch {
    dim3 grid;
    hipStream_t st;
    const int8_t* W;
    const float* S;
    int64_t stride, N;
    const uint16_t* x;
    uint16_t* y;
    int K, gs, G;
    template <int R, int PU, bool V, bool CS, bool FL>
    void go() const {
        hipLaunchKernelGGL((gemv_int8_kernel<R, PU, V, CS, FL>), grid, dim3(64), 0, st, W, S, stride, N, x, y, K, gs,
                           G);
    }
};

struct BatchedInt8Launch {
    int64_t P;
    hipStream_t st;
    const int8_t* const* Wp;
    const float* const* Sp;
    const uint16_t* const* Xp;
    uint16_t* const* Yp;
    int64_t stride, N;
    int K, gs, G;
    template <int R, int PU, bool V, bool CS, bool FL>
    void go() const {
        const int tiles = static_cast<int>(ceil_div64(N, R));
        const dim3 grid(static_cast<unsigned>(P * tiles));
        hipLaunchKernelGGL((gemv_int8_batched_kernel<R, PU, V, CS, FL>), grid, dim3(64), 0, st, Wp, Sp, Xp, Yp, stride,
                           N, K, gs, G, tiles);
    }
};

extern "C" int soi_gemv_w8a16(const int8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N,
                              int64_t K, int64_t group_size, int64_t num_groups, int64_t scale_row_stride,
                              void* stream) {
    const char* what = "soi_gemv_w8a16";
    int s = check_int8(N, K, group_size, num_groups, scale_row_stride, what);
    if (s) return s;
    if (N == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && x && y, "%s: null pointer", what);
    const bool vec = (K % 16 == 0) && aligned16(Wq) && aligned16(x);
    const bool chunk_scale = (num_groups == 1) || (group_size % 16 == 0);
    const Int8Plan pl = plan_int8(N, K, vec);
    const bool full = vec && (N % pl.R == 0) && ((K / 16) % (kWave * pl.PU) == 0);
    SingleInt8Launch L{dim3(static_cast<unsigned>(ceil_div64(N, pl.R))), as_stream(stream), Wq, scale,
                       scale_row_stride, N, x, y, static_cast<int>(K), static_cast<int>(group_size),
                       static_cast<int>(num_groups)};
    dispatch_int8(pl, vec, full, chunk_scale, L);
    return launch_status(what);
}

extern "C" int soi_gemv_w8a16_batched(const int8_t* const* Wq_ptrs, const float* const* scale_ptrs,
                                      const uint16_t* const* x_ptrs, uint16_t* const* y_ptrs, int64_t P, int64_t N,
                                      int64_t K, int64_t group_size, int64_t num_groups, int64_t scale_row_stride,
                                      void* stream) {
    const char* what = "soi_gemv_w8a16_batched";
    int s = check_int8(N, K, group_size, num_groups, scale_row_stride, what);
    if (s) return s;
    SOI_REQUIRE(P >= 0 && P <= (int64_t(1) << 20), "%s: P out of range", what);
    if (N == 0 || P == 0) return SOI_OK;
    SOI_REQUIRE(Wq_ptrs && scale_ptrs && x_ptrs && y_ptrs, "%s: null pointer table", what);
    // the single form's passes per batch for this shape (with aligned operands)
    const bool vec = K % 16 == 0;
    const bool chunk_scale = (num_groups == 1) || (group_size % 16 == 0);
    Int8Plan pl = plan_int8(N, K, vec);
    // several problems fill the grid whatever the tile, so the tile takes the most rows its pass count allows
    // (8 / 4 / 2 rows at 1 / 2 / 3-4 passes, rows dividing N); a row's arithmetic does not depend on the tile, so
    // y still equals the single launch's bit for bit. Qwen3-1.7B classes, back to back: down 71.5 -> 61.7 us,
    // gate/up 132.4 -> 121.2, q/o 45.6 -> 41.7, k/v 25.7 -> 23.2 (28 / 56 problems)
    if (P > 1) {
        const int rmax = pl.PU == 1 ? 8 : pl.PU == 2 ? 4 : 2;
        while (pl.R < rmax && N % (2 * pl.R) == 0) pl.R *= 2;
    }
    const bool full = vec && (N % pl.R == 0) && ((K / 16) % (kWave * pl.PU) == 0);
    SOI_REQUIRE(P * ceil_div64(N, pl.R) <= (int64_t(1) << 31) - 1, "%s: grid too large", what);
    BatchedInt8Launch L{P, as_stream(stream), Wq_ptrs, scale_ptrs, x_ptrs, y_ptrs, scale_row_stride, N,
                        static_cast<int>(K), static_cast<int>(group_size), static_cast<int>(num_groups)};
    dispatch_int8(pl, vec, full, chunk_scale, L);
    return launch_status(what);
}
