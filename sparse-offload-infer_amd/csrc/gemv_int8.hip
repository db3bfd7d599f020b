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

template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool FULL>
__global__ __launch_bounds__(64) void gemv_int8_kernel(const int8_t* __restrict__ W, const float* __restrict__ S,
                                                       int64_t srow_stride, int64_t N, const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, int K, int gs, int G) {
    constexpr int SC = CHUNK_SCALE ? 1 : 4;
    const int lane = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
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

extern "C" int soi_gemv_w8a16(const int8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N,
                              int64_t K, int64_t group_size, int64_t num_groups, int64_t scale_row_stride,
                              void* stream) {
    const char* what = "soi_gemv_w8a16";
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
    if (N == 0) return SOI_OK;
    SOI_REQUIRE(Wq && scale && x && y, "%s: null pointer", what);
    const bool vec = (K % 16 == 0) && aligned16(Wq) && aligned16(x);
    const bool chunk_scale = (num_groups == 1) || (group_size % 16 == 0);
    const Int8Plan pl = plan_int8(N, K, vec);
    const bool full = vec && (N % pl.R == 0) && ((K / 16) % (kWave * pl.PU) == 0);
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, pl.R)));
    hipStream_t st = as_stream(stream);
    const int Ki = static_cast<int>(K), gi = static_cast<int>(group_size), Gi = static_cast<int>(num_groups);
#define SOI_L(RR, PP, V, CS, FL)                                                                                   \
    hipLaunchKernelGGL((gemv_int8_kernel<RR, PP, V, CS, FL>), grid, dim3(64), 0, st, Wq, scale, scale_row_stride, N, \
                       x, y, Ki, gi, Gi)
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
    return launch_status(what);
}
