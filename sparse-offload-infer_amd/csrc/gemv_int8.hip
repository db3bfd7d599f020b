// INT8 GEMV for batch-1 decode on gfx950.
//
// Restates the reference's gemv_w8a16 (csrc/kernels/gemv_w8a16.cu:22-62):
// y[n] = sum_k s[n*stride + k/gs] * q[n,k] * x[k], stride 0 = per-tensor
// scale, fp32 accumulation, binary16 output.
//
// One wave per workgroup, R rows per wave. Lane l owns 16-byte chunk l of each
// 64-chunk pass (16 consecutive k), so a wave-wide dwordx4 load reads 1 KB of
// a row. Bytes become exact binary16 integers (soi_device.h), pairs are
// accumulated with an ordered v_dot2 chain, and the scale is applied once per
// chunk (per word when 16 does not divide group_size).
//
// One deliberate difference: with num_groups == 1 every element uses the
// row's single scale. The reference indexes scale[row*stride + k/gs] even
// then, which reads past a [N,1] scale when the caller passes gs < K.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

template <int R, bool VEC, bool CHUNK_SCALE>
__global__ __launch_bounds__(64) void gemv_int8_kernel(const int8_t* __restrict__ W, const float* __restrict__ S,
                                                       int64_t srow_stride, int64_t N, const uint16_t* __restrict__ x,
                                                       uint16_t* __restrict__ y, int K, int gs, int G) {
    const int lane = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
    const int chunks = (K + 15) >> 4;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    for (int c0 = 0; c0 < chunks; c0 += kWave) {
        const int c = c0 + lane;
        if (c >= chunks) continue;
        const int k0 = 16 * c;
        uint32_t wv[R][4];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t n = row0 + r;
            const int8_t* row = W + (n < N ? n : 0) * static_cast<int64_t>(K);
            if (n >= N) {
                wv[r][0] = wv[r][1] = wv[r][2] = wv[r][3] = 0u;
            } else if (VEC) {
                const u32x4 t = reinterpret_cast<const u32x4*>(row)[c];
                wv[r][0] = t.x;
                wv[r][1] = t.y;
                wv[r][2] = t.z;
                wv[r][3] = t.w;
            } else {
                const uint8_t* rb = reinterpret_cast<const uint8_t*>(row);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t word = 0;
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const int kk = k0 + 4 * i + b;
                        // padding bytes read as 0x00 -> value 0; x there is 0 too
                        word |= (kk < K ? static_cast<uint32_t>(rb[kk]) : 0u) << (8 * b);
                    }
                    wv[r][i] = word;
                }
            }
        }
        float sc[R][CHUNK_SCALE ? 1 : 4];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t n = row0 + r;
            const float* srow = S + (n < N ? n : 0) * srow_stride;
            if (CHUNK_SCALE) {
                sc[r][0] = (n < N) ? srow[G == 1 ? 0 : k0 / gs] : 0.0f;
            } else {
#pragma unroll
                for (int i = 0; i < (CHUNK_SCALE ? 1 : 4); ++i) {
                    const int kk = k0 + 4 * i;
                    sc[r][i] = (n < N && kk < K) ? srow[kk / gs] : 0.0f;
                }
            }
        }
        f16x2 xv[8];
        if (VEC && k0 + 16 <= K) {
            const u32x4* xp = reinterpret_cast<const u32x4*>(x + k0);
            const u32x4 a = xp[0], b = xp[1];
            xv[0] = as_f16x2(a.x);
            xv[1] = as_f16x2(a.y);
            xv[2] = as_f16x2(a.z);
            xv[3] = as_f16x2(a.w);
            xv[4] = as_f16x2(b.x);
            xv[5] = as_f16x2(b.y);
            xv[6] = as_f16x2(b.z);
            xv[7] = as_f16x2(b.w);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int ka = k0 + 2 * e, kb = ka + 1;
                const uint32_t lo = (ka < K) ? x[ka] : 0u;
                const uint32_t hi = (kb < K) ? x[kb] : 0u;
                xv[e] = as_f16x2(lo | (hi << 16));
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (CHUNK_SCALE) {
                float t = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f16x2 q[2];
                    dequant_int8x4(wv[r][i], q);
                    t = dot2(q[0], xv[2 * i], t);
                    t = dot2(q[1], xv[2 * i + 1], t);
                }
                acc[r] = fmaf(sc[r][0], t, acc[r]);
            } else {
#pragma unroll
                for (int i = 0; i < (CHUNK_SCALE ? 1 : 4); ++i) {
                    f16x2 q[2];
                    dequant_int8x4(wv[r][i], q);
                    float t = dot2(q[0], xv[2 * i], 0.0f);
                    t = dot2(q[1], xv[2 * i + 1], t);
                    acc[r] = fmaf(sc[r][i], t, acc[r]);
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float total = wave_sum_lane63(acc[r]);
        if (lane == 63 && row0 + r < N) y[row0 + r] = f32_to_f16_bits(total);
    }
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
    const int R = N >= 4096 ? 4 : (N >= 2048 ? 2 : 1);
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, R)));
    hipStream_t st = as_stream(stream);
    const int Ki = static_cast<int>(K), gi = static_cast<int>(group_size), Gi = static_cast<int>(num_groups);
#define SOI_L(RR, V, CS)                                                                                          \
    hipLaunchKernelGGL((gemv_int8_kernel<RR, V, CS>), grid, dim3(64), 0, st, Wq, scale, scale_row_stride, N, x, y, \
                       Ki, gi, Gi)
#define SOI_LR(V, CS)                    \
    switch (R) {                         \
        case 4: SOI_L(4, V, CS); break;  \
        case 2: SOI_L(2, V, CS); break;  \
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
