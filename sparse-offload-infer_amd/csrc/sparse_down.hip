// Sparse down projection over selected rows of down_proj^T (gfx950).
//
// Restates csrc/kernels/gemv_sparse_accumulate.cu:10-38 and the descriptor
// form gemv_dip_fused.cu:116-154:
//   y[c] = sum_{j<k} (h_j * s[j, c/gs]) * q[j, c],  fp32 accumulation, fp16 out.
// The reference runs one thread per output column over all k rows, which
// touches 4 bytes per row per thread and uses a handful of CUs. Here:
//   pass 1 (partial): workgroup g owns rows [g*R, (g+1)*R) (R chosen so that
//     k rows spread over ~256 workgroups); its 4 waves take blocks of U = 4
//     rows in turn; lane l owns a 16-byte chunk (32 consecutive columns) of a
//     2048-column slab, so each row is read as one coalesced 1 KB wave load.
//     Each lane keeps 32 fp32 sums; per row: coef = fl(h_j*s),
//     acc_c = fma(coef, q_c, acc_c) with q_c an exact binary16 integer
//     (v_fma_mix_f32). The waves are summed in LDS in wave order and the
//     workgroup's partial row is written to the workspace.
//   pass 2 (reduce): y[c] = fp16(sum over g of partial[g,c]): 8 interleaved
//     groups of g per column, each summed in ascending g with its loads
//     issued 8 at a time, then the 8 group sums in a fixed order.
// Fixed partition and fixed order: deterministic, and every row source
// (gathered rows, hot cache + staging descriptors, resident index list) gives
// bit-identical results for the same logical rows.
#include "soi_device.h"
#include "soi_host.h"
#include "soi_rows.h"

namespace soi {

constexpr int kDownWaves = 4;
constexpr int kDownThreads = kDownWaves * kWave;
constexpr int kSlabCols = kWave * 32;  // columns covered by one wave-wide row load
constexpr int kRedPad = kWave + 1;      // LDS row pitch (floats) for the wave-sum transpose

// U rows per wave per batch, all loads of a batch issued before arithmetic
// (a lane with no chunk or a row past the range reads g_zero16 instead).
template <int U, bool VEC, bool CHUNK_SCALE, class Rows>
__global__ __launch_bounds__(kDownThreads) void sparse_down_partial_kernel(Rows rows, const uint16_t* __restrict__ h,
                                                                            float* __restrict__ partial, int64_t k,
                                                                            int H, int gs, int rows_per_wg) {
    constexpr int SC = CHUNK_SCALE ? 1 : 4;
    __shared__ float red[kDownWaves * 32 * kRedPad];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int words = (H + 7) >> 3;
    const int chunks = (words + 3) >> 2;
    const int c = blockIdx.y * kWave + lane;
    const bool cvalid = c < chunks;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * rows_per_wg;
    const int64_t j1 = (j0 + rows_per_wg < k) ? j0 + rows_per_wg : k;
    const uint32_t* z = g_zero16;
    const float* zf = reinterpret_cast<const float*>(g_zero16);

    float acc[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) acc[i] = 0.0f;

    for (int64_t jb = j0 + static_cast<int64_t>(wave) * U; jb < j1; jb += static_cast<int64_t>(kDownWaves) * U) {
        uint32_t wv[U][4];
        float coef[U][SC];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t j = jb + u;
            const bool in = j < j1;
            const RowRef ref = rows.get(in ? j : j0);
            const bool ok = in && ref.ok && cvalid;
            const float hj = in ? f16_bits_to_f32(h[in ? j : j0]) : 0.0f;
            if (VEC) {
                const u32x4 t = __builtin_nontemporal_load(ok ? reinterpret_cast<const u32x4*>(ref.w) + c
                                                              : reinterpret_cast<const u32x4*>(z));
                wv[u][0] = t.x;
                wv[u][1] = t.y;
                wv[u][2] = t.z;
                wv[u][3] = t.w;
            } else {
                const uint32_t* rw = reinterpret_cast<const uint32_t*>(ref.w);
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[u][i] = *((ok && 4 * c + i < words) ? rw + 4 * c + i : z);
            }
            const float bad = (in && !ref.ok) ? __builtin_nanf("") : 1.0f;  // unresolvable row -> NaN
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                const int wi = 4 * c + i;
                const float sv = CHUNK_SCALE ? *(ok ? ref.s + (32 * c) / gs : zf)
                                             : *((ok && wi < words) ? ref.s + (8 * wi) / gs : zf);
                coef[u][i] = (hj * sv) * bad;
            }
        }
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

#pragma unroll
    for (int i = 0; i < 32; ++i) red[(wave * 32 + i) * kRedPad + lane] = acc[i];
    __syncthreads();
    // 2048 slab values, 4 per thread; value v -> (lane l = v/32, column-in-chunk i = v%32)
    const int64_t out_base = static_cast<int64_t>(blockIdx.x) * H + static_cast<int64_t>(blockIdx.y) * kSlabCols;
#pragma unroll
    for (int m = 0; m < (kSlabCols / kDownThreads); ++m) {
        const int v = threadIdx.x + m * kDownThreads;
        const int l = v >> 5, i = v & 31;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kDownWaves; ++w) s += red[(w * 32 + i) * kRedPad + l];
        const int col = blockIdx.y * kSlabCols + v;
        if (col < H) partial[out_base + v] = s;
    }
}

// Thread (c4, t): columns 4*c4..4*c4+3, partial rows g = t, t+8, t+16, ...;
// the 8 group sums are then added in t order through LDS. A fixed order for a
// given G: deterministic. G == 0 writes zeros (the empty sum).
constexpr int kRedGroups = 8;
constexpr int kRedCols = 128;  // columns per workgroup (32 threads x 4)

__global__ __launch_bounds__(256) void sparse_down_reduce_kernel(const float* __restrict__ partial, int G, int H,
                                                                  uint16_t* __restrict__ y, int vec_ok) {
    __shared__ f32x4 s_part[kRedGroups][kRedCols / 4];
    const int c4 = threadIdx.x & 31, t = threadIdx.x >> 5;
    const int col = blockIdx.x * kRedCols + 4 * c4;
    const bool vec = vec_ok != 0;  // H % 4 == 0 and a 16-byte aligned workspace
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    if (col < H) {
        int g = t;
        for (; g + 7 * kRedGroups < G; g += 8 * kRedGroups) {
            f32x4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const float* p = partial + static_cast<int64_t>(g + u * kRedGroups) * H + col;
                v[u] = vec ? ldg(reinterpret_cast<const f32x4*>(p))
                           : f32x4{ldg(p), col + 1 < H ? ldg(p + 1) : 0.0f, col + 2 < H ? ldg(p + 2) : 0.0f,
                                    col + 3 < H ? ldg(p + 3) : 0.0f};
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc.x += v[u].x;
                acc.y += v[u].y;
                acc.z += v[u].z;
                acc.w += v[u].w;
            }
        }
        for (; g < G; g += kRedGroups) {
            const float* p = partial + static_cast<int64_t>(g) * H + col;
            const f32x4 v = vec ? ldg(reinterpret_cast<const f32x4*>(p))
                                 : f32x4{ldg(p), col + 1 < H ? ldg(p + 1) : 0.0f, col + 2 < H ? ldg(p + 2) : 0.0f,
                                          col + 3 < H ? ldg(p + 3) : 0.0f};
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
    }
    s_part[t][c4] = acc;
    __syncthreads();
    if (t == 0 && col < H) {
        f32x4 s = s_part[0][c4];
#pragma unroll
        for (int u = 1; u < kRedGroups; ++u) {
            const f32x4 o = s_part[u][c4];
            s.x += o.x;
            s.y += o.y;
            s.z += o.z;
            s.w += o.w;
        }
        const float r[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (col + e < H) stg(y + col + e, f32_to_f16_bits(r[e]));
    }
}

// Rows per workgroup: a multiple of waves x U (one batch per wave at least),
// chosen to spread k rows over ~256 workgroups (one per CU).
constexpr int kDownU = 4;  // rows per wave per batch

static int64_t pick_rows_per_wg(int64_t k) {
    const int64_t step = static_cast<int64_t>(kDownWaves) * kDownU;
    int64_t r = ceil_div64(k, 256);
    if (r < step) r = step;
    return ceil_div64(r, step) * step;
}

static int64_t num_splits(int64_t k) { return k == 0 ? 0 : ceil_div64(k, pick_rows_per_wg(k)); }

template <class Rows>
static int launch_sparse_down(const Rows& rows, int64_t k, const uint16_t* h, uint16_t* y, int64_t H, int64_t gs,
                              bool vec, void* workspace, size_t ws_bytes, hipStream_t st, const char* what) {
    const int64_t G = num_splits(k);
    const size_t need = static_cast<size_t>(G) * static_cast<size_t>(H) * sizeof(float);
    if (k > 0) {
        if (!workspace || ws_bytes < need) {
            set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, ws_bytes);
            return SOI_ERR_WORKSPACE;
        }
        const int64_t rpw = pick_rows_per_wg(k);
        const dim3 grid(static_cast<unsigned>(G), static_cast<unsigned>(ceil_div64(H, kSlabCols)));
        float* partial = static_cast<float*>(workspace);
        const bool cs = (gs % 32) == 0;
        const int Hi = static_cast<int>(H), gi = static_cast<int>(gs), ri = static_cast<int>(rpw);
#define SOI_D(V, CS)                                                                                             \
    hipLaunchKernelGGL((sparse_down_partial_kernel<kDownU, V, CS, Rows>), grid, dim3(kDownThreads), 0, st, rows, h, partial, \
                       k, Hi, gi, ri)
        if (vec) {
            if (cs) SOI_D(true, true); else SOI_D(true, false);
        } else {
            if (cs) SOI_D(false, true); else SOI_D(false, false);
        }
#undef SOI_D
        int s = launch_status(what);
        if (s) return s;
        hipLaunchKernelGGL(sparse_down_reduce_kernel, dim3(static_cast<unsigned>(ceil_div64(H, kRedCols))), dim3(256), 0,
                           st, partial, static_cast<int>(G), Hi, y, (H % 4 == 0 && aligned16(partial)) ? 1 : 0);
        return launch_status(what);
    }
    // k == 0: y = 0 (empty sum), as the reference's loop yields; a fill kernel
    // rather than a memset so the call stays capturable in a HIP graph.
    hipLaunchKernelGGL(sparse_down_reduce_kernel, dim3(static_cast<unsigned>(ceil_div64(H, kRedCols))), dim3(256), 0, st,
                       static_cast<const float*>(nullptr), 0, static_cast<int>(H), y, 0);
    return launch_status(what);
}

static int check_down(int64_t H, int64_t k, int64_t gs, int64_t G, const char* what) {
    SOI_REQUIRE(H >= 1 && H <= (int64_t(1) << 30), "%s: H must be in [1, 2^30]", what);
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1, "%s: k out of range", what);
    SOI_REQUIRE(gs >= 1 && gs % 8 == 0, "%s: group_size must be a positive multiple of 8", what);
    SOI_REQUIRE(G == ceil_div64(H, gs), "%s: num_groups must be ceil(H/group_size) = %lld, got %lld", what,
                (long long)ceil_div64(H, gs), (long long)G);
    return SOI_OK;
}

}  // namespace soi

using namespace soi;

extern "C" size_t soi_sparse_accumulate_workspace_bytes(int64_t H, int64_t k) {
    if (H <= 0 || k <= 0) return 0;
    return static_cast<size_t>(num_splits(k)) * static_cast<size_t>(H) * sizeof(float);
}

extern "C" int soi_gemv_w4a16_sparse_accumulate(const uint8_t* Wq_sel, const float* scale_sel, const uint16_t* h_sel,
                                                uint16_t* y, int64_t H, int64_t k, int64_t group_size,
                                                int64_t num_groups, void* workspace, size_t workspace_bytes,
                                                void* stream) {
    const char* what = "soi_gemv_w4a16_sparse_accumulate";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(y && (k == 0 || (Wq_sel && scale_sel && h_sel)), "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq_sel);
    DenseRows rows{Wq_sel, scale_sel, row_bytes, num_groups};
    return launch_sparse_down(rows, k, h_sel, y, H, group_size, vec, workspace, workspace_bytes, as_stream(stream),
                              what);
}

extern "C" int soi_gemv_dip_fused_down(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                       const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                                       const int32_t* desc, int64_t k, const uint16_t* h_sel, uint16_t* y, int64_t H,
                                       int64_t group_size, int64_t num_groups, void* workspace,
                                       size_t workspace_bytes, void* stream) {
    const char* what = "soi_gemv_dip_fused_down";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(cache_rows >= 0 && staging_rows >= 0, "%s: negative row count", what);
    SOI_REQUIRE(y && (k == 0 || (desc && h_sel)), "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && (cache_rows == 0 || aligned16(cache_Wq)) &&
                     (staging_rows == 0 || aligned16(staging_Wq));
    DescRows rows{cache_Wq, cache_scale, cache_rows, staging_Wq, staging_scale, staging_rows, desc, row_bytes,
                  num_groups};
    return launch_sparse_down(rows, k, h_sel, y, H, group_size, vec, workspace, workspace_bytes, as_stream(stream),
                              what);
}

extern "C" int soi_gemv_w4a16_indexed_accumulate(const uint8_t* Wq_T, const float* scale_T, int64_t num_rows,
                                                 const int32_t* idx, int64_t k, const uint16_t* h_sel, uint16_t* y,
                                                 int64_t H, int64_t group_size, int64_t num_groups, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
    const char* what = "soi_gemv_w4a16_indexed_accumulate";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(num_rows >= 0, "%s: negative num_rows", what);
    SOI_REQUIRE(y && (k == 0 || (Wq_T && scale_T && idx && h_sel)), "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq_T);
    IndexRows rows{Wq_T, scale_T, num_rows, idx, row_bytes, num_groups};
    return launch_sparse_down(rows, k, h_sel, y, H, group_size, vec, workspace, workspace_bytes, as_stream(stream),
                              what);
}
