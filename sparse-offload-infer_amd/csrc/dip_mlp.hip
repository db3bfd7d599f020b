// The DIP MLP of one decoder layer in ONE launch (gfx950), hidden size 2048.
//
// Computes exactly what the four-launch DIP layer computes (the reference's
// op sequence, generate.py:276-310):
//   x     = rmsnorm(a + d, w)                    (RegNormX, the norm on load)
//   gate  = INT4 GEMV(W_gate, x)                 [I], binary16
//   idx   = rule-A top-k of |gate|               (topk_select.cu:19-95)
//   h_j   = fp16(silu(gate[idx_j]) * fp16(W_up[idx_j] . x))
//   y     = sum_j h_j * W_down^T[idx_j, :]       [2048], binary16
// with the same tiles, selection and sparse-down partition as those launches,
// so every output (gate, idx, count, h, y, and the next residual a + d) is
// bit-identical to them, and to the hot-cache variants that share them.
//
// One workgroup per CU (P <= number of CUs, 8 waves each), all resident at
// once; two grid barriers (soi_sync.h) separate three phases:
//   1. every wave: the RMSNorm of its 32 x elements (registers), then the gate
//      rows of its 4-row tiles (tile t -> workgroup t % P, wave t / P);
//   -- barrier: every gate written --
//   2. every workgroup: the rule-A selection over all I gates (the radix
//      select of soi_select.h; each workgroup computes it, which costs no
//      more latency than one doing it), keeping the channels of its own
//      positions [b*ppw, (b+1)*ppw); its waves run the up GEMV of those
//      positions with the SiLU gating and write h_sel and idx;
//   -- barrier: every h_sel / idx written --
//   3. the sparse-down items (column slice, row chunk) of down_plan, two per
//      workgroup (4 waves each), with the last-arrival combine per slice.
// Workspace: the grid-sync block, then the sparse-down counters, then its
// partial rows; all zero-filled once by the caller and left reusable.
#include "soi_device.h"
#include "soi_down.h"
#include "soi_host.h"
#include "soi_int4_tile.h"
#include "soi_rows.h"
#include "soi_select.h"
#include "soi_sync.h"

namespace soi {

constexpr int kMlpWaves = 8;
constexpr int kMlpThreads = kMlpWaves * kWave;
constexpr int kMlpK = 2048;  // hidden size: every gate / up / down^T row holds 2048 values, one 64-chunk pass
constexpr int kMlpRowBytes = kMlpK / 2;
constexpr int kGateR = 4;        // gate rows per tile
constexpr int kMlpMaxPpw = 64;   // selected positions per workgroup in phase 2
constexpr int kMlpMaxP = 1024;   // workgroups (flags in the sync block)
constexpr size_t kMlpAlign = 256;

struct MlpArgs {
    const uint16_t* a;   // residual stream
    const uint16_t* d;   // residual delta (may be null)
    const uint16_t* nw;  // RMSNorm weight
    float eps;
    uint16_t* x_out;  // a + d (may be null)
    uint16_t* h_out;  // rmsnorm(a + d) (may be null)
    const uint8_t* gW;
    const float* gS;
    const uint8_t* uW;
    const float* uS;
    const uint8_t* dW;
    const float* dS;
    int I, k, gs, G;
    uint16_t* gate;   // [I]
    int32_t* idx;     // [k]
    int32_t* cnt;     // [1]
    uint16_t* h_sel;  // [k]
    uint16_t* y;      // [2048]
    uint32_t* sync;
    uint32_t* counters;
    float* partial;
    int ppw;  // selected positions per workgroup (phase 2)
    int rpc, Rd, S;  // sparse-down partition (down_plan)
};

// Up rows of phase 2: local position j -> row s_ch[j] of the resident up matrix.
struct LdsChannelRows {
    const uint8_t* W;
    const float* S;
    const int32_t* ch;  // LDS
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return ch[j]; }
    __device__ __forceinline__ RowRef resolve(int64_t c, int64_t) const {
        return {W + c * kMlpRowBytes, S + c * G, true};
    }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
};

// Epilogue of phase 2: h[j] = fp16(silu(gate) * fp16(u_j)), gate = the raw
// binary16 gate of local position j (LDS); the rounding of SiluIdxY.
struct SiluLdsY {
    static constexpr bool kSwiglu = false;
    static constexpr bool kPrefetch = false;
    struct Pre {};
    uint16_t* h;           // h_sel + first position of the workgroup
    const uint16_t* g;     // LDS
    __device__ __forceinline__ void store(int64_t row, float total, bool valid) const {
        const float u = f16_bits_to_f32(f32_to_f16_bits(total));
        const float gv = f16_bits_to_f32(g[row]);
        stg(h + row, valid ? f32_to_f16_bits(silu_f32(gv) * u) : uint16_t(0x7e00u));
    }
};

template <int E, int RU>
__global__ __launch_bounds__(kMlpThreads) void dip_mlp_kernel(MlpArgs p) {
    __shared__ uint32_t s_hist[radix_hist_offset<F16AbsValues>(F16AbsValues::kPasses)];
    __shared__ float s_max[kMlpWaves];
    __shared__ uint32_t s_tot[kMlpWaves];
    __shared__ int32_t s_ch[kMlpMaxPpw];
    __shared__ uint16_t s_g[kMlpMaxPpw];
    __shared__ float s_red[2][kRedFloats];
    __shared__ int s_last[2];
    __shared__ uint32_t s_epoch;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
    const int b = static_cast<int>(blockIdx.x), P = static_cast<int>(gridDim.x);
    const int I = p.I;

    // ---- phase 1: x = rmsnorm(a + d) per lane chunk, gate rows in 4-row tiles ----
    RegNormX xs;
    {
        const u32x4* a4 = reinterpret_cast<const u32x4*>(p.a);
        const u32x4* w4 = reinterpret_cast<const u32x4*>(p.nw);
        const u32x4* e4 = reinterpret_cast<const u32x4*>(p.d ? p.d : p.a);  // unconditional loads
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xs.t[i] = ldg(a4 + 4 * lane + i);
            xs.g[i] = ldg(w4 + 4 * lane + i);
            xs.e[i] = ldg(e4 + 4 * lane + i);
        }
    }
    xs.has_d = p.d != nullptr;
    xs.eps = p.eps;
    xs.K = kMlpK;
    xs.x_out = (b == 0 && wave == 0) ? p.x_out : nullptr;
    xs.h_out = (b == 0 && wave == 0) ? p.h_out : nullptr;
    xs.b = p.a;
    const uint32_t epoch = grid_epoch(p.sync, &s_epoch);
    const DenseRows grows{p.gW, p.gS, kMlpRowBytes, p.G};
    const int tiles = I / kGateR;
    for (int t = wave * P + b; t < tiles; t += kMlpWaves * P) {
        gemv_int4_tile<kGateR, 1, true, true, true, true>(grows, I, xs, StoreY{p.gate}, kMlpK, p.gs,
                                                        static_cast<int64_t>(t) * kGateR);
        xs.x_out = nullptr;
        xs.h_out = nullptr;
    }
    // this lane's 32 normed x values, kept for the up GEMV (the same arithmetic as inside the tile)
    f16x2 xv[16];
    {
        RegNormX x2 = xs;
        x2.x_out = nullptr;
        x2.h_out = nullptr;
        x2.template load<true, true>(kMlpK, lane, true, xv);
    }
    grid_barrier(p.sync, 2u * epoch + 1u);

    // ---- phase 2: rule-A selection over all I gates, then the up GEMV of this workgroup's positions ----
    const int base_i = wave * kWave * E + lane;
    uint32_t raw[E];
    float val[E];
    uint32_t key[E];
    float local_max = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = base_i + j * kWave;
        raw[j] = ldg(p.gate + (i < I ? i : I - 1));
    }
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = base_i + j * kWave;
        val[j] = (i < I) ? f16_bits_to_f32(static_cast<uint16_t>(raw[j] & 0x7fffu)) : __builtin_nanf("");
        key[j] = F16AbsValues::key_of(val[j]);
        local_max = fmaxf(local_max, val[j]);
    }
    const float tau = rule_a_tau<E, kMlpWaves, F16AbsValues>(key, local_max, s_hist, s_max, p.k, tid);
    const int64_t p0 = static_cast<int64_t>(b) * p.ppw;
    const int64_t p1 = (p0 + p.ppw < p.k) ? p0 + p.ppw : static_cast<int64_t>(p.k);
    const uint32_t total = rule_a_compact<E, kMlpWaves>(val, tau, s_tot, tid, [&](uint32_t pos, int j) {
        if (pos >= p0 && pos < p1) {
            const int c = base_i + j * kWave;
            s_ch[pos - p0] = c;
            s_g[pos - p0] = static_cast<uint16_t>(raw[j]);
            stg(p.idx + pos, static_cast<int32_t>(c));
        }
    });
    const int64_t kk = total < static_cast<uint32_t>(p.k) ? static_cast<int64_t>(total) : static_cast<int64_t>(p.k);
    if (b == 0 && tid == 0) stg(p.cnt, static_cast<int32_t>(kk));
    __syncthreads();  // s_ch / s_g complete
    const int64_t q1 = p1 < kk ? p1 : kk;
    const int64_t n_loc = q1 > p0 ? q1 - p0 : 0;  // this workgroup's selected positions
    if (static_cast<int64_t>(wave) * RU < n_loc)
        gemv_int4_tile<RU, 1, true, true, true, false>(LdsChannelRows{p.uW, p.uS, s_ch, p.G}, n_loc, RegX{xv, p.a},
                                                       SiluLdsY{p.h_sel + p0, s_g}, kMlpK, p.gs,
                                                       static_cast<int64_t>(wave) * RU);
    grid_barrier(p.sync, 2u * epoch + 2u);

    // ---- phase 3: the sparse down over the selected rows, items (slice, chunk) of down_plan, two per workgroup ----
    const int items = p.S * p.Rd;
    const int half = wave >> 2;
    const IndexRows drows{p.dW, p.dS, static_cast<int64_t>(I), p.idx, kMlpRowBytes, p.G};
    for (int base = 0; base < items; base += 2 * P) {
        const int it = base + half * P + b;
        const bool active = it < items;
        sparse_down_item<kDownU, true, true>(drows, PlainH{p.h_sel}, p.y, p.partial, p.counters, kk, kMlpK, p.gs,
                                             p.rpc, p.Rd, s_red[half], &s_last[half], active ? it % p.S : 0,
                                             active ? it / p.S : 0, tid & (kDownThreads - 1), active);
    }
    grid_epoch_advance(p.sync, epoch);
}

// ---- host side ----

static size_t round_up(size_t n) { return (n + kMlpAlign - 1) / kMlpAlign * kMlpAlign; }

static size_t mlp_sync_bytes() { return round_up(kSyncHeaderBytes + sizeof(uint32_t) * kMlpMaxP); }

static size_t mlp_workspace_bytes(int64_t k) {
    const DownPlan d = down_plan(kMlpK, k);
    return mlp_sync_bytes() + round_up(static_cast<size_t>(d.S) * sizeof(uint32_t)) +
           static_cast<size_t>(d.R) * kMlpK * sizeof(float);
}

// One workgroup per CU: P = the device's CU count, provided one workgroup of
// this kernel fits on a CU (checked once per device), so all P are resident.
static int mlp_grid(const void* kernel, int* P, const char* what) {
    int dev = 0;
    SOI_HIP_TRY(hipGetDevice(&dev), what);
    int cus = 0;
    SOI_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), what);
    int per_cu = 0;
    SOI_HIP_TRY(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kMlpThreads, 0), what);
    SOI_REQUIRE(per_cu >= 1 && cus >= 1, "%s: one workgroup of %d threads does not fit on a CU", what, kMlpThreads);
    *P = cus < kMlpMaxP ? cus : kMlpMaxP;
    return SOI_OK;
}

}  // namespace soi

using namespace soi;

extern "C" size_t soi_dip_mlp_workspace_bytes(int64_t k) { return k >= 1 ? mlp_workspace_bytes(k) : 0; }

extern "C" int soi_dip_mlp(const uint16_t* x, const uint16_t* delta, const uint16_t* norm_weight, float eps,
                           uint16_t* x_out, uint16_t* h_out, const uint8_t* gate_Wq, const float* gate_scale,
                           const uint8_t* up_Wq, const float* up_scale, const uint8_t* down_T_Wq,
                           const float* down_T_scale, int64_t I, int64_t H, int64_t k, int64_t group_size,
                           int64_t num_groups, uint16_t* gate_out, int32_t* out_indices, int32_t* out_count,
                           uint16_t* h_sel, uint16_t* y, void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "soi_dip_mlp";
    SOI_REQUIRE(H == kMlpK, "%s: the single-launch DIP MLP is built for hidden size %d, got %lld", what, kMlpK,
                (long long)H);
    SOI_REQUIRE(group_size >= 32 && group_size % 32 == 0 && group_size <= kMlpK,
                "%s: group_size must be a multiple of 32 in [32, %d]", what, kMlpK);
    SOI_REQUIRE(num_groups == ceil_div64(H, group_size), "%s: num_groups must be ceil(H/group_size)", what);
    SOI_REQUIRE(I >= kGateR && I % kGateR == 0 && I <= kMlpThreads * 24,
                "%s: the intermediate size must be a multiple of %d in [%d, %d]", what, kGateR, kGateR,
                kMlpThreads * 24);
    SOI_REQUIRE(k >= 1 && k <= I, "%s: k must be in [1, I]", what);
    SOI_REQUIRE(x && norm_weight && gate_Wq && gate_scale && up_Wq && up_scale && down_T_Wq && down_T_scale &&
                    gate_out && out_indices && out_count && h_sel && y,
                "%s: null pointer", what);
    SOI_REQUIRE(aligned16(x) && aligned16(norm_weight) && (!delta || aligned16(delta)) && (!x_out || aligned16(x_out)) &&
                    (!h_out || aligned16(h_out)) && aligned16(gate_Wq) && aligned16(up_Wq) && aligned16(down_T_Wq),
                "%s: x, delta, norm_weight, x_out, h_out and the weights must be 16-byte aligned", what);
    SOI_REQUIRE(x_out != x && x_out != delta && (!x_out || x_out != h_out),
                "%s: x_out must not alias x, delta or h_out (other workgroups still read them)", what);
    const size_t need = mlp_workspace_bytes(k);
    if (!workspace || workspace_bytes < need) {
        set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    int P = 0;
    // every instance has the same resources (the selection and tile sizes only change loop counts)
    int s = mlp_grid(reinterpret_cast<const void*>(&dip_mlp_kernel<24, 8>), &P, what);
    if (s) return s;
    const int64_t ppw = ceil_div64(k, P);
    SOI_REQUIRE(ppw <= kMlpMaxPpw, "%s: k = %lld is more than %d positions per workgroup on %d workgroups", what,
                (long long)k, kMlpMaxPpw, P);
    const DownPlan d = down_plan(H, k);
    MlpArgs a;
    a.a = x;
    a.d = delta;
    a.nw = norm_weight;
    a.eps = eps;
    a.x_out = x_out;
    a.h_out = h_out;
    a.gW = gate_Wq;
    a.gS = gate_scale;
    a.uW = up_Wq;
    a.uS = up_scale;
    a.dW = down_T_Wq;
    a.dS = down_T_scale;
    a.I = static_cast<int>(I);
    a.k = static_cast<int>(k);
    a.gs = static_cast<int>(group_size);
    a.G = static_cast<int>(num_groups);
    a.gate = gate_out;
    a.idx = out_indices;
    a.cnt = out_count;
    a.h_sel = h_sel;
    a.y = y;
    char* ws = static_cast<char*>(workspace);
    a.sync = reinterpret_cast<uint32_t*>(ws);
    a.counters = reinterpret_cast<uint32_t*>(ws + mlp_sync_bytes());
    a.partial = reinterpret_cast<float*>(ws + mlp_sync_bytes() + round_up(static_cast<size_t>(d.S) * sizeof(uint32_t)));
    a.ppw = static_cast<int>(ppw);
    a.rpc = static_cast<int>(d.rpc);
    a.Rd = static_cast<int>(d.R);
    a.S = static_cast<int>(d.S);
    const int64_t E = ceil_div64(I, kMlpThreads);
    const int64_t ru = ceil_div64(ppw, kMlpWaves);
    hipStream_t st = as_stream(stream);
    const dim3 grid(static_cast<unsigned>(P)), block(kMlpThreads);
#define SOI_M(EE, RR) hipLaunchKernelGGL((dip_mlp_kernel<EE, RR>), grid, block, 0, st, a)
#define SOI_MR(EE)                   \
    do {                             \
        if (ru <= 1) SOI_M(EE, 1);   \
        else if (ru <= 2) SOI_M(EE, 2); \
        else if (ru <= 4) SOI_M(EE, 4); \
        else SOI_M(EE, 8);           \
    } while (0)
    if (E <= 4) SOI_MR(4);
    else if (E <= 8) SOI_MR(8);
    else if (E <= 12) SOI_MR(12);
    else if (E <= 16) SOI_MR(16);
    else SOI_MR(24);
#undef SOI_MR
#undef SOI_M
    return launch_status(what);
}

extern "C" int soi_dip_mlp_check(const void* workspace, void* stream) {
    const char* what = "soi_dip_mlp_check";
    SOI_REQUIRE(workspace, "%s: null workspace", what);
    GridSync gs_host{};
    SOI_HIP_TRY(hipMemcpyAsync(&gs_host, workspace, sizeof(gs_host), hipMemcpyDeviceToHost, as_stream(stream)), what);
    SOI_HIP_TRY(hipStreamSynchronize(as_stream(stream)), what);
    if (gs_host.error) {
        set_last_error("%s: a grid barrier wait gave up (the workgroups were not all resident); outputs of the "
                       "calls since the workspace was cleared are not valid", what);
        return SOI_ERR_HIP;
    }
    return SOI_OK;
}
