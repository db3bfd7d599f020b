// Sparse down projection over selected rows of down_proj^T (gfx950).
//
// Restates csrc/kernels/gemv_sparse_accumulate.cu:10-38 and the descriptor
// form gemv_dip_fused.cu:116-154:
//   y[c] = sum_{j<k} (h_j * s[j, c/gs]) * q[j, c],  fp32 accumulation, fp16 out.
// The reference runs one thread per output column over all k rows, which
// touches 4 bytes per row per thread and uses a handful of CUs. Here one
// launch tiles (column slice) x (row chunk):
//   * a slice is 256 columns = 8 16-byte chunks (128 bytes of each packed
//     row); lane l of a wave owns chunk (l & 7) of row (l >> 3) of an 8-row
//     group, so one wave-wide 16-byte load reads 8 rows x 128 bytes;
//   * a workgroup (4 waves) owns rows [r*rpc, (r+1)*rpc) of its slice; wave w
//     takes the 8-row groups w, w+4, w+8, ..., U groups per batch, all loads of
//     a batch issued before any arithmetic. Each lane keeps 32 fp32 sums; per
//     row: coef = fl(h_j*s), acc_c = fma(coef, q_c, acc_c) with q_c an exact
//     binary16 integer;
//   * the 32 (wave, row-in-group) partials of each column are summed through
//     LDS in a fixed order and the workgroup writes one fp32 partial row of
//     256 columns to the workspace;
//   * the partial rows are written and read device-coherent (st_agent /
//     ld_agent); arrival (arrive_coherent): every wave waits for its partial
//     stores to complete, then one thread counts the workgroup in on the
//     slice's counter; the last of the slice's R workgroups sums the R partial
//     rows of the slice in ascending r, writes fp16 y, and resets the counter
//     to zero (no L2 write-back or invalidate);
//   * items are placed XCD-aware (down_item): the workgroups of one row chunk
//     share an XCD, so the chunk's scales, indices and coefficients are
//     fetched into one L2 once.
// Fixed partition and fixed order: deterministic, and every row source
// (gathered rows, hot cache + staging descriptors, resident index list) gives
// bit-identical results for the same logical rows.
#include <mutex>

#include "soi_device.h"
#include "soi_down.h"
#include "soi_host.h"
#include "soi_rows.h"
#include "soi_select.h"

namespace soi {

template <int U, bool VEC, bool CHUNK_SCALE, class Rows, class HS>
__global__ __launch_bounds__(kDownThreads) void sparse_down_kernel(Rows rows, const HS hs,
                                                                    uint16_t* __restrict__ y, float* __restrict__ partial,
                                                                    uint32_t* __restrict__ counters, int64_t k, int H,
                                                                    int gs, int rpc, int R) {
    __shared__ float red[kRedFloats];
    __shared__ int s_last;
    int slice, r;
    down_item(slice, r);
    sparse_down_item<U, VEC, CHUNK_SCALE>(rows, hs, y, partial, counters, k, H, gs, rpc, R, red, &s_last, slice, r,
                                          static_cast<int>(threadIdx.x), true);
}

// k == 0: y = 0 (the empty sum, as the reference's loop yields); a fill kernel
// rather than a memset so the call stays capturable in a HIP graph.
__global__ __launch_bounds__(256) void sparse_down_zero_kernel(uint16_t* __restrict__ y, int64_t H) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i < H) stg(y + i, uint16_t(0));
}

// Fused DIP selection + gated down projection. Every workgroup of the sparse
// down grid first computes the rule-A selection over |gate| itself (the
// top-k radix select of soi_select.h over n <= 256*E binary16 gates, read
// from L2), keeps the channels (and raw gates) of its own row chunk in LDS,
// and then runs the gated sparse down on them: no top-k launch and no global
// index round trip. The row partition, coefficients and arithmetic are those
// of sparse_down_kernel over IndexRows + GatedH, so y equals the top-k launch
// followed by the gated down bit for bit; the selection equals the top-k
// kernel's (slice-0 workgroups write the indices of their chunks, workgroup
// (0, 0) the count). Positions at or past the selected count contribute
// nothing.
constexpr int kFusedMaxRpc = 1024;

struct LdsIndexRows {
    const uint8_t* W;
    const float* S;
    const int32_t* ch;  // LDS: channel of row j0 + i
    int64_t j0;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return ch[j - j0]; }
    __device__ __forceinline__ RowRef resolve(int64_t c, int64_t) const { return {W + c * row_bytes, S + c * G, true}; }
};
struct LdsGatedH {
    const uint16_t* g;  // LDS: raw binary16 gate of row j0 + i
    const int32_t* ch;  // LDS: its channel
    const uint16_t* up;
    int64_t j0;
    struct Raw {
        uint16_t g, u;
    };
    __device__ __forceinline__ int64_t key(int64_t j) const { return j - j0; }
    __device__ __forceinline__ Raw fetch(int64_t i) const { return {g[i], ldg(up + ch[i])}; }
    __device__ __forceinline__ static float value(Raw r) {
        return f16_bits_to_f32(f32_to_f16_bits(silu_f32(f16_bits_to_f32(r.g)) * f16_bits_to_f32(r.u)));
    }
};

template <int E, int U, bool VEC, bool CHUNK_SCALE>
__global__ __launch_bounds__(kDownThreads) void dip_select_down_kernel(
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up, int n, int k, int32_t* __restrict__ out_idx,
    int32_t* __restrict__ out_count, const uint8_t* __restrict__ W, const float* __restrict__ S, int64_t row_bytes,
    int64_t G, uint16_t* __restrict__ y, float* __restrict__ partial, uint32_t* __restrict__ counters, int H, int gs,
    int rpc, int R) {
    __shared__ float red[kRedFloats];
    __shared__ int s_last;
    __shared__ uint32_t s_hist[radix_hist_offset<F16AbsValues>(F16AbsValues::kPasses)];
    __shared__ float s_max[kDownWaves];
    __shared__ uint32_t s_tot[kDownWaves];
    __shared__ int32_t s_ch[kFusedMaxRpc];
    __shared__ uint16_t s_g[kFusedMaxRpc];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int base_i = wave * kWave * E + lane;
    int slice, chunk;
    down_item(slice, chunk);
    const int64_t j0 = static_cast<int64_t>(chunk) * rpc;
    const int64_t j1 = (j0 + rpc < k) ? j0 + rpc : static_cast<int64_t>(k);

    uint32_t raw[E];
    float val[E];
    uint32_t key[E];
    float local_max = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {  // clamped index: every load is issued unconditionally
        const int i = base_i + j * kWave;
        raw[j] = ldg(gate + (i < n ? i : n - 1));
    }
    // the histograms are zeroed and published while the gates are in flight (rule A's SYNCED form)
    rule_a_zero_hist<kDownWaves, F16AbsValues>(s_hist, tid);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = base_i + j * kWave;
        val[j] = (i < n) ? f16_bits_to_f32(static_cast<uint16_t>(raw[j] & 0x7fffu)) : __builtin_nanf("");
        key[j] = F16AbsValues::key_of(val[j]);
        local_max = fmaxf(local_max, val[j]);
    }
    const float tau =
        rule_a_tau<E, kDownWaves, F16AbsValues, true, NoMid, true>(key, local_max, s_hist, s_max, k, tid);
    const bool writer = slice == 0;
    // only this workgroup's chunk [j0, j1) of the positions is emitted
    const uint32_t total = rule_a_compact<E, kDownWaves>(
        val, tau, s_tot, tid, static_cast<uint32_t>(j0), static_cast<uint32_t>(j1), [&](uint32_t pos, int j) {
            const int c = base_i + j * kWave;
            s_ch[pos - j0] = c;
            s_g[pos - j0] = static_cast<uint16_t>(raw[j]);
            if (writer) stg(out_idx + pos, static_cast<int32_t>(c));
        });
    const int64_t kk = total < static_cast<uint32_t>(k) ? static_cast<int64_t>(total) : static_cast<int64_t>(k);
    if (writer && chunk == 0 && tid == 0) stg(out_count, static_cast<int32_t>(kk));
    __syncthreads();  // s_ch / s_g of the chunk complete
    sparse_down_item<U, VEC, CHUNK_SCALE>(LdsIndexRows{W, S, s_ch, j0, row_bytes, G},
                                               LdsGatedH{s_g, s_ch, up, j0}, y, partial, counters, kk, H, gs, rpc,
                                               R, red, &s_last, slice, chunk, tid, true);
}

// Workspace: the S arrival counters first (their place depends on H only, so
// calls with any k can share a workspace), then the R x H fp32 partial rows.
constexpr size_t kDownAlign = 256;

static size_t down_counter_bytes(const DownPlan& p) {
    return (static_cast<size_t>(p.S) * sizeof(uint32_t) + kDownAlign - 1) / kDownAlign * kDownAlign;
}

static size_t down_workspace_bytes(int64_t H, int64_t k) {
    if (H <= 0 || k <= 0) return 0;
    const DownPlan p = down_plan(H, k);
    return down_counter_bytes(p) + static_cast<size_t>(p.R) * static_cast<size_t>(H) * sizeof(float);
}

// counters: S zeroed words (left zero); partial: R x H floats
template <class Rows, class HS>
static int launch_sparse_down_on(const Rows& rows, int64_t k, const HS& h, uint16_t* y, int64_t H, int64_t gs,
                                 bool vec, uint32_t* counters, float* partial, hipStream_t st, const char* what) {
    if (k == 0) {
        hipLaunchKernelGGL(sparse_down_zero_kernel, dim3(static_cast<unsigned>(ceil_div64(H, 256))), dim3(256), 0, st,
                           y, H);
        return launch_status(what);
    }
    const DownPlan p = down_plan(H, k);
    SOI_REQUIRE(p.R <= 65535 && p.S <= (int64_t(1) << 31) - 1, "%s: partition out of range", what);
    const dim3 grid(static_cast<unsigned>(p.S), static_cast<unsigned>(p.R));
    const bool cs = (gs % 32) == 0;
    const int Hi = static_cast<int>(H), gi = static_cast<int>(gs), ri = static_cast<int>(p.rpc),
              Ri = static_cast<int>(p.R);
    // 8-row groups per wave per batch: as many as a chunk gives each wave (rpc / 32), in steps of 2, 3 and 6; a
    // batch slot past the chunk loads the zero buffer, and those repeated loads of one address cost time
    const int64_t gpw = p.rpc / (static_cast<int64_t>(kDownWaves) * kGroupRows);
#define SOI_D(U, V, CS)                                                                                        \
    hipLaunchKernelGGL((sparse_down_kernel<U, V, CS, Rows, HS>), grid, dim3(kDownThreads), 0, st, rows, h, y,  \
                       partial, counters, k, Hi, gi, ri, Ri)
#define SOI_DU(V, CS)                                                                                          \
    do {                                                                                                       \
        if (gpw <= 2) SOI_D(2, V, CS);                                                                         \
        else if (gpw <= 3) SOI_D(3, V, CS);                                                                    \
        else SOI_D(kDownU, V, CS);                                                                             \
    } while (0)
    if (vec) {
        if (cs) SOI_DU(true, true); else SOI_DU(true, false);
    } else {
        if (cs) SOI_DU(false, true); else SOI_DU(false, false);
    }
#undef SOI_DU
#undef SOI_D
    return launch_status(what);
}

// workspace = [S counters, rounded to 256 bytes][R x H partial rows]
template <class Rows, class HS>
static int launch_sparse_down(const Rows& rows, int64_t k, const HS& h, uint16_t* y, int64_t H, int64_t gs,
                              bool vec, void* workspace, size_t ws_bytes, hipStream_t st, const char* what) {
    if (k > 0) {
        const size_t need = down_workspace_bytes(H, k);
        if (!workspace || ws_bytes < need) {
            set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, ws_bytes);
            return SOI_ERR_WORKSPACE;
        }
    }
    const size_t cb = k > 0 ? down_counter_bytes(down_plan(H, k)) : 0;
    return launch_sparse_down_on(rows, k, h, y, H, gs, vec, static_cast<uint32_t*>(workspace),
                                 reinterpret_cast<float*>(static_cast<char*>(workspace) + cb), st, what);
}

// ---------------------------------------------------------------------------
// Allocation-free form. Its workspace is `scratch`, a file-scope device array
// of kNoAllocScratchBytes that every GPU holds for the life of the process.
// Host code never passes the array's name to a kernel (in host code it is a
// stand-in, not a device address): the device address is looked up once per
// device with hipGetSymbolAddress and kept in g_scratch_addr.
// ---------------------------------------------------------------------------
// Layout: a fixed 16 KB counter area first (slice s of any call uses word s,
// so calls with different H never see another call's partial rows in their
// counters), then the R x H partial rows.
constexpr size_t kNoAllocScratchBytes = size_t(2) << 20;
constexpr size_t kNoAllocCounterBytes = size_t(16) << 10;
constexpr int kNoAllocMaxDevices = 64;
static __device__ __attribute__((aligned(256))) uint8_t scratch[kNoAllocScratchBytes];

// clears the arrival-counter area at set-up (a fill kernel, not a memset, so a
// first call made under stream capture stays capturable)
__global__ __launch_bounds__(256) void scratch_clear_kernel(uint32_t* __restrict__ p, int64_t words) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < words;
         i += static_cast<int64_t>(gridDim.x) * 256)
        stg(p + i, 0u);
}

static std::mutex g_scratch_mu;
static void* g_scratch_addr[kNoAllocMaxDevices] = {};

// The current device's scratch address; on a device's first call, looks it up
// and zeroes the counter area (the array is zero at load as well; every call
// leaves its counters at zero again).
static int noalloc_scratch(hipStream_t st, void** out, const char* what) {
    int dev = -1;
    SOI_HIP_TRY(hipGetDevice(&dev), what);
    SOI_REQUIRE(dev >= 0 && dev < kNoAllocMaxDevices, "%s: device %d out of range", what, dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        SOI_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), what);
        SOI_REQUIRE(p != nullptr, "%s: no device address for the scratch array", what);
        const int64_t words = static_cast<int64_t>(kNoAllocCounterBytes / sizeof(uint32_t));
        hipLaunchKernelGGL(scratch_clear_kernel, dim3(16), dim3(256), 0, st, static_cast<uint32_t*>(p), words);
        const int s = launch_status(what);
        if (s) return s;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return SOI_OK;
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

extern "C" size_t soi_sparse_accumulate_workspace_bytes(int64_t H, int64_t k) { return down_workspace_bytes(H, k); }

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
    return launch_sparse_down(rows, k, PlainH{h_sel}, y, H, group_size, vec, workspace, workspace_bytes,
                              as_stream(stream), what);
}

extern "C" size_t soi_sparse_accumulate_noalloc_max_scratch_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int soi_gemv_w4a16_sparse_accumulate_noalloc(const uint8_t* Wq_sel, const float* scale_sel,
                                                        const uint16_t* h_sel, uint16_t* y, int64_t H, int64_t k,
                                                        int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_w4a16_sparse_accumulate_noalloc";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(y && (k == 0 || (Wq_sel && scale_sel && h_sel)), "%s: null pointer", what);
    if (k > 0) {
        const DownPlan p = down_plan(H, k);
        const size_t need = kNoAllocCounterBytes + static_cast<size_t>(p.R) * static_cast<size_t>(H) * sizeof(float);
        SOI_REQUIRE(static_cast<size_t>(p.S) * sizeof(uint32_t) <= kNoAllocCounterBytes && need <= kNoAllocScratchBytes,
                    "%s: H = %lld, k = %lld needs %zu bytes of scratch, more than the %zu this form holds per GPU; "
                    "call soi_gemv_w4a16_sparse_accumulate with a workspace instead",
                    what, (long long)H, (long long)k, need, kNoAllocScratchBytes);
    }
    hipStream_t st = as_stream(stream);
    void* ws = nullptr;
    s = noalloc_scratch(st, &ws, what);
    if (s) return s;
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq_sel);
    DenseRows rows{Wq_sel, scale_sel, row_bytes, num_groups};
    return launch_sparse_down_on(rows, k, PlainH{h_sel}, y, H, group_size, vec, static_cast<uint32_t*>(ws),
                                 reinterpret_cast<float*>(static_cast<char*>(ws) + kNoAllocCounterBytes), st, what);
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
    return launch_sparse_down(rows, k, PlainH{h_sel}, y, H, group_size, vec, workspace, workspace_bytes,
                              as_stream(stream), what);
}

extern "C" int soi_gemv_dip_cached_down(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                        const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                                        const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* h_sel,
                                        uint16_t* y, int64_t H, int64_t group_size, int64_t num_groups,
                                        const uint8_t* staging_Wq, void* workspace, size_t workspace_bytes,
                                        void* stream) {
    const char* what = "soi_gemv_dip_cached_down";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(cache_rows >= 0 && num_channels >= 0 && num_channels <= (int64_t(1) << 31) - 1,
                "%s: negative or too large row / channel count", what);
    SOI_REQUIRE(k == 0 || num_channels >= 1, "%s: a selection needs at least one channel", what);
    SOI_REQUIRE(y && (k == 0 || (sel && slot_of && (full_Wq || staging_Wq) && full_scale && h_sel)),
                "%s: null pointer", what);
    SOI_REQUIRE(k == 0 || cache_rows == 0 || (cache_Wq && cache_scale), "%s: null cache", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const uint8_t* miss_src = staging_Wq ? staging_Wq : full_Wq;
    const bool vec = (row_bytes % 16 == 0) && (k == 0 || aligned16(miss_src)) &&
                     (cache_rows == 0 || aligned16(cache_Wq));
    hipStream_t st = as_stream(stream);
    if (staging_Wq) {
        SlotStageRows rows{cache_Wq, cache_scale, cache_rows, staging_Wq, full_scale, num_channels, sel, slot_of,
                           row_bytes, num_groups};
        return launch_sparse_down(rows, k, PlainH{h_sel}, y, H, group_size, vec, workspace, workspace_bytes, st,
                                  what);
    }
    SlotRows rows{cache_Wq, cache_scale, cache_rows, full_Wq, full_scale, num_channels, sel, slot_of, row_bytes,
                  num_groups};
    return launch_sparse_down(rows, k, PlainH{h_sel}, y, H, group_size, vec, workspace, workspace_bytes, st, what);
}

extern "C" int soi_gemv_w4a16_indexed_accumulate_gated(const uint8_t* Wq_T, const float* scale_T, int64_t num_rows,
                                                       const int32_t* idx, int64_t k, const uint16_t* gate,
                                                       const uint16_t* up, int64_t num_channels, uint16_t* y,
                                                       int64_t H, int64_t group_size, int64_t num_groups,
                                                       void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "soi_gemv_w4a16_indexed_accumulate_gated";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(num_rows >= 0 && num_channels >= 0 && num_channels <= (int64_t(1) << 31) - 1,
                "%s: negative or too large row / channel count", what);
    SOI_REQUIRE(k == 0 || num_channels >= 1, "%s: a selection needs at least one channel", what);
    SOI_REQUIRE(y && (k == 0 || (Wq_T && scale_T && idx && gate && up)), "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq_T);
    IndexRows rows{Wq_T, scale_T, num_rows, idx, row_bytes, num_groups};
    return launch_sparse_down(rows, k, GatedH{gate, up, idx, static_cast<int>(num_channels)}, y, H, group_size, vec,
                              workspace, workspace_bytes, as_stream(stream), what);
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
    return launch_sparse_down(rows, k, PlainH{h_sel}, y, H, group_size, vec, workspace, workspace_bytes,
                              as_stream(stream), what);
}

extern "C" int soi_dip_select_gated_down(const uint16_t* gate, const uint16_t* up, int64_t num_channels, int64_t k,
                                         const uint8_t* Wq_T, const float* scale_T, int64_t num_rows,
                                         int32_t* out_indices, int32_t* out_count, uint16_t* y, int64_t H,
                                         int64_t group_size, int64_t num_groups, void* workspace,
                                         size_t workspace_bytes, void* stream) {
    const char* what = "soi_dip_select_gated_down";
    int s = check_down(H, k, group_size, num_groups, what);
    if (s) return s;
    SOI_REQUIRE(num_channels >= 1 && num_channels <= (int64_t(1) << 30), "%s: num_channels must be in [1, 2^30]",
                what);
    SOI_REQUIRE(k >= 1 && k <= num_channels, "%s: k must be in [1, num_channels]", what);
    SOI_REQUIRE(num_rows >= num_channels, "%s: down_proj^T has %lld rows, fewer than the %lld channels", what,
                (long long)num_rows, (long long)num_channels);
    SOI_REQUIRE(gate && up && Wq_T && scale_T && out_indices && out_count && y, "%s: null pointer", what);
    const int64_t row_bytes = ceil_div64(H, 8) * 4;
    const bool vec = (row_bytes % 16 == 0) && aligned16(Wq_T) && (group_size % 32) == 0;
    const size_t need = down_workspace_bytes(H, k);
    if (!workspace || workspace_bytes < need) {  // checked before either path launches anything
        set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    const DownPlan p = down_plan(H, k);
    const int64_t E = ceil_div64(num_channels, kDownThreads);
    if (!vec || E > 32 || p.rpc > kFusedMaxRpc) {
        // outside the fused kernel's limits: the top-k kernel, then the gated down over its indices
        s = soi_topk_threshold_select_f16abs(gate, num_channels, k, out_indices, out_count, stream);
        if (s) return s;
        return soi_gemv_w4a16_indexed_accumulate_gated(Wq_T, scale_T, num_rows, out_indices, k, gate, up,
                                                       num_channels, y, H, group_size, num_groups, workspace,
                                                       workspace_bytes, stream);
    }
    SOI_REQUIRE(p.R <= 65535, "%s: partition out of range", what);
    uint32_t* counters = static_cast<uint32_t*>(workspace);
    float* partial = reinterpret_cast<float*>(static_cast<char*>(workspace) + down_counter_bytes(p));
    const dim3 grid(static_cast<unsigned>(p.S), static_cast<unsigned>(p.R));
    const int ni = static_cast<int>(num_channels), ki = static_cast<int>(k), Hi = static_cast<int>(H),
              gi = static_cast<int>(group_size), ri = static_cast<int>(p.rpc), Ri = static_cast<int>(p.R);
    hipStream_t st = as_stream(stream);
#define SOI_F(EE, UU)                                                                                              \
    hipLaunchKernelGGL((dip_select_down_kernel<EE, UU, true, true>), grid, dim3(kDownThreads), 0, st, gate, up, ni, \
                       ki, out_indices, out_count, Wq_T, scale_T, row_bytes, num_groups, y, partial, counters, Hi, gi, \
                       ri, Ri)
#define SOI_FU(EE)                                                                                                 \
    do {                                                                                                           \
        if (gpw <= 2) SOI_F(EE, 2);                                                                                \
        else if (gpw <= 3) SOI_F(EE, 3);                                                                           \
        else SOI_F(EE, kDownU);                                                                                    \
    } while (0)
    const int64_t gpw = p.rpc / (static_cast<int64_t>(kDownWaves) * kGroupRows);  // as in launch_sparse_down_on
    if (E <= 8) SOI_FU(8);
    else if (E <= 16) SOI_FU(16);
    else if (E <= 24) SOI_FU(24);
    else SOI_FU(32);
#undef SOI_FU
#undef SOI_F
    return launch_status(what);
}
