// DIP down projection for resident weights as ONE dense launch: the rule-A
// selection and y = sum over the selected channels c of h_c * s_T[c, col/gs]
// * q_T[c, col] (the sparse accumulate of the reference's DIP MLP,
// generate.py:304-308, gemv_sparse_accumulate.cu:10-38), computed as a GEMV
// over a transposed copy of the same quantized values.
//
// down_proj^T's INT4 values q_T[c, col] and scales s_T[c, col/gs] are kept a
// second time transposed: Wt [H, n/2] (row col = the n channels' nibbles of
// output column col, packed like every other INT4 row) and St [H/gs, n]
// (St[g, c] = s_T[c, g]). Output col is then a dot product over the n
// channels with the coefficient vector x_g[c] = sel(c) * h_c * St[g, c] of its
// column group g: the same terms as the reference's sum (fp32 products
// h * s * q), in another order, with no cross-workgroup reduction at all.
//
// Workgroup = 8 waves x kDdRowsPerWave rows, consecutive output columns of
// one column group.
//   1. it requests the gates the selection reads, the gate / h / St[g] values
//      of its 8-channel groups, then every packed chunk of its rows;
//   2. it forms every channel's coefficient h_c * St[g, c] in fp32 and their
//      largest magnitude (handed over through the selection's first barrier);
//   3. it runs the rule-A selection over all n gates itself (radix select and
//      bisection replay, soi_select.h) while the row chunks land, and the cut
//      that keeps the first k channels at or above the threshold
//      (rule_a_cut): sel(c) = |gate_c| >= tau and c < cut;
//   4. x_g[c] = sel(c) * coefficient is scaled by a power of two 2^e (exact;
//      e from the largest magnitude) and split into binary16 hi + lo parts in
//      LDS (hi = fp16(x), lo = fp16(x - hi): x to ~2^-22 relative), so the
//      dot products run as v_dot2 on exact binary16 q values with fp32
//      accumulation;
//   5. each wave sums its rows over its lanes (DPP), rescales by 2^-e and
//      stores y.
// The index list of the selection is written only when asked for, after y.
#include "soi_device.h"
#include "soi_host.h"
#include "soi_select.h"

namespace soi {

constexpr int kDdRowsPerWave = 1;  // output rows per wave: one, for the most workgroups per launch
constexpr int kDdWaves = 8;
constexpr int kDdThreads = kDdWaves * kWave;
constexpr int kDdMaxChannels = kDdThreads * 32;    // the selection's E <= 32 keys per thread
constexpr int kDdMaxChunks = kDdMaxChannels / 32;  // 16-byte (32-channel) chunks of a row
constexpr int kDdMaxGroups = 4;                    // 8-channel groups per thread for the coefficients
constexpr int kXcds = 8;                           // accelerator complex dies, each with its own L2
constexpr int kDdPitch = 80;                       // LDS bytes per chunk of 32 binary16 x values (64 + 16)

struct DdArgs {
    const uint16_t* gate;  // [n]
    const uint16_t* h;     // [n] fp16(silu(gate) * up)
    const uint8_t* W;      // [H, n/2]
    const float* S;        // [G, n]
    int32_t* out_idx;      // [k] or null
    int32_t* out_count;    // [1] or null
    uint16_t* y;           // [H]
    int n, k, H, gs;
};

// x values of channels 32c .. 32c+31 at LDS byte offset kDdPitch * c: with the 80-byte pitch the 16-byte reads
// of 16 lanes (chunks c .. c+15) cover the 64 banks once. RPW output rows per wave, 8 * RPW per workgroup.
template <int E, int NCH, int RPW>
__global__ __launch_bounds__(kDdThreads) void dip_dense_down_kernel(DdArgs a) {
    __shared__ uint32_t s_hist[radix_hist_offset<F16AbsValues>(F16AbsValues::kPasses)];
    __shared__ float s_max[kDdWaves];
    __shared__ uint32_t s_tot[kDdWaves];
    __shared__ float s_cmax[kDdWaves];
    __shared__ int32_t s_cut;
    __shared__ __attribute__((aligned(16))) uint8_t s_xh[kDdMaxChunks * kDdPitch];
    __shared__ __attribute__((aligned(16))) uint8_t s_xl[kDdMaxChunks * kDdPitch];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
    const int n = a.n;
    const int chunks = n >> 5;  // n % 32 == 0 (checked on the host)
    const int groups8 = n >> 3;
    // workgroups go to the 8 XCDs round-robin by linear id; tile (b % 8) * (nb / 8) + b / 8 gives XCD x the
    // consecutive tiles x * nb/8 .. (x+1) * nb/8 - 1, so the workgroups sharing a column group (and its St row)
    // mostly share one L2 instead of fetching the row once per XCD
    const int nb = gridDim.x, b = blockIdx.x;
    const int tile = (nb % kXcds == 0) ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    const int row_base = tile * (kDdWaves * RPW);
    const int g = row_base / a.gs;  // the workgroup's column group (8 * RPW divides gs)
    const int base_i = wave * kWave * E + lane;
    const u32x4* z4 = reinterpret_cast<const u32x4*>(g_zero16);

    // 1. requested first (loads return in order): the selection's gates (blocked: thread owns
    // wave*64E + 64j + lane), then the gate / h / St[g] values of the thread's 8-channel groups q = tid + 512m
    uint32_t raw[E];
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int i = base_i + j * kWave;
        raw[j] = ldg(a.gate + (i < n ? i : n - 1));
    }
    u32x4 gq[kDdMaxGroups], hq[kDdMaxGroups], sq0[kDdMaxGroups], sq1[kDdMaxGroups];
    const float* sg = a.S + static_cast<int64_t>(g) * n;
#pragma unroll
    for (int m = 0; m < kDdMaxGroups; ++m) {
        const int q = tid + m * kDdThreads;
        const bool ok = q < groups8;
        gq[m] = ldg(ok ? reinterpret_cast<const u32x4*>(a.gate) + q : z4);
        hq[m] = ldg(ok ? reinterpret_cast<const u32x4*>(a.h) + q : z4);
        sq0[m] = ldg(ok ? reinterpret_cast<const u32x4*>(sg) + 2 * q : z4);
        sq1[m] = ldg(ok ? reinterpret_cast<const u32x4*>(sg) + 2 * q + 1 : z4);
    }
    // every chunk of the wave's rows (lane takes chunks lane, lane + 64, ...)
    u32x4 wv[RPW][NCH];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row_base + wave * RPW + r;
        const u32x4* rp = reinterpret_cast<const u32x4*>(a.W + static_cast<int64_t>(row < a.H ? row : 0) * (n >> 1));
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = lane + i * kWave;
            wv[r][i] = __builtin_nontemporal_load((row < a.H && c < chunks) ? rp + c : z4);
        }
    }

    // 2. the coefficients h * St[g] of every channel (fp32, unmasked) and their largest magnitude, handed to
    // the other waves through the selection's first barrier
    float xc[kDdMaxGroups][8];
    float cmax = 0.0f;
#pragma unroll
    for (int m = 0; m < kDdMaxGroups; ++m) {
        // vector lanes are copied to scalars before the bit cast: __builtin_bit_cast applied to a lane of an
        // ext_vector value (sq0[m].y) was compiled as a cast of lane 0
        const uint32_t hw[4] = {hq[m].x, hq[m].y, hq[m].z, hq[m].w};
        const uint32_t su[8] = {sq0[m].x, sq0[m].y, sq0[m].z, sq0[m].w, sq1[m].x, sq1[m].y, sq1[m].z, sq1[m].w};
        float sv[8];
#pragma unroll
        for (int p = 0; p < 8; ++p) sv[p] = __builtin_bit_cast(float, su[p]);
#pragma unroll
        for (int p = 0; p < 8; ++p) {
            const uint16_t hb = static_cast<uint16_t>(hw[p >> 1] >> (16 * (p & 1)));
            xc[m][p] = f16_bits_to_f32(hb) * sv[p];
            cmax = fmaxf(cmax, fabsf(xc[m][p]));
        }
    }
    cmax = wave_max_bcast(cmax);
    if (lane == 0) s_cmax[wave] = cmax;

    // 3. tau and the cut; past the end the pattern is made a NaN (key 0, never selected) by a bit select
    float val[E];
    float tau;
    int32_t cut;
    uint32_t total;
    {
        uint32_t key[E];
        float local_max = 0.0f;
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const int i = base_i + j * kWave;
            const uint32_t bits = (raw[j] & 0x7fffu) | (i < n ? 0u : 0x7e00u);
            val[j] = f16_bits_to_f32(static_cast<uint16_t>(bits));
            key[j] = F16AbsValues::key_of(val[j]);
            local_max = fmaxf(local_max, val[j]);
        }
        tau = rule_a_tau<E, kDdWaves, F16AbsValues>(key, local_max, s_hist, s_max, a.k, tid);
        total = rule_a_cut<E, kDdWaves>(val, tau, a.k, s_tot, &s_cut, tid, cut);
    }

    // 4. x_g[c] = sel(c) * h_c * St[g, c] scaled by 2^e (exact; e from the largest |h * s| of all channels, a
    // bound for the selected ones) and split into binary16 hi + lo: 16-byte LDS stores per 8-channel group
    float mx = s_cmax[0];
#pragma unroll
    for (int w = 1; w < kDdWaves; ++w) mx = fmaxf(mx, s_cmax[w]);
    const int e = 15 - __builtin_amdgcn_frexp_expf(mx);  // max * 2^e < 2^15: no binary16 overflow
#pragma unroll
    for (int m = 0; m < kDdMaxGroups; ++m) {
        const int q = tid + m * kDdThreads;
        if (q < groups8) {
            const uint32_t gw[4] = {gq[m].x, gq[m].y, gq[m].z, gq[m].w};
            uint32_t hp[4], lp[4];
#pragma unroll
            for (int p2 = 0; p2 < 4; ++p2) {
                uint16_t hb[2], lb[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const int p = 2 * p2 + t;
                    const int c = 8 * q + p;
                    const uint16_t gb = static_cast<uint16_t>(gw[p2] >> (16 * t));
                    const float gv = f16_bits_to_f32(static_cast<uint16_t>(gb & 0x7fffu));
                    const bool sel = gv >= tau && c < cut;  // NaN gates are never selected
                    const float xs = sel ? __builtin_ldexpf(xc[m][p], e) : 0.0f;
                    hb[t] = f32_to_f16_bits(xs);
                    lb[t] = f32_to_f16_bits(xs - f16_bits_to_f32(hb[t]));  // exact difference
                }
                hp[p2] = static_cast<uint32_t>(hb[0]) | (static_cast<uint32_t>(hb[1]) << 16);
                lp[p2] = static_cast<uint32_t>(lb[0]) | (static_cast<uint32_t>(lb[1]) << 16);
            }
            const int off = kDdPitch * (q >> 2) + 16 * (q & 3);
            *reinterpret_cast<u32x4*>(s_xh + off) = u32x4{hp[0], hp[1], hp[2], hp[3]};
            *reinterpret_cast<u32x4*>(s_xl + off) = u32x4{lp[0], lp[1], lp[2], lp[3]};
        }
    }
    __syncthreads();

    // 5. the wave's rows: chunk by chunk, the rows share the chunk's x values
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
        const int c = lane + i * kWave;
        if (c < chunks) {
            const u32x4* ph = reinterpret_cast<const u32x4*>(s_xh + kDdPitch * c);
            const u32x4* pl = reinterpret_cast<const u32x4*>(s_xl + kDdPitch * c);
            u32x4 xh[4], xl[4];
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                xh[wd] = ph[wd];
                xl[wd] = pl[wd];
            }
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                const uint32_t wq[4] = {wv[r][i].x, wv[r][i].y, wv[r][i].z, wv[r][i].w};
                float th = 0.0f, tl = 0.0f;
#pragma unroll
                for (int wd = 0; wd < 4; ++wd) {
                    f16x2 qv[4];
                    dequant_int4x8_bitfield(wq[wd], qv);
                    const uint32_t hx[4] = {xh[wd].x, xh[wd].y, xh[wd].z, xh[wd].w};
                    const uint32_t lx[4] = {xl[wd].x, xl[wd].y, xl[wd].z, xl[wd].w};
#pragma unroll
                    for (int p = 0; p < 4; ++p) {
                        th = dot2(qv[p], as_f16x2(hx[p]), th);
                        tl = dot2(qv[p], as_f16x2(lx[p]), tl);
                    }
                }
                acc[r] += th + tl;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const float t = wave_sum_bcast(acc[r]);
        const int row = row_base + wave * RPW + r;
        if (lane == 0 && row < a.H) stg(a.y + row, f32_to_f16_bits(__builtin_ldexpf(t, -e)));
    }

    // 6. the index list when asked for (after y): workgroup b writes positions [b*win, (b+1)*win)
    const uint32_t kk = total < static_cast<uint32_t>(a.k) ? total : static_cast<uint32_t>(a.k);
    if (blockIdx.x == 0 && tid == 0 && a.out_count) stg(a.out_count, static_cast<int32_t>(kk));
    if (!a.out_idx) return;  // workgroup-uniform
    const uint32_t win = (kk + gridDim.x - 1) / gridDim.x;
    const uint32_t lo = blockIdx.x * win;
    const uint32_t hi = lo + win < kk ? lo + win : kk;
    if (lo >= hi) return;  // workgroup-uniform
    rule_a_compact<E, kDdWaves>(val, tau, s_tot, tid, lo, hi, [&](uint32_t pos, int j) {
        stg(a.out_idx + pos, static_cast<int32_t>(base_i + j * kWave));
    });
}

}  // namespace soi

using namespace soi;

extern "C" int soi_dip_select_dense_down(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                                         const uint8_t* Wt, const float* St, int32_t* out_indices,
                                         int32_t* out_count, uint16_t* y, int64_t H, int64_t group_size,
                                         int64_t num_groups, void* stream) {
    const char* what = "soi_dip_select_dense_down";
    const int64_t n = num_channels;
    SOI_REQUIRE(n >= 32 && n <= kDdMaxChannels && n % 32 == 0, "%s: num_channels must be a multiple of 32 in [32, %d]",
                what, kDdMaxChannels);
    SOI_REQUIRE(k >= 1 && k <= n, "%s: k must be in [1, num_channels]", what);
    SOI_REQUIRE(H >= 1 && H <= (int64_t(1) << 24), "%s: H out of range", what);
    SOI_REQUIRE(group_size >= kDdWaves * kDdRowsPerWave && group_size % (kDdWaves * kDdRowsPerWave) == 0,
                "%s: group_size must be a positive multiple of %d", what, kDdWaves * kDdRowsPerWave);
    SOI_REQUIRE(num_groups == ceil_div64(H, group_size), "%s: num_groups must be ceil(H / group_size)", what);
    SOI_REQUIRE(gate && h && Wt && St && y, "%s: null pointer", what);
    SOI_REQUIRE(aligned16(Wt), "%s: Wt must be 16-byte aligned", what);
    DdArgs a{gate, h, Wt, St, out_indices, out_count, y, static_cast<int>(n), static_cast<int>(k),
             static_cast<int>(H), static_cast<int>(group_size)};
    constexpr int RPW = kDdRowsPerWave;
    const dim3 grid(static_cast<unsigned>(ceil_div64(H, kDdWaves * RPW))), block(kDdThreads);
    const int64_t E = ceil_div64(n, kDdThreads);
    const int64_t nch = ceil_div64(n / 32, kWave);
    hipStream_t st = as_stream(stream);
#define SOI_DD(EE, CC) hipLaunchKernelGGL((dip_dense_down_kernel<EE, CC, RPW>), grid, block, 0, st, a)
#define SOI_DDC(EE)                       \
    do {                                  \
        if (nch <= 1) SOI_DD(EE, 1);      \
        else if (nch <= 2) SOI_DD(EE, 2); \
        else if (nch <= 3) SOI_DD(EE, 3); \
        else if (nch <= 4) SOI_DD(EE, 4); \
        else if (nch <= 6) SOI_DD(EE, 6); \
        else SOI_DD(EE, 8);               \
    } while (0)
    if (E <= 4) SOI_DDC(4);
    else if (E <= 8) SOI_DDC(8);
    else if (E <= 12) SOI_DDC(12);
    else if (E <= 16) SOI_DDC(16);
    else if (E <= 24) SOI_DDC(24);
    else SOI_DDC(32);
#undef SOI_DDC
#undef SOI_DD
    return launch_status(what);
}
