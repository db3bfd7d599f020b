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
// Workgroup = 8 waves, one output row per wave: 8 consecutive output columns
// of one column group (tiles placed XCD-aware, below). Thread t owns the
// 4-channel groups t + 512m (m < NC = n / 2048 rounded up); lane l of every
// wave owns the 32-channel chunks l + 64i (i < NC) of its row.
//   1. it requests the gate values of its groups, zeroes its share of the
//      selection's histograms and meets one barrier (every wave's gate
//      requests precede the rest: the CU returns them roughly in request
//      order), then requests the h / St[g] values of its groups and every
//      packed chunk of its row;
//   2. it forms every channel's coefficient h_c * St[g, c] in fp32 and their
//      largest magnitude (handed over through the selection's first barrier);
//   3. it runs rule A's threshold search over all n gates itself (radix
//      select and bisection replay, soi_select.h) while the row chunks land;
//   4. x_g[c] = [|gate_c| >= tau] * coefficient is scaled by a power of two
//      2^e (exact; e from the largest magnitude) and split into binary16
//      hi + lo parts in LDS (hi = fp16(x), lo = fp16(x - hi): x to ~2^-22
//      relative), and the 32-bit mask [|gate| >= tau] of every chunk goes to
//      LDS beside them (one barrier);
//   5. rule A keeps the first k channels with |gate| >= tau in index order:
//      every wave counts its lanes' chunk masks in chunk order (one wave
//      prefix sum per i), so each lane knows whether its chunk lies wholly
//      before the k-th kept channel (kept), wholly after it (skipped) or holds
//      it (the x values past it are masked off in that lane's registers);
//   6. the dot products run as v_dot2 on exact binary16 q values with fp32
//      accumulation; each wave sums over its lanes (DPP), rescales by 2^-e and
//      stores y.
// The index list of the selection is written only when asked for, after y,
// from the same chunk masks and counts.
#include <mutex>

#include "soi_device.h"
#include "soi_down.h"
#include "soi_host.h"
#include "soi_select.h"

namespace soi {


constexpr int kDdWaves = 8;  // = output rows per workgroup (one per wave)
constexpr int kDdThreads = kDdWaves * kWave;
constexpr int kDdChannelsPerPass = kDdThreads * 4;        // one 4-channel group per thread
constexpr int kDdMaxNC = 12;                              // 4-channel groups per thread (= chunks per lane)
constexpr int kDdMaxChannels = kDdChannelsPerPass * kDdMaxNC;
constexpr int kDdMaxChunks = kDdMaxChannels / 32;         // 32-channel chunks
constexpr int kXcds = 8;                                  // accelerator complex dies, each with its own L2
constexpr int kDdPitch = 80;                              // LDS bytes per chunk of 32 binary16 x values (64 + 16)

struct DdArgs {
    const uint16_t* gate;  // [n]
    const uint16_t* h;     // [n] fp16(silu(gate) * up)
    const uint8_t* W;      // [H, n/2]
    const float* S;        // [G, n]
    int32_t* out_idx;      // [k] or null
    int32_t* out_count;    // [1] or null
    uint16_t* y;           // [H]
    const uint16_t* res;   // [H] or null: the residual stream that y is added to
    uint16_t* res_out;     // [H] or null: res + y, rounded once to binary16
    int n, k, H, gs;
};

// Bit position of the r-th lowest set bit of x (1 <= r <= popcount(x)): a binary search on popcounts.
__device__ __forceinline__ int nth_set_bit(uint32_t x, uint32_t r) {
    int pos = 0;
#pragma unroll
    for (int w = 16; w >= 1; w >>= 1) {
        const uint32_t low = static_cast<uint32_t>(__builtin_popcount(x & ((1u << w) - 1u)));
        if (low < r) {
            r -= low;
            x >>= w;
            pos += w;
        }
    }
    return pos;
}

// OR over the 8 lanes 8j .. 8j+7 (quad swaps, then the 8-lane mirror); every lane of the 8 gets it.
__device__ __forceinline__ uint32_t or8_lanes(uint32_t v) {
    v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xb1, 0xf, 0xf, false));
    v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4e, 0xf, 0xf, false));
    v |= static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x141, 0xf, 0xf, false));
    return v;
}

// x values of channels 32c .. 32c+31 at LDS byte offset kDdPitch * c: with the 80-byte pitch the 16-byte reads
// of 16 lanes (chunks c .. c+15) cover the 64 banks once.
template <int NC>
__global__ __launch_bounds__(kDdThreads) void dip_dense_down_kernel(DdArgs a) {
    constexpr int E = 4 * NC;  // selection keys per thread
    __shared__ uint32_t s_hist[radix_hist_offset<F16AbsValues>(F16AbsValues::kPasses)];
    __shared__ float s_max[kDdWaves];
    __shared__ float s_cmax[kDdWaves];
    __shared__ uint32_t s_bits[kDdMaxChunks];
    __shared__ __attribute__((aligned(16))) uint8_t s_xh[kDdMaxChunks * kDdPitch];
    __shared__ __attribute__((aligned(16))) uint8_t s_xl[kDdMaxChunks * kDdPitch];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
    const int n = a.n;
    const int chunks = n >> 5;  // n % 32 == 0 (checked on the host)
    const int groups4 = n >> 2;
    // workgroups go to the 8 XCDs round-robin by linear id; tile (b % 8) * (nb / 8) + b / 8 gives XCD x the
    // consecutive tiles x * nb/8 .. (x+1) * nb/8 - 1, so the workgroups sharing a column group (and its St row)
    // mostly share one L2 instead of fetching the row once per XCD
    const int nb = gridDim.x, b = blockIdx.x;
    const int tile = (nb % kXcds == 0) ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    const int row = tile * kDdWaves + wave;
    const int g = (tile * kDdWaves) / a.gs;  // the workgroup's column group (8 divides gs)
    const u32x4* z4 = reinterpret_cast<const u32x4*>(g_zero16);
    const u32x2* z2 = reinterpret_cast<const u32x2*>(g_zero16);

    // 1. requested first (loads return in order): gate / h / St[g] of the thread's groups q = tid + 512m. Every
    // wave requests its gate words before any wave requests the rest (the barrier, which also orders the zeroed
    // histograms before the first radix pass): the requests return through the CU roughly in request order, and
    // the first radix pass needs every wave's gate
    u32x2 gq[NC], hq[NC];
    u32x4 sq[NC];
    const float* sg = a.S + static_cast<int64_t>(g) * n;
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        gq[m] = ldg(q < groups4 ? reinterpret_cast<const u32x2*>(a.gate) + q : z2);
    }
    rule_a_zero_hist<kDdWaves, F16AbsValues>(s_hist, tid);
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        const bool ok = q < groups4;
        hq[m] = ldg(ok ? reinterpret_cast<const u32x2*>(a.h) + q : z2);
        sq[m] = ldg(ok ? reinterpret_cast<const u32x4*>(sg) + q : z4);
    }
    // every chunk of the wave's row (lane takes chunks lane, lane + 64, ...)
    u32x4 wv[NC];
    {
        const u32x4* rp = reinterpret_cast<const u32x4*>(a.W + static_cast<int64_t>(row < a.H ? row : 0) * (n >> 1));
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            wv[i] = __builtin_nontemporal_load((row < a.H && c < chunks) ? rp + c : z4);
        }
    }
    // the residual element of the row (a zero word when there is none; a select, so the load is not branched)
    const uint16_t rv = ldg(a.res_out && row < a.H ? a.res + row : reinterpret_cast<const uint16_t*>(g_zero16));

    // 2. |gate| keys (NaN past the end: key 0, never counted or selected): the binary16 pattern of |g| with the
    // sign bit set (F16AbsValues::key_of of the value, formed from the bits); the largest key gives the largest
    // value
    float xc[NC][4];
    uint32_t key[E];
    uint32_t key_max = 0u;
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const bool ok = tid + m * kDdThreads < groups4;
        const uint32_t gw[2] = {gq[m].x, gq[m].y};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t gb = (gw[p >> 1] >> (16 * (p & 1))) & 0x7fffu;
            const uint32_t kv = (ok && gb <= 0x7c00u) ? (gb | 0x8000u) : 0u;
            key[4 * m + p] = kv;
            key_max = kv > key_max ? kv : key_max;
        }
    }
    const float local_max = F16AbsValues::value_of(key_max);

    // 3. tau of rule A. After its first radix pass (the h and St values have landed meanwhile): the coefficients
    // h * St[g] (fp32, unmasked) and their largest magnitude, handed to the other waves through the second pass's
    // barrier
    auto coefficients = [&]() {
        float cmax = 0.0f;
#pragma unroll
        for (int m = 0; m < NC; ++m) {
            // vector lanes are copied to scalars before the bit cast: __builtin_bit_cast applied to a lane of an
            // ext_vector value (sq[m].y) was compiled as a cast of lane 0
            const uint32_t hw[2] = {hq[m].x, hq[m].y};
            const uint32_t su[4] = {sq[m].x, sq[m].y, sq[m].z, sq[m].w};
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const uint16_t hb = static_cast<uint16_t>(hw[p >> 1] >> (16 * (p & 1)));
                xc[m][p] = f16_bits_to_f32(hb) * __builtin_bit_cast(float, su[p]);
                // finite magnitudes only: an infinite coefficient (h = +-inf) would otherwise set e = 15 and make
                // every selected coefficient >= 2 overflow in its binary16 hi part; NaN is ignored by fmaxf
                const float ax = fabsf(xc[m][p]);
                cmax = ax < __builtin_inff() ? fmaxf(cmax, ax) : cmax;
            }
        }
        cmax = wave_max_bcast(cmax);
        if (lane == 0) s_cmax[wave] = cmax;
    };
    const float tau = rule_a_tau<E, kDdWaves, F16AbsValues, true, decltype(coefficients), true>(
        key, local_max, s_hist, s_max, a.k, tid, coefficients);

    // 4. x_g[c] = [|gate_c| >= tau] * h_c * St[g, c] scaled by 2^e (exact; e from the largest finite |h * s| of
    // all channels, a bound for the selected finite ones), split into binary16 hi + lo (8-byte LDS stores per
    // group; an infinite x keeps hi = x and lo = 0, so its products are +-inf as in the fp32 sum, and NaN for
    // q = 0), and the chunk masks: lanes 8j .. 8j+7 hold the 8 groups of chunk (tid >> 3) + 64m
    float mx = s_cmax[0];
#pragma unroll
    for (int w = 1; w < kDdWaves; ++w) mx = fmaxf(mx, s_cmax[w]);
    const int e = 15 - __builtin_amdgcn_frexp_expf(mx);  // max * 2^e < 2^15: no binary16 overflow
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        uint32_t m4 = 0u;
        uint16_t hb[4], lb[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            // |g| >= tau; key 0 (NaN, padding) never
            const bool sel = key[4 * m + p] != 0u && F16AbsValues::value_of(key[4 * m + p]) >= tau;
            const float xs = sel ? __builtin_ldexpf(xc[m][p], e) : 0.0f;
            hb[p] = f32_to_f16_bits(xs);
            const float d = xs - f16_bits_to_f32(hb[p]);  // exact difference (NaN for an infinite xs)
            lb[p] = f32_to_f16_bits(fabsf(xs) < __builtin_inff() ? d : 0.0f);
            m4 |= (sel ? 1u : 0u) << p;
        }
        const uint32_t cm = or8_lanes(m4 << (4 * (lane & 7)));
        if (q < groups4) {
            const int off = kDdPitch * (q >> 3) + 8 * (q & 7);
            *reinterpret_cast<u32x2*>(s_xh + off) =
                u32x2{hb[0] | (static_cast<uint32_t>(hb[1]) << 16), hb[2] | (static_cast<uint32_t>(hb[3]) << 16)};
            *reinterpret_cast<u32x2*>(s_xl + off) =
                u32x2{lb[0] | (static_cast<uint32_t>(lb[1]) << 16), lb[2] | (static_cast<uint32_t>(lb[3]) << 16)};
            if ((lane & 7) == 0) s_bits[q >> 3] = cm;
        }
    }
    __syncthreads();

    // 5. the first k channels with |gate| >= tau, chunk by chunk in index order (i-major, then lane):
    // before[i] = kept channels of all earlier chunks, keep[i] = channels of the lane's chunk i that stay
    // (0: none, 32: all; else the chunk holds the k-th kept channel and channels >= keep[i] are dropped)
    const uint32_t k = static_cast<uint32_t>(a.k);
    uint32_t total = 0u;
    uint32_t before[NC], bits[NC];
    int keep[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + i * kWave;
        bits[i] = c < chunks ? s_bits[c] : 0u;
        const uint32_t cnt = static_cast<uint32_t>(__builtin_popcount(bits[i]));
        const uint32_t incl = wave_prefix_u32(cnt);
        before[i] = total + incl - cnt;
        total += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1));
        keep[i] = before[i] >= k ? 0 : (before[i] + cnt <= k ? 32 : nth_set_bit(bits[i], k - before[i]) + 1);
    }

    // 6. the wave's row
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + i * kWave;
        if (c < chunks && keep[i] > 0) {
            const u32x4* ph = reinterpret_cast<const u32x4*>(s_xh + kDdPitch * c);
            const u32x4* pl = reinterpret_cast<const u32x4*>(s_xl + kDdPitch * c);
            uint32_t hx[16], lx[16];
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const u32x4 vh = ph[wd], vl = pl[wd];
                hx[4 * wd] = vh.x, hx[4 * wd + 1] = vh.y, hx[4 * wd + 2] = vh.z, hx[4 * wd + 3] = vh.w;
                lx[4 * wd] = vl.x, lx[4 * wd + 1] = vl.y, lx[4 * wd + 2] = vl.z, lx[4 * wd + 3] = vl.w;
            }
            if (keep[i] < 32) {  // the chunk holding the k-th kept channel: channels >= keep[i] dropped
#pragma unroll
                for (int w = 0; w < 16; ++w) {
                    const uint32_t mk = (2 * w < keep[i] ? 0x0000ffffu : 0u) | (2 * w + 1 < keep[i] ? 0xffff0000u : 0u);
                    hx[w] &= mk;
                    lx[w] &= mk;
                }
            }
            const uint32_t wq[4] = {wv[i].x, wv[i].y, wv[i].z, wv[i].w};
            float th = 0.0f, tl = 0.0f;
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                f16x2 qv[4];
                dequant_int4x8_bitfield(wq[wd], qv);
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    th = dot2(qv[p], as_f16x2(hx[4 * wd + p]), th);
                    tl = dot2(qv[p], as_f16x2(lx[4 * wd + p]), tl);
                }
            }
            acc += th + tl;
        }
    }
    {
        const float t = wave_sum_bcast(acc);
        if (lane == 0 && row < a.H) {
            const uint16_t yb = f32_to_f16_bits(__builtin_ldexpf(t, -e));
            stg(a.y + row, yb);
            if (a.res_out) stg(a.res_out + row, static_cast<uint16_t>(add_f16x2(rv, yb)));
        }
    }

    // 7. the index list when asked for (after y), by wave 0: workgroup b writes positions [b*win, (b+1)*win)
    const uint32_t kk = total < k ? total : k;
    if (b == 0 && tid == 0 && a.out_count) stg(a.out_count, static_cast<int32_t>(kk));
    if (!a.out_idx || wave != 0) return;  // wave-uniform
    const uint32_t win = (kk + nb - 1) / nb;
    const uint32_t lo = b * win;
    const uint32_t hi = lo + win < kk ? lo + win : kk;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + i * kWave;
        uint32_t x = keep[i] >= 32 ? bits[i] : (bits[i] & ((1u << keep[i]) - 1u));
        uint32_t pos = before[i];
        if (c >= chunks || pos >= hi || pos + static_cast<uint32_t>(__builtin_popcount(x)) <= lo) continue;
        while (x != 0u) {
            if (pos >= lo && pos < hi) stg(a.out_idx + pos, static_cast<int32_t>(32 * c + __builtin_ctz(x)));
            ++pos;
            x &= x - 1u;
        }
    }
}

// ---------------------------------------------------------------------------
// The selection + down in the sparse accumulate's own order, over the
// transposed copy (soi_dip_select_down_ordered).
//
// y equals the top-k launch followed by the sparse down over the selected
// channels' h values (soi_gemv_w4a16_indexed_accumulate with h_sel =
// h[idx]) bit for bit, with no cross-workgroup step: each wave owns one
// output column, as in the dense down above, and replays the sparse down's
// summation for it. That kernel (soi_down.h) splits the k selected positions
// into R row chunks of rpc positions (down_plan for (H, k)); inside chunk r,
// the sub-partial g = 8w + rs of its (wave w, row lane rs) is the fma chain
// acc = fma(coef_p, q_p, acc) over the positions p = r*rpc + g + 32i <
// min((r+1)*rpc, kept) in ascending i, from acc = 0; the chunk's partial is
// 0 + sub_0 + sub_1 + ... + sub_31 in that order, and y = 0 + partial_0 + ...
// + partial_{R-1}. Here coef_p = fl(h_c * St[g, c]) with c the p-th kept
// channel, and q_p the exact INT4 value of channel c in the column's
// transposed row: the same products in the same order.
//   1. the thread of 4-channel group q requests the gate words of its
//      channels; one barrier (after the histograms are zeroed) so every
//      wave's gate requests precede the rest; then h and St[g] of its
//      channels, and every lane its row chunks (as the dense down);
//   2. rule A's threshold over |gate| (the coefficients fl(h * s) are formed
//      after the first radix pass);
//   3. the chunk masks [|gate| >= tau] and each wave's packed row go to LDS
//      (one barrier); each thread finds the positions of its selected
//      channels from the chunk prefix counts and writes (coef, location of
//      the channel's nibble in a row) per position p < k (one barrier);
//   4. thread t runs chain (r, g) = (t / 32, t % 32) (then t + 512, ...) for
//      all 8 rows of the workgroup, two positions per step: one read of two
//      table entries feeds 16 row-byte reads (a signed bitfield extract gives
//      q) and 8 accumulators; then each wave's ordered sums: lane r sums chunk
//      r's 32 sub-partials, and the chunk partials are summed in order; y and
//      optionally res + y (one binary16 add) are stored.
// Limits: R <= 64 row chunks, and the tables (8k + 8 * 1024 * ceil(n / 2048)
// + 8 * 144 * R bytes) within kOdMaxLds of LDS.
// ---------------------------------------------------------------------------
constexpr int kOdMaxR = 64;
constexpr int kOdMaxLds = 144 * 1024;
constexpr int kOdSubPitch = 36;  // floats per (wave, chunk) row of sub-partials: 32 + 4 of padding

// The 4-bit field of b at bit sh, sign-extended (v_bfe_i32): the exact INT4
// value q, as a float. The builtin's result type is unsigned, so it is read as
// int before the conversion (an unsigned conversion would turn -1 into 2^32).
__device__ __forceinline__ float s4_field(int b, int sh) {
    return static_cast<float>(static_cast<int>(__builtin_amdgcn_sbfe(b, sh, 4)));
}

struct OdArgs {
    const uint16_t* gate;  // [n]
    const uint16_t* h;     // [n] fp16(silu(gate) * up)
    const uint8_t* W;      // [H, n/2]
    const float* S;        // [G, n]
    int32_t* out_idx;      // [k] or null
    int32_t* out_count;    // [1] or null
    uint16_t* y;           // [H]
    const uint16_t* res;   // [H] or null
    uint16_t* res_out;     // [H] or null: res + y, rounded once to binary16
    int n, k, H, gs, rpc, R;
    int pos_bytes;  // LDS: position table (8 bytes per position, rounded to 16); then 8 packed rows, NC KB apart
};

template <int NC>
__global__ __launch_bounds__(kDdThreads) void dip_down_ordered_kernel(OdArgs a) {
    constexpr int E = 4 * NC;
    __shared__ uint32_t s_hist[radix_hist_offset<F16AbsValues>(F16AbsValues::kPasses)];
    __shared__ float s_max[kDdWaves];
    __shared__ uint32_t s_bits[kDdMaxChunks];
    extern __shared__ __attribute__((aligned(16))) uint8_t s_dyn[];
    const int n = a.n;
    u32x2* s_pos = reinterpret_cast<u32x2*>(s_dyn);  // per position: coef bits, byte of the row | nibble shift << 16
    // row w (packed, n / 2 bytes) at w * RS: a compile-time stride, so each row read takes its row's offset
    // in the LDS instruction's immediate field instead of an address add
    constexpr int RS = NC * (kDdChannelsPerPass / 2);
    uint8_t* s_row = s_dyn + a.pos_bytes;
    // sub-partials [wave][r][kOdSubPitch]: lane r of the in-order sums reads its chunk's 32 values as 8 16-byte
    // words, and the 36-float pitch puts the lanes' words in distinct LDS banks
    float* s_sub = reinterpret_cast<float*>(s_dyn + a.pos_bytes + kDdWaves * RS);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
    const int chunks = n >> 5;  // n % 32 == 0 (checked on the host)
    const int groups4 = n >> 2;
    const int nb = gridDim.x, b = blockIdx.x;
    const int tile = (nb % kXcds == 0) ? (b % kXcds) * (nb / kXcds) + b / kXcds : b;
    const int row = tile * kDdWaves + wave;
    const int g = (tile * kDdWaves) / a.gs;
    const u32x4* z4 = reinterpret_cast<const u32x4*>(g_zero16);
    const u32x2* z2 = reinterpret_cast<const u32x2*>(g_zero16);

    // 1. gate first, then h and St[g], then the row chunks (loads return in order). Every wave requests its gate
    // words before any wave requests the rest (the barrier): the workgroup's 72 KB (n = 6144) of requests return
    // through the CU roughly in request order, and the first radix pass needs every wave's gate
    u32x2 gq[NC], hq[NC];
    u32x4 sq[NC];
    const float* sg = a.S + static_cast<int64_t>(g) * n;
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        gq[m] = ldg(q < groups4 ? reinterpret_cast<const u32x2*>(a.gate) + q : z2);
    }
    rule_a_zero_hist<kDdWaves, F16AbsValues>(s_hist, tid);
    __syncthreads();  // also orders the zeroed histograms before the first radix pass
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        const bool ok = q < groups4;
        hq[m] = ldg(ok ? reinterpret_cast<const u32x2*>(a.h) + q : z2);
        sq[m] = ldg(ok ? reinterpret_cast<const u32x4*>(sg) + q : z4);
    }
    u32x4 wv[NC];
    {
        const u32x4* rp = reinterpret_cast<const u32x4*>(a.W + static_cast<int64_t>(row < a.H ? row : 0) * (n >> 1));
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            wv[i] = __builtin_nontemporal_load((row < a.H && c < chunks) ? rp + c : z4);
        }
    }
    const uint16_t rv = ldg(a.res_out && row < a.H ? a.res + row : reinterpret_cast<const uint16_t*>(g_zero16));

    // 2. |gate| keys (NaN past the end: key 0, never counted or selected) and rule A's threshold; after the first
    // radix pass, the coefficients fl(h * St[g]). The key of |g| is its binary16 pattern with the sign bit set
    // (F16AbsValues::key_of of the value, formed from the bits), and the largest key gives the largest value
    float xc[NC][4];
    uint32_t key[E];
    uint32_t key_max = 0u;
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const bool ok = tid + m * kDdThreads < groups4;
        const uint32_t gw[2] = {gq[m].x, gq[m].y};
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t gb = (gw[p >> 1] >> (16 * (p & 1))) & 0x7fffu;
            const uint32_t kv = (ok && gb <= 0x7c00u) ? (gb | 0x8000u) : 0u;
            key[4 * m + p] = kv;
            key_max = kv > key_max ? kv : key_max;
        }
    }
    const float local_max = F16AbsValues::value_of(key_max);
    auto coefficients = [&]() {
#pragma unroll
        for (int m = 0; m < NC; ++m) {
            // vector lanes copied to scalars before any bit cast (see the dense down)
            const uint32_t hw[2] = {hq[m].x, hq[m].y};
            const uint32_t su[4] = {sq[m].x, sq[m].y, sq[m].z, sq[m].w};
#pragma unroll
            for (int p = 0; p < 4; ++p)
                xc[m][p] = f16_bits_to_f32(static_cast<uint16_t>(hw[p >> 1] >> (16 * (p & 1)))) *
                           __builtin_bit_cast(float, su[p]);
        }
    };
    const float tau = rule_a_tau<E, kDdWaves, F16AbsValues, true, decltype(coefficients), true>(
        key, local_max, s_hist, s_max, a.k, tid, coefficients);

    // 3. chunk masks (lanes 8j .. 8j+7 hold the 8 groups of chunk (tid >> 3) + 64m, and each of them keeps the
    // chunk's mask for the position table) and the wave's packed row
    uint32_t cmask[NC];
#pragma unroll
    for (int m = 0; m < NC; ++m) {
        const int q = tid + m * kDdThreads;
        uint32_t m4 = 0u;
#pragma unroll
        for (int p = 0; p < 4; ++p)  // |g| >= tau; key 0 (NaN, padding) never
            m4 |= (key[4 * m + p] != 0u && F16AbsValues::value_of(key[4 * m + p]) >= tau ? 1u : 0u) << p;
        cmask[m] = or8_lanes(m4 << (4 * (lane & 7)));
        if (q < groups4 && (lane & 7) == 0) s_bits[q >> 3] = cmask[m];
    }
    {
        uint8_t* my_row = s_row + wave * RS;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = lane + i * kWave;
            if (c < chunks) *reinterpret_cast<u32x4*>(my_row + 16 * c) = wv[i];
        }
    }
    __syncthreads();

    // kept channels of the earlier chunks, chunk by chunk in index order (lane l: chunks l + 64i; all NC words
    // requested at once: lane + 64i < 64 NC <= kDdMaxChunks, words past the chunks read but not used)
    const uint32_t k = static_cast<uint32_t>(a.k);
    uint32_t total = 0u;
    uint32_t before[NC], bits[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) bits[i] = s_bits[lane + i * kWave];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + i * kWave;
        bits[i] = c < chunks ? bits[i] : 0u;
        const uint32_t cnt = static_cast<uint32_t>(__builtin_popcount(bits[i]));
        const uint32_t incl = wave_prefix_u32(cnt);
        before[i] = total + incl - cnt;
        total += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1));
    }
    const uint32_t kk = total < k ? total : k;
    // the position table: group q = tid + 512m lies in chunk (tid >> 3) + 64m, whose count of earlier kept
    // channels this wave's lane 8 * wave + (lane >> 3) holds at index m; the group's channels sit at bits
    // 4 (lane & 7) .. + 3 of the chunk's mask
    {
        const int src = 8 * wave + (lane >> 3);
        const uint32_t sh = 4u * static_cast<uint32_t>(lane & 7);
#pragma unroll
        for (int m = 0; m < NC; ++m) {
            const uint32_t cb = cmask[m];
            uint32_t pos = static_cast<uint32_t>(__shfl(static_cast<int>(before[m]), src, kWave)) +
                           static_cast<uint32_t>(__builtin_popcount(cb & ((1u << sh) - 1u)));
            // AWQ order: logical element j of a word sits at nibble (j >> 1) + 4 (j & 1). The group's channels
            // 4t .. 4t + 3 (t = q) are elements 4 (t & 1) + p of word t >> 1: nibble 2 (t & 1) + (p >> 1) + 4 (p & 1),
            // i.e. byte 4 (t >> 1) + (t & 1) + 2 (p & 1) of the row, shift 4 (p >> 1)
            const uint32_t t = static_cast<uint32_t>(tid + m * kDdThreads);
            const uint32_t byte0 = 4u * (t >> 1) + (t & 1u);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const bool on = ((cb >> (sh + static_cast<uint32_t>(p))) & 1u) != 0u;
                if (on && pos < k) {
                    const uint32_t loc = (byte0 + 2u * static_cast<uint32_t>(p & 1)) |
                                         ((4u * static_cast<uint32_t>(p >> 1)) << 16);
                    s_pos[pos] = u32x2{__builtin_bit_cast(uint32_t, xc[m][p]), loc};
                }
                pos += on ? 1u : 0u;
            }
        }
    }
    __syncthreads();

    // 4. the chains: thread t takes chain (r, gsub) = (t / 32, t % 32), then t + 512, ..., for all 8 rows of the
    // workgroup at once (sparse-down wave gsub >> 3 and row lane gsub & 7 read positions r * rpc + gsub + 32i)
    const int R = a.R, rpc = a.rpc;
    for (int cn = tid; cn < R * 32; cn += kDdThreads) {
        const int r = cn >> 5, gsub = cn & 31;
        const int j0 = r * rpc;
        const int j1 = j0 + rpc < static_cast<int>(kk) ? j0 + rpc : static_cast<int>(kk);
        float acc[kDdWaves];
#pragma unroll
        for (int w = 0; w < kDdWaves; ++w) acc[w] = 0.0f;
        // two positions per step (p, then p + 32: the chain's order), both entries and all 16 row bytes
        // requested before the first fma
        int p = j0 + gsub;
        for (; p + 32 < j1; p += 64) {
            const u32x2 e0 = s_pos[p], e1 = s_pos[p + 32];
            const int o0 = static_cast<int>(e0.y & 0xffffu), h0 = static_cast<int>(e0.y >> 16);
            const int o1 = static_cast<int>(e1.y & 0xffffu), h1 = static_cast<int>(e1.y >> 16);
            int b0[kDdWaves], b1[kDdWaves];
#pragma unroll
            for (int w = 0; w < kDdWaves; ++w) {
                b0[w] = s_row[w * RS + o0];
                b1[w] = s_row[w * RS + o1];
            }
            const float c0 = __builtin_bit_cast(float, e0.x), c1 = __builtin_bit_cast(float, e1.x);
#pragma unroll
            for (int w = 0; w < kDdWaves; ++w) acc[w] = fmaf(c0, s4_field(b0[w], h0), acc[w]);
#pragma unroll
            for (int w = 0; w < kDdWaves; ++w) acc[w] = fmaf(c1, s4_field(b1[w], h1), acc[w]);
        }
        if (p < j1) {
            const u32x2 e = s_pos[p];
            const float cf = __builtin_bit_cast(float, e.x);
            const int off = static_cast<int>(e.y & 0xffffu), sh = static_cast<int>(e.y >> 16);
#pragma unroll
            for (int w = 0; w < kDdWaves; ++w)
                acc[w] = fmaf(cf, s4_field(s_row[w * RS + off], sh), acc[w]);
        }
#pragma unroll
        for (int w = 0; w < kDdWaves; ++w) s_sub[(w * R + r) * kOdSubPitch + gsub] = acc[w];
    }
    __syncthreads();
    float part = 0.0f;
    if (lane < R) {
        const float4* src = reinterpret_cast<const float4*>(s_sub + (wave * R + lane) * kOdSubPitch);
        float4 v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[j];
#pragma unroll
        for (int j = 0; j < 8; ++j) part = (((part + v[j].x) + v[j].y) + v[j].z) + v[j].w;
    }
    float sum = 0.0f;
    for (int r = 0; r < R; ++r)
        sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, part), r));
    if (lane == 0 && row < a.H) {
        const uint16_t yb = f32_to_f16_bits(sum);
        stg(a.y + row, yb);
        if (a.res_out) stg(a.res_out + row, static_cast<uint16_t>(add_f16x2(rv, yb)));
    }

    // 5. the index list when asked for (after y), by wave 0: workgroup b writes positions [b*win, (b+1)*win)
    if (b == 0 && tid == 0 && a.out_count) stg(a.out_count, static_cast<int32_t>(kk));
    if (!a.out_idx || wave != 0) return;  // wave-uniform
    const uint32_t win = (kk + nb - 1) / nb;
    const uint32_t lo = b * win;
    const uint32_t hi = lo + win < kk ? lo + win : kk;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + i * kWave;
        const int keep = before[i] >= k ? 0
                         : (before[i] + static_cast<uint32_t>(__builtin_popcount(bits[i])) <= k
                                ? 32
                                : nth_set_bit(bits[i], k - before[i]) + 1);
        uint32_t x = keep >= 32 ? bits[i] : (bits[i] & ((1u << keep) - 1u));
        uint32_t pos = before[i];
        if (c >= chunks || pos >= hi || pos + static_cast<uint32_t>(__builtin_popcount(x)) <= lo) continue;
        while (x != 0u) {
            if (pos >= lo && pos < hi) stg(a.out_idx + pos, static_cast<int32_t>(32 * c + __builtin_ctz(x)));
            ++pos;
            x &= x - 1u;
        }
    }
}

}  // namespace soi

using namespace soi;

static int dense_down(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k, const uint8_t* Wt,
                      const float* St, int32_t* out_indices, int32_t* out_count, uint16_t* y, const uint16_t* res,
                      uint16_t* res_out, int64_t H, int64_t group_size, int64_t num_groups, void* stream,
                      const char* what) {
    const int64_t n = num_channels;
    SOI_REQUIRE(n >= 32 && n <= kDdMaxChannels && n % 32 == 0, "%s: num_channels must be a multiple of 32 in [32, %d]",
                what, kDdMaxChannels);
    SOI_REQUIRE(k >= 1 && k <= n, "%s: k must be in [1, num_channels]", what);
    SOI_REQUIRE(H >= 1 && H <= (int64_t(1) << 24), "%s: H out of range", what);
    SOI_REQUIRE(group_size >= kDdWaves && group_size % kDdWaves == 0, "%s: group_size must be a positive multiple of %d",
                what, kDdWaves);
    SOI_REQUIRE(num_groups == ceil_div64(H, group_size), "%s: num_groups must be ceil(H / group_size)", what);
    SOI_REQUIRE(gate && h && Wt && St && y, "%s: null pointer", what);
    SOI_REQUIRE(aligned16(Wt) && aligned16(St), "%s: Wt and St must be 16-byte aligned", what);
    SOI_REQUIRE((reinterpret_cast<uintptr_t>(gate) & 7u) == 0 && (reinterpret_cast<uintptr_t>(h) & 7u) == 0,
                "%s: gate and h must be 8-byte aligned", what);
    DdArgs a{gate, h, Wt, St, out_indices, out_count, y, res, res_out, static_cast<int>(n), static_cast<int>(k),
             static_cast<int>(H), static_cast<int>(group_size)};
    const dim3 grid(static_cast<unsigned>(ceil_div64(H, kDdWaves))), block(kDdThreads);
    const int64_t nc = ceil_div64(n, kDdChannelsPerPass);
    hipStream_t st = as_stream(stream);
#define SOI_DD(NN) hipLaunchKernelGGL((dip_dense_down_kernel<NN>), grid, block, 0, st, a)
    switch (nc) {
        case 1: SOI_DD(1); break;
        case 2: SOI_DD(2); break;
        case 3: SOI_DD(3); break;
        case 4: SOI_DD(4); break;
        case 5: SOI_DD(5); break;
        case 6: SOI_DD(6); break;
        case 7: SOI_DD(7); break;
        case 8: SOI_DD(8); break;
        case 9: SOI_DD(9); break;
        case 10: SOI_DD(10); break;
        case 11: SOI_DD(11); break;
        default: SOI_DD(12); break;
    }
#undef SOI_DD
    return launch_status(what);
}

extern "C" int soi_dip_select_dense_down(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                                         const uint8_t* Wt, const float* St, int32_t* out_indices,
                                         int32_t* out_count, uint16_t* y, int64_t H, int64_t group_size,
                                         int64_t num_groups, void* stream) {
    return dense_down(gate, h, num_channels, k, Wt, St, out_indices, out_count, y, nullptr, nullptr, H, group_size,
                      num_groups, stream, "soi_dip_select_dense_down");
}

extern "C" int soi_dip_select_dense_down_residual(const uint16_t* gate, const uint16_t* h, int64_t num_channels,
                                                  int64_t k, const uint8_t* Wt, const float* St,
                                                  int32_t* out_indices, int32_t* out_count, uint16_t* y,
                                                  const uint16_t* res, uint16_t* res_out, int64_t H,
                                                  int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_dip_select_dense_down_residual";
    SOI_REQUIRE(res && res_out, "%s: null pointer", what);
    return dense_down(gate, h, num_channels, k, Wt, St, out_indices, out_count, y, res, res_out, H, group_size,
                      num_groups, stream, what);
}

// LDS of the ordered down for (H, n, k): the position table, the 8 packed rows and the chains' sub-partials;
// 0 when the shape is outside the kernel's limits.
static size_t ordered_lds(int64_t H, int64_t n, int64_t k, DownPlan* plan) {
    if (H < 1 || n < 32 || n % 32 != 0 || n > kDdMaxChannels || k < 1 || k > n) return 0;
    const DownPlan p = down_plan(H, k);
    if (p.R > kOdMaxR) return 0;
    const size_t pos = (static_cast<size_t>(k) * 8 + 15) / 16 * 16;
    const size_t row_stride = static_cast<size_t>(ceil_div64(n, kDdChannelsPerPass)) * (kDdChannelsPerPass / 2);
    const size_t lds = pos + static_cast<size_t>(kDdWaves) * row_stride +
                       static_cast<size_t>(kDdWaves) * static_cast<size_t>(p.R) * kOdSubPitch * sizeof(float);
    if (lds > static_cast<size_t>(kOdMaxLds)) return 0;
    if (plan) *plan = p;
    return lds;
}

// The ordered kernels may take more than 64 KB of dynamic LDS: the limit is raised to kOdMaxLds once per device
// and instantiation (the first call on a device; launches below the limit need nothing more).
constexpr int kOdMaxDevices = 64;
static std::mutex g_od_mu;
static bool g_od_attr[kOdMaxDevices][kDdMaxNC + 1] = {};

template <int NN>
static int ordered_lds_limit(const char* what) {
    int dev = -1;
    SOI_HIP_TRY(hipGetDevice(&dev), what);
    SOI_REQUIRE(dev >= 0 && dev < kOdMaxDevices, "%s: device %d out of range", what, dev);
    std::lock_guard<std::mutex> lock(g_od_mu);
    if (!g_od_attr[dev][NN]) {
        SOI_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(&dip_down_ordered_kernel<NN>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kOdMaxLds),
                    what);
        g_od_attr[dev][NN] = true;
    }
    return SOI_OK;
}

extern "C" size_t soi_dip_select_down_ordered_lds_bytes(int64_t H, int64_t num_channels, int64_t k) {
    return ordered_lds(H, num_channels, k, nullptr);
}

extern "C" int soi_dip_select_down_ordered(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                                           const uint8_t* Wt, const float* St, int32_t* out_indices,
                                           int32_t* out_count, uint16_t* y, const uint16_t* res, uint16_t* res_out,
                                           int64_t H, int64_t group_size, int64_t num_groups, void* stream) {
    const char* what = "soi_dip_select_down_ordered";
    const int64_t n = num_channels;
    SOI_REQUIRE(n >= 32 && n <= kDdMaxChannels && n % 32 == 0, "%s: num_channels must be a multiple of 32 in [32, %d]",
                what, kDdMaxChannels);
    SOI_REQUIRE(k >= 1 && k <= n, "%s: k must be in [1, num_channels]", what);
    SOI_REQUIRE(H >= 1 && H <= (int64_t(1) << 24), "%s: H out of range", what);
    SOI_REQUIRE(group_size >= kDdWaves && group_size % kDdWaves == 0, "%s: group_size must be a positive multiple of %d",
                what, kDdWaves);
    SOI_REQUIRE(num_groups == ceil_div64(H, group_size), "%s: num_groups must be ceil(H / group_size)", what);
    SOI_REQUIRE(gate && h && Wt && St && y, "%s: null pointer", what);
    SOI_REQUIRE(!res_out || res, "%s: res_out needs res", what);
    SOI_REQUIRE(aligned16(Wt) && aligned16(St), "%s: Wt and St must be 16-byte aligned", what);
    SOI_REQUIRE((reinterpret_cast<uintptr_t>(gate) & 7u) == 0 && (reinterpret_cast<uintptr_t>(h) & 7u) == 0,
                "%s: gate and h must be 8-byte aligned", what);
    DownPlan p{};
    const size_t lds = ordered_lds(H, n, k, &p);
    SOI_REQUIRE(lds > 0, "%s: H = %lld, k = %lld: the sparse down's plan has more than %d row chunks or the tables "
                "need more than %d bytes of LDS; use the top-k kernel and the sparse down", what, (long long)H,
                (long long)k, kOdMaxR, kOdMaxLds);
    OdArgs a{gate, h, Wt, St, out_indices, out_count, y, res, res_out, static_cast<int>(n), static_cast<int>(k),
             static_cast<int>(H), static_cast<int>(group_size), static_cast<int>(p.rpc), static_cast<int>(p.R),
             static_cast<int>((static_cast<size_t>(k) * 8 + 15) / 16 * 16)};
    const dim3 grid(static_cast<unsigned>(ceil_div64(H, kDdWaves))), block(kDdThreads);
    const int64_t nc = ceil_div64(n, kDdChannelsPerPass);
    hipStream_t st = as_stream(stream);
    const unsigned sh = static_cast<unsigned>(lds);
#define SOI_OD(NN)                                                                                             \
    do {                                                                                                       \
        const int ls = ordered_lds_limit<NN>(what);                                                            \
        if (ls) return ls;                                                                                     \
        hipLaunchKernelGGL((dip_down_ordered_kernel<NN>), grid, block, sh, st, a);                             \
    } while (0)
    switch (nc) {
        case 1: SOI_OD(1); break;
        case 2: SOI_OD(2); break;
        case 3: SOI_OD(3); break;
        case 4: SOI_OD(4); break;
        case 5: SOI_OD(5); break;
        case 6: SOI_OD(6); break;
        case 7: SOI_OD(7); break;
        case 8: SOI_OD(8); break;
        case 9: SOI_OD(9); break;
        case 10: SOI_OD(10); break;
        case 11: SOI_OD(11); break;
        default: SOI_OD(12); break;
    }
#undef SOI_OD
    return launch_status(what);
}
