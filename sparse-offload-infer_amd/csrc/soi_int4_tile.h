// The INT4 dequant-GEMV tile shared by the GEMV kernels (gemv_int4.hip) and
// the o projection that combines split attention states on load
// (decode_attention.hip): x sources, epilogues and gemv_int4_tile, which computes R rows of y = W x per wave with fp32
// accumulation in a fixed order. Every kernel built on it returns the same
// row totals for the same logical rows and x, whatever the tile height.
#pragma once

#include "soi_device.h"
#include "soi_rows.h"

namespace soi {

template <bool BITFIELD>
__device__ __forceinline__ void nibble_pairs(uint32_t w, f16x2 lo[2], f16x2 hi[2]) {
    if (BITFIELD)
        int4x8_subnormal_bitfield(w, lo, hi);
    else
        int4x8_subnormal_scalar(w, lo, hi);
}

// sum q*x of one word's 8 values from its subnormal pairs and sum(x) (see soi_device.h)
constexpr float kTwo24 = 16777216.0f;
constexpr float kTwo20 = 1048576.0f;

// Loads are unconditional and go through the global address space. With FULL
// (every row exists and every lane of every pass has a chunk: N % R == 0 and
// chunks % 64 == 0, true for all Qwen3 shapes) there are no guards at all:
// row pointers stay wave-uniform (SGPR base + lane offset). Otherwise a lane
// or row with nothing to read loads from g_zero16 instead (address select, no
// branch), contributing exact zeros.

template <bool VEC, bool FULL>
__device__ __forceinline__ void load_w_chunk(const uint8_t* __restrict__ row, bool ok, int words, int c,
                                             uint32_t wv[4]) {
    const uint32_t* z = g_zero16;
    if (VEC) {
        const u32x4* p = reinterpret_cast<const u32x4*>(row) + c;
        if (!FULL) p = ok ? p : reinterpret_cast<const u32x4*>(z);
        const u32x4 t = ldg_stream(p);  // weights are read once: non-temporal
        wv[0] = t.x;
        wv[1] = t.y;
        wv[2] = t.z;
        wv[3] = t.w;
    } else {
        const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int wi = 4 * c + i;
            wv[i] = ldg((ok && wi < words) ? rw + wi : z);
        }
    }
}

template <bool VEC, bool FULL>
__device__ __forceinline__ void load_x_chunk(const uint16_t* __restrict__ x, int K, int c, bool cv, f16x2 xv[16]) {
    const int k0 = 32 * c;
    if (VEC) {  // K % 32 == 0: a valid chunk is fully inside x
        const u32x4* z = reinterpret_cast<const u32x4*>(g_zero16);
        const u32x4* xp = reinterpret_cast<const u32x4*>(x + k0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 t = ldg(FULL ? xp + i : (cv ? xp + i : z));
            xv[4 * i + 0] = as_f16x2(t.x);
            xv[4 * i + 1] = as_f16x2(t.y);
            xv[4 * i + 2] = as_f16x2(t.z);
            xv[4 * i + 3] = as_f16x2(t.w);
        }
    } else {
        const uint16_t* z = reinterpret_cast<const uint16_t*>(g_zero16);
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int ka = k0 + 2 * e, kb = ka + 1;
            const uint32_t lo = ldg((cv && ka < K) ? x + ka : z);
            const uint32_t hi = ldg((cv && kb < K) ? x + kb : z);
            xv[e] = as_f16x2(lo | (hi << 16));
        }
    }
}

// x sources. PlainX: x as given. NormX: x = rmsnorm(a (+ d), w) computed on
// load, with inv = 1/sqrt(mean((a+d)^2) + eps) precomputed by the workgroup:
// element h = fp16(fp16(a + d) * inv * w), the rounding points of the separate
// residual add and RMSNorm (VEC only: K % 32 == 0, 16-byte aligned vectors).
// base(): a K-element fp16 vector (2K bytes), a legal read target for a row
// that cannot be resolved (its K/2 packed bytes and K/gs scales fit in it).
struct PlainX {
    static constexpr bool kSinglePass = false;
    const uint16_t* x;
    __device__ __forceinline__ const uint16_t* base() const { return x; }
    template <bool VEC, bool FULL>
    __device__ __forceinline__ void load(int K, int c, bool cv, f16x2 xv[16]) const {
        load_x_chunk<VEC, FULL>(x, K, c, cv, xv);
    }
};

struct NormX {
    static constexpr bool kSinglePass = false;
    const uint16_t* a;
    const uint16_t* d;  // may be null
    const uint16_t* w;
    float inv;
    __device__ __forceinline__ const uint16_t* base() const { return a; }
    template <bool VEC, bool FULL>
    __device__ __forceinline__ void load(int, int c, bool cv, f16x2 xv[16]) const {
        const u32x4* z = reinterpret_cast<const u32x4*>(g_zero16);
        const u32x4* a4 = reinterpret_cast<const u32x4*>(a) + 4 * c;
        const u32x4* d4 = reinterpret_cast<const u32x4*>(d) + 4 * c;
        const u32x4* w4 = reinterpret_cast<const u32x4*>(w) + 4 * c;
        const bool ok = FULL || cv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4 t = ldg(ok ? a4 + i : z);
            if (d) {
                const u32x4 e = ldg(ok ? d4 + i : z);
                t.x = add_f16x2(t.x, e.x);
                t.y = add_f16x2(t.y, e.y);
                t.z = add_f16x2(t.z, e.z);
                t.w = add_f16x2(t.w, e.w);
            }
            const u32x4 g = ldg(ok ? w4 + i : z);
            xv[4 * i + 0] = as_f16x2(norm_f16x2(t.x, g.x, inv));
            xv[4 * i + 1] = as_f16x2(norm_f16x2(t.y, g.y, inv));
            xv[4 * i + 2] = as_f16x2(norm_f16x2(t.z, g.z, inv));
            xv[4 * i + 3] = as_f16x2(norm_f16x2(t.w, g.w, inv));
        }
    }
};

// RegNormX (K == 2048 with one pass: lane l's GEMV chunk is elements
// 32l..32l+31): the lane's chunks of a, d and the norm weight w are loaded
// into registers before the tile issues its weight loads, and load() does
// the residual add, the RMSNorm (one wave reduction) and, when x_out / h_out
// are given (workgroup 0 only), their stores. So the norm's arithmetic runs
// while the weight loads are in flight instead of before they are issued.
// The rounding points are those of the separate add and norm, but the sum of
// squares runs in another order (per lane over its 32 elements, then one wave
// reduction; the separate norm and NormX sum in other partitions), so inv and
// hence each x element can differ from the separate norm's by one binary16
// rounding.
struct RegNormX {
    static constexpr bool kSinglePass = true;
    u32x4 t[4], e[4], g[4];  // a, d (when has_d), w
    bool has_d;
    float eps;
    int K;
    uint16_t* x_out;
    uint16_t* h_out;
    const uint16_t* b;  // a K-element vector for unresolvable rows
    __device__ __forceinline__ const uint16_t* base() const { return b; }
    template <bool VEC, bool FULL>
    __device__ __forceinline__ void load(int, int, bool, f16x2 xv[16]) const {
        const int lane = threadIdx.x & (kWave - 1);
        u32x4 s[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s[i] = t[i];
            if (has_d) {
                s[i].x = add_f16x2(t[i].x, e[i].x);
                s[i].y = add_f16x2(t[i].y, e[i].y);
                s[i].z = add_f16x2(t[i].z, e[i].z);
                s[i].w = add_f16x2(t[i].w, e[i].w);
            }
        }
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            ss += sumsq_f16x2(s[i].x) + sumsq_f16x2(s[i].y) + sumsq_f16x2(s[i].z) + sumsq_f16x2(s[i].w);
        const float inv = rsqrtf(wave_sum_bcast(ss) / static_cast<float>(K) + eps);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4 r;
            r.x = norm_f16x2(s[i].x, g[i].x, inv);
            r.y = norm_f16x2(s[i].y, g[i].y, inv);
            r.z = norm_f16x2(s[i].z, g[i].z, inv);
            r.w = norm_f16x2(s[i].w, g[i].w, inv);
            xv[4 * i + 0] = as_f16x2(r.x);
            xv[4 * i + 1] = as_f16x2(r.y);
            xv[4 * i + 2] = as_f16x2(r.z);
            xv[4 * i + 3] = as_f16x2(r.w);
            if (x_out) stg(reinterpret_cast<u32x4*>(x_out) + 4 * lane + i, s[i]);
            if (h_out) stg(reinterpret_cast<u32x4*>(h_out) + 4 * lane + i, r);
        }
    }
};

// Epilogues: row r of the tile has its fp32 total in the lanes reduce_rows_row
// assigns to it. StoreY: y[row] = fp16(total) (NaN for an unresolvable row).
// SiluIdxY: y[row] = fp16(silu(gate[idx[row]]) * fp16(total)), the SwiGLU gating
// of the selected channels (generate.py:304-305). SwigluY (R = 8 only, rows
// interleaved by 8-row tiles as 4 gate rows then the 4 matching up rows):
// y[4*tile + i] = fp16(silu(fp16(gate_i)) * fp16(up_i)) (generate.py:178).
struct StoreY {
    static constexpr bool kSwiglu = false;
    static constexpr bool kPrefetch = false;
    struct Pre {};
    uint16_t* y;
    __device__ __forceinline__ void store(int64_t row, float total, bool valid) const {
        stg(y + row, valid ? f32_to_f16_bits(total) : uint16_t(0x7e00u));
    }
};

// StoreYAdd: StoreY, and res_out[row] = res[row] + y[row] as one binary16 addition
// (the residual update the next RMSNorm would otherwise do on load, with the same
// rounding). res[row] is requested before the tile's weights.
struct StoreYAdd {
    static constexpr bool kSwiglu = false;
    static constexpr bool kPrefetch = true;
    uint16_t* y;
    const uint16_t* res;
    uint16_t* res_out;
    struct Pre {
        uint16_t r;
    };
    template <int R>
    __device__ __forceinline__ Pre prefetch(int64_t row0, int r_lane, int64_t N) const {
        return {ldg(res + (row0 + r_lane < N ? row0 + r_lane : N - 1))};
    }
    __device__ __forceinline__ void store(int64_t row, float total, bool valid, Pre p) const {
        const uint16_t yb = valid ? f32_to_f16_bits(total) : uint16_t(0x7e00u);
        stg(y + row, yb);
        stg(res_out + row, static_cast<uint16_t>(add_f16x2(p.r, yb)));
    }
};

// SiluIdxY requests its gate value before the tile's weight loads: the tile's
// R channels are read with wave-uniform (scalar) loads, the lane's one is
// selected and gate[c] is requested right away, instead of two dependent
// loads after the dot products.
struct SiluIdxY {
    static constexpr bool kSwiglu = false;
    static constexpr bool kPrefetch = true;
    uint16_t* y;
    const uint16_t* gate;
    const int32_t* idx;
    int n_gate;
    struct Pre {
        uint16_t g;
        bool ok;
    };
    // rows row0 .. row0 + R - 1 (clamped to N - 1); the lane stores row row0 + r_lane
    template <int R>
    __device__ __forceinline__ Pre prefetch(int64_t row0, int r_lane, int64_t N) const {
        int32_t c = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int32_t cr = ldg(idx + (row0 + r < N ? row0 + r : N - 1));
            c = r == r_lane ? cr : c;
        }
        const bool ok = c >= 0 && c < n_gate;
        return {ldg(gate + (ok ? c : 0)), ok};
    }
    __device__ __forceinline__ void store(int64_t row, float total, bool valid, Pre p) const {
        const bool ok = valid && p.ok;
        const float u = f16_bits_to_f32(f32_to_f16_bits(total));
        const float g = ok ? f16_bits_to_f32(p.g) : 0.0f;
        stg(y + row, ok ? f32_to_f16_bits(silu_f32(g) * u) : uint16_t(0x7e00u));
    }
};

// SwigluY: y[4t + i] = fp16(silu(g) * u) of the tile's gate row g = fp16(row 8t + i) and up row
// u = fp16(row 8t + 4 + i); with gate set, also gate[4t + i] = g (the value SplitGUY writes).
struct SwigluY {
    static constexpr bool kSwiglu = true;
    static constexpr bool kPrefetch = false;
    struct Pre {};
    uint16_t* y;
    uint16_t* gate = nullptr;
};

// SplitGUY (rows interleaved by 8-row tiles as for SwigluY): row 8t + i goes to
// gate[4t + i] for i < 4 and to up[4t + i - 4] otherwise, each fp16(total) as
// StoreY would write it, so both halves equal the plain GEMV of those rows.
struct SplitGUY {
    static constexpr bool kSwiglu = false;
    static constexpr bool kPrefetch = false;
    struct Pre {};
    uint16_t* gate;
    uint16_t* up;
    __device__ __forceinline__ void store(int64_t row, float total, bool valid) const {
        const int64_t t = row >> 3;
        const int i = static_cast<int>(row & 7);
        uint16_t* dst = i < 4 ? gate + 4 * t + i : up + 4 * t + (i - 4);
        stg(dst, valid ? f32_to_f16_bits(total) : uint16_t(0x7e00u));
    }
};

// Streaming GEMV kernels ask the compiler for at least 6 resident waves per
// SIMD (<= 80 VGPRs, no spills at these tile sizes): with the default
// allocation the 8-row tile takes ~120 VGPRs (4 waves), and the extra waves'
// loads in flight are worth ~5% of HBM bandwidth on the gate/up batch.
#define SOI_GEMV_OCCUPANCY __attribute__((amdgpu_waves_per_eu(6, 8)))

// R rows per wave; PU passes (64 chunks each) loaded per batch, so a wave has
// R*PU 1 KB row segments in flight before it does any arithmetic.
template <int R, int PU, bool VEC, bool CHUNK_SCALE, bool BITFIELD, bool FULL, class Rows, class XS, class EP>
__device__ __forceinline__ void gemv_int4_tile(const Rows& rows, int64_t N, const XS& xsrc, const EP& ep, int K,
                                               int gs, int64_t row0) {
    constexpr int SC = CHUNK_SCALE ? 1 : 4;
    const int lane = threadIdx.x & (kWave - 1);  // lane in its wave (workgroups may hold several waves)
    const int words = (K + 7) >> 3;
    const int chunks = (words + 3) >> 2;

    RowRef ref[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (FULL) {
            ref[r] = rows.get(row0 + r);
        } else {
            const bool in = row0 + r < N;
            ref[r] = rows.get(in ? row0 + r : N - 1);
            if (!in) ref[r].ok = false;
        }
    }
    // the rows of a tile are the same for every lane: keep their addresses in scalar registers
#pragma unroll
    for (int r = 0; r < R; ++r) {
        ref[r].w = uniform_ptr(ref[r].w);
        ref[r].s = uniform_ptr(ref[r].s);
    }
    bool valid[R];  // row exists and resolved (else y untouched / NaN)
#pragma unroll
    for (int r = 0; r < R; ++r) valid[r] = ref[r].ok;
    if (FULL) {
        // an unresolvable row reads row 0 of the batch instead (wave-uniform select) and is written as NaN
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!valid[r]) {
                ref[r].w = ref[0].ok ? ref[0].w : reinterpret_cast<const uint8_t*>(xsrc.base());
                ref[r].s = ref[0].ok ? ref[0].s : reinterpret_cast<const float*>(xsrc.base());
            }
        }
    }

    // epilogue operands that do not depend on the result are requested before the weights
    typename EP::Pre pre{};
    if constexpr (EP::kPrefetch) pre = ep.template prefetch<R>(row0, reduce_rows_row<R>(static_cast<uint32_t>(lane)), N);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    const int c_end = XS::kSinglePass ? kWave * PU : chunks;  // single pass: no loop for the compiler to keep
    for (int c0 = 0; c0 < c_end; c0 += kWave * PU) {
        uint32_t wv[PU][R][4];
        float sc[PU][R][SC];
        f16x2 xv[PU][16];
        float xs[PU][SC];  // sum of x over the chunk (or over each word)
#pragma unroll
        for (int p = 0; p < PU; ++p) {
            const int c = c0 + p * kWave + lane;
            const bool cv = FULL || c < chunks;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const bool ok = FULL || (valid[r] && cv);
                load_w_chunk<VEC, FULL>(ref[r].w, ok, words, c, wv[p][r]);
                const float* zf = reinterpret_cast<const float*>(g_zero16);
                if (CHUNK_SCALE) {
                    sc[p][r][0] = ldg(ok ? ref[r].s + (32 * c) / gs : zf);
                } else {
#pragma unroll
                    for (int i = 0; i < SC; ++i) {
                        const int wi = 4 * c + i;
                        sc[p][r][i] = ldg((ok && wi < words) ? ref[r].s + (8 * wi) / gs : zf);
                    }
                }
            }
            // a single-pass x source computes x from registers: keep that work after the weight loads
            if constexpr (XS::kSinglePass) __builtin_amdgcn_sched_barrier(0);
            xsrc.template load<VEC, FULL>(K, c, cv, xv[p]);
        }
        // the x sums only after every pass's loads are issued (summing pass p's x first would make the wave wait
        // for it before requesting pass p + 1); with several passes the order is pinned for the scheduler too
        if constexpr (PU > 1) __builtin_amdgcn_sched_barrier(0);
        const f16x2 ones = {(f16)1.0f, (f16)1.0f};
#pragma unroll
        for (int p = 0; p < PU; ++p) {
#pragma unroll
            for (int i = 0; i < SC; ++i) {
                float t = 0.0f;
#pragma unroll
                for (int e = 0; e < 16 / SC; ++e) t = dot2(xv[p][(16 / SC) * i + e], ones, t);
                xs[p][i] = t;
            }
        }
#pragma unroll
        for (int p = 0; p < PU; ++p) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (CHUNK_SCALE) {
                    float ta = 0.0f, tb = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        f16x2 lo[2], hi[2];
                        nibble_pairs<BITFIELD>(wv[p][r][i], lo, hi);
                        ta = dot2(lo[0], xv[p][4 * i + 0], ta);
                        tb = dot2(hi[0], xv[p][4 * i + 1], tb);
                        ta = dot2(lo[1], xv[p][4 * i + 2], ta);
                        tb = dot2(hi[1], xv[p][4 * i + 3], tb);
                    }
                    const float v = fmaf(ta, kTwo24, fmaf(tb, kTwo20, -8.0f * xs[p][0]));
                    acc[r] = fmaf(sc[p][r][0], v, acc[r]);
                } else {
#pragma unroll
                    for (int i = 0; i < SC; ++i) {
                        f16x2 lo[2], hi[2];
                        nibble_pairs<BITFIELD>(wv[p][r][i], lo, hi);
                        float ta = dot2(lo[0], xv[p][4 * i + 0], 0.0f);
                        float tb = dot2(hi[0], xv[p][4 * i + 1], 0.0f);
                        ta = dot2(lo[1], xv[p][4 * i + 2], ta);
                        tb = dot2(hi[1], xv[p][4 * i + 3], tb);
                        const float v = fmaf(ta, kTwo24, fmaf(tb, kTwo20, -8.0f * xs[p][i]));
                        acc[r] = fmaf(sc[p][r][i], v, acc[r]);
                    }
                }
            }
        }
    }

    const float total = reduce_rows<R>(acc);
    const int r = reduce_rows_row<R>(static_cast<uint32_t>(lane));
    bool vr = valid[0];
#pragma unroll
    for (int i = 1; i < R; ++i) vr = (r == i) ? valid[i] : vr;
    if constexpr (EP::kSwiglu) {
        static_assert(R == 8, "the SwiGLU epilogue pairs rows i and i+4 of an 8-row tile");
        // lanes 0-31 hold rows 7..4 (up), lanes 32-63 rows 3..0 (gate): row r and r-4 are 32 lanes apart
        const float other = __shfl_xor(total, 32, kWave);
        const bool vo = __shfl_xor(vr ? 1 : 0, 32, kWave) != 0;
        if ((lane & 7) == 0 && r >= 4) {
            const uint16_t gb = f32_to_f16_bits(other);
            const float g = f16_bits_to_f32(gb);
            const float u = f16_bits_to_f32(f32_to_f16_bits(total));
            stg(ep.y + (row0 >> 1) + (r - 4), (vr && vo) ? f32_to_f16_bits(silu_f32(g) * u) : uint16_t(0x7e00u));
            if (ep.gate) stg(ep.gate + (row0 >> 1) + (r - 4), vo ? gb : uint16_t(0x7e00u));
        }
    } else {
        if ((lane & (64 / R - 1)) == 0 && (FULL || row0 + r < N)) {
            if constexpr (EP::kPrefetch)
                ep.store(row0 + r, total, vr, pre);
            else
                ep.store(row0 + r, total, vr);
        }
    }
}

}  // namespace soi
