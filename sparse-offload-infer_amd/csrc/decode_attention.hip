// Batch-1 GQA decode attention on gfx950.
//
// Restates csrc/kernels/decode_attention.cu:17-55 (binding scale =
// 1/sqrt(head_dim), bindings.cpp:482): for each query head h with KV head
// kvh = h / (NQ/NKV), out[h] = sum_t softmax_t(scale * q_h . k_t) v_t over
// t < cur_len, fp32 softmax state, fp16 output.
//
// The reference runs one block per query head and two block barriers per
// timestep. Here (fast path, head_dim % 8 == 0, head_dim <= 512, <= 8 query
// heads per KV head):
//   * workgroup (kvh, split) = 4 waves streaming one KV head over a
//     contiguous range of timesteps; every query head that shares the KV head
//     is processed from the same K/V loads (each K/V byte is read once);
//   * a timestep row of head_dim fp16 is read by head_dim/8 lanes with 16-byte
//     loads, so one wave instruction reads 64*16 contiguous bytes;
//   * scores: v_dot2 over the lane's 8 dims, then a butterfly over the row's
//     lanes; softmax runs in the log2 domain (scores pre-multiplied by
//     scale*log2(e), v_exp_f32) with the online max/sum recurrence of the
//     reference (m0 = -1e30);
//   * lane groups, then waves (in wave order), then splits (in split order)
//     are merged with the standard (m, l, acc) rescaling. Fixed order:
//     deterministic.
// Other shapes use a simple one-wave-per-head kernel with the same math.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr float kNegBig = -1e30f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Context length: the host value, or (device form) pos[0] + 1 clamped to [1, S].
// A split that starts at or past L writes the neutral state (m = -1e30, l = 0).
__device__ __forceinline__ int cur_len_of(int L_arg, const int32_t* pos, int S) {
    if (!pos) return L_arg;
    const int p = ldg(pos);
    return p < 0 ? 1 : (p >= S ? S : p + 1);
}

// Split plan for a context of L timesteps: about 256 workgroups over the KV
// cache, tps a multiple of the timesteps one workgroup iteration covers. The
// host (plan_attention) and the device (the device-position forms, which read
// L at run time) use this same formula, so both give the same partition and
// bit-identical results. ns <= ceil(256 / NKV) for every L.
__host__ __device__ __forceinline__ void split_plan(int64_t L, int64_t NKV, int64_t step, int& tps, int& ns) {
    int64_t t = (L * NKV + 255) / 256;
    t = (t + step - 1) / step * step;
    if (t < step) t = step;
    tps = static_cast<int>(t);
    ns = static_cast<int>((L + t - 1) / t);
}

template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int mask = 1; mask < LPR; mask <<= 1) v += __shfl_xor(v, mask, kWave);
    return v;
}

// Partial state layout per (query head, split): [m, l, acc[hd]] in fp32.
//
// attn_core: one workgroup streams timesteps [t0, t1) of KV head kvh for the
// REP query heads held in registers (qv), and writes their partial states
// for split `split`. Timestep tnew (or none, tnew < 0) takes its K/V rows from
// LDS (knew/vnew: the token being appended in the same launch).
template <int LPR, int REP>
__device__ __forceinline__ void attn_core(const f16x2 (&qv)[REP][4], int rep, int kvh, int split, int t0, int t1,
                                          int S, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                                          float* __restrict__ part, int nsplit, float scale_log2, int tnew,
                                          const u32x4* knew, const u32x4* vnew,
                                          float (*s_state)[REP][LPR * 8 + 2], const u32x4* first_k = nullptr,
                                          const u32x4* first_v = nullptr) {
    constexpr int HD = LPR * 8;
    constexpr int RPI = kWave / LPR;  // timesteps per wave instruction
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int g = lane / LPR, u = lane % LPR;
    float m[REP], l[REP], acc[REP][8];
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        m[hh] = kNegBig;
        l[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) acc[hh][d] = 0.0f;
    }

    const uint16_t* kbase = kc + static_cast<int64_t>(kvh) * S * HD;
    const uint16_t* vbase = vc + static_cast<int64_t>(kvh) * S * HD;
    // Software pipeline: the next iteration's K/V rows are requested before the
    // current ones are consumed. Rows past the range are clamped to the last
    // valid row (always a legal address) and masked out of the softmax.
    auto load_kv = [&](int tb_, u32x4& kk_, u32x4& vv_) {
        const int t = tb_ + g;
        const int tl = t < t1 ? t : t1 - 1;
        kk_ = ldg(reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(tl) * HD) + u);
        vv_ = ldg(reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(tl) * HD) + u);
        if (tl == tnew) {
            kk_ = knew[u];
            vv_ = vnew[u];
        }
    };
    u32x4 kk, vv;
    int tb = t0 + wave * RPI;
    if (first_k) {  // the caller issued the first rows' loads early; patch in the appended row
        kk = *first_k;
        vv = *first_v;
        const int t = tb + g;
        if ((t < t1 ? t : t1 - 1) == tnew) {
            kk = knew[u];
            vv = vnew[u];
        }
    } else {
        load_kv(tb, kk, vv);
    }
    for (; tb < t1; tb += kAttnWaves * RPI) {
        u32x4 kn, vn;
        load_kv(tb + kAttnWaves * RPI, kn, vn);
        const bool valid = tb + g < t1;
        const f16x2 k0 = as_f16x2(kk.x), k1 = as_f16x2(kk.y), k2 = as_f16x2(kk.z), k3 = as_f16x2(kk.w);
        const f16x2 v2[4] = {as_f16x2(vv.x), as_f16x2(vv.y), as_f16x2(vv.z), as_f16x2(vv.w)};
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            if (hh >= rep) break;
            float part_s = dot2(qv[hh][0], k0, 0.0f);
            part_s = dot2(qv[hh][1], k1, part_s);
            part_s = dot2(qv[hh][2], k2, part_s);
            part_s = dot2(qv[hh][3], k3, part_s);
            float sc = group_sum<LPR>(part_s) * scale_log2;  // every lane of the group takes part
            if (!valid) sc = -__builtin_inff();
            const float mn = fmaxf(m[hh], sc);
            const float corr = fast_exp2(m[hh] - mn);
            const float p = fast_exp2(sc - mn);
            l[hh] = fmaf(l[hh], corr, p);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[hh][2 * e] = fmaf(acc[hh][2 * e], corr, p * static_cast<float>(v2[e].x));
                acc[hh][2 * e + 1] = fmaf(acc[hh][2 * e + 1], corr, p * static_cast<float>(v2[e].y));
            }
            m[hh] = mn;
        }
        kk = kn;
        vv = vn;
    }

    // merge lane groups (same u, different timesteps) inside the wave
#pragma unroll
    for (int mask = LPR; mask < kWave; mask <<= 1) {
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            if (hh >= rep) break;
            const float mo = __shfl_xor(m[hh], mask, kWave);
            const float lo = __shfl_xor(l[hh], mask, kWave);
            const float mn = fmaxf(m[hh], mo);
            const float ca = fast_exp2(m[hh] - mn), cb = fast_exp2(mo - mn);
            l[hh] = l[hh] * ca + lo * cb;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const float ao = __shfl_xor(acc[hh][d], mask, kWave);
                acc[hh][d] = acc[hh][d] * ca + ao * cb;
            }
            m[hh] = mn;
        }
    }
    if (g == 0) {
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            if (hh >= rep) break;
            if (u == 0) {
                s_state[wave][hh][0] = m[hh];
                s_state[wave][hh][1] = l[hh];
            }
#pragma unroll
            for (int d = 0; d < 8; ++d) s_state[wave][hh][2 + 8 * u + d] = acc[hh][d];
        }
    }
    __syncthreads();
    // merge the waves in order; thread i handles element i of [m, l, acc...]
    for (int hh = 0; hh < rep; ++hh) {
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) M = fmaxf(M, s_state[w][hh][0]);
        float* out = part + (static_cast<int64_t>(kvh * rep + hh) * nsplit + split) * (HD + 2);
        for (int i = threadIdx.x; i < HD + 2; i += kAttnThreads) {
            float v = 0.0f;
            if (i == 0) {
                v = M;
            } else {
#pragma unroll
                for (int w = 0; w < kAttnWaves; ++w) v += s_state[w][hh][i] * fast_exp2(s_state[w][hh][0] - M);
            }
            stg(out + i, v);
        }
    }
}

template <int LPR, int REP>
__global__ __launch_bounds__(kAttnThreads) void attn_split_kernel(const uint16_t* __restrict__ q,
                                                                   const uint16_t* __restrict__ kc,
                                                                   const uint16_t* __restrict__ vc,
                                                                   float* __restrict__ part, int rep, int S, int L_arg,
                                                                   const int32_t* __restrict__ pos, int tps, int nsplit,
                                                                   float scale_log2) {
    constexpr int HD = LPR * 8;
    __shared__ float s_state[kAttnWaves][REP][HD + 2];
    const int lane = threadIdx.x & 63;
    const int u = lane % LPR;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int L = cur_len_of(L_arg, pos, S);
    if (pos) {  // device-position form: the plan follows the current length
        int ns;
        split_plan(L, gridDim.x, kWave / LPR * kAttnWaves, tps, ns);
        if (split >= ns) return;
    }
    const int t0 = split * tps;
    const int t1 = min(L, t0 + tps);
    f16x2 qv[REP][4];
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        const int h = kvh * rep + (hh < rep ? hh : 0);
        const u32x4 t = ldg(reinterpret_cast<const u32x4*>(q + static_cast<int64_t>(h) * HD) + u);
        qv[hh][0] = as_f16x2(t.x);
        qv[hh][1] = as_f16x2(t.y);
        qv[hh][2] = as_f16x2(t.z);
        qv[hh][3] = as_f16x2(t.w);
    }
    attn_core<LPR, REP>(qv, rep, kvh, split, t0, t1, S, kc, vc, part, nsplit, scale_log2, -1, nullptr, nullptr,
                        s_state);
}

// out[h,d] = (sum_s acc_s[d] 2^(m_s-M)) / (sum_s l_s 2^(m_s-M)) over the active
// splits (all of them, or, in the device-position form, those that start
// below the current length: the others hold the neutral state and add exact
// zeros). M and the denominator are block reductions over the splits; each
// thread then sums its dimension over the splits in ascending order with the
// loads issued 8 at a time. Fixed order: deterministic.
constexpr int kCombineThreads = 128;
constexpr int kCombineMaxSplits = 256;  // nsplit <= 256 by construction of the plan

template <int NT>
__device__ __forceinline__ float block_reduce(float v, float* s_red, bool is_max) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = is_max ? wave_max_bcast(v) : wave_sum_bcast(v);
    __syncthreads();
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float r = s_red[0];
#pragma unroll
    for (int w = 1; w < NT / kWave; ++w) r = is_max ? fmaxf(r, s_red[w]) : r + s_red[w];
    return r;
}

// Combine the first ns split states of head h into out[h, :] (NT threads).
template <int NT>
__device__ __forceinline__ void combine_head(const float* __restrict__ part, uint16_t* __restrict__ out, int h, int hd,
                                             int nsplit, int ns, float* s_w, float* s_red) {
    const int tid = threadIdx.x;
    const int stride = hd + 2;
    const float* ph = part + static_cast<int64_t>(h) * nsplit * stride;
    float m = kNegBig;
    for (int sp = tid; sp < ns; sp += NT) m = fmaxf(m, ldg(ph + sp * stride));
    const float M = block_reduce<NT>(m, s_red, true);
    float lp = 0.0f;
    for (int sp = tid; sp < ns; sp += NT) {
        const float w = fast_exp2(ldg(ph + sp * stride) - M);
        if (sp < kCombineMaxSplits) s_w[sp] = w;
        lp = fmaf(ldg(ph + sp * stride + 1), w, lp);
    }
    const float Lsum = block_reduce<NT>(lp, s_red, false);
    __syncthreads();  // s_w complete
    for (int d = tid; d < hd; d += NT) {
        float a = 0.0f;
        int sp = 0;
        for (; sp + 8 <= ns && sp + 8 <= kCombineMaxSplits; sp += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ldg(ph + (sp + u) * stride + 2 + d);
#pragma unroll
            for (int u = 0; u < 8; ++u) a = fmaf(v[u], s_w[sp + u], a);
        }
        for (; sp < ns; ++sp) {
            const float w = sp < kCombineMaxSplits ? s_w[sp] : fast_exp2(ldg(ph + sp * stride) - M);
            a = fmaf(ldg(ph + sp * stride + 2 + d), w, a);
        }
        stg(out + static_cast<int64_t>(h) * hd + d, f32_to_f16_bits(a / Lsum));
    }
    __syncthreads();  // s_w / s_red reusable
}

__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                        uint16_t* __restrict__ out, int hd,
                                                                        int nsplit, int NKV, int step,
                                                                        const int32_t* __restrict__ pos, int S) {
    __shared__ float s_w[kCombineMaxSplits];
    __shared__ float s_red[kCombineThreads / kWave];
    int ns = nsplit;
    if (pos) {
        int tps;
        split_plan(cur_len_of(0, pos, S), NKV, step, tps, ns);
    }
    combine_head<kCombineThreads>(part, out, blockIdx.x, hd, nsplit, ns, s_w, s_red);
}

// One launch per decoder layer (the decode engine's form): per workgroup
// (kvh, split), q/k RMSNorm + RoPE of the fused projection qkv
// [q (NQ*hd) | k (NKV*hd) | v (NKV*hd)] at position p = pos[0] (the same
// binary16 rounding points as qk_norm_rope_append), the KV append of k, v at
// p by the workgroup whose split holds p (which also reads timestep p from
// LDS, not from the cache it is writing), the split's online softmax, and,
// in the last workgroup of KV head kvh to finish (a device-scope counter),
// the combine of its query heads. Splits that start at or past p + 1 exit at
// once. counters[kvh] must be 0 before the launch; the last workgroup resets it.
template <int LPR, int REP>
__global__ __launch_bounds__(kAttnThreads) void attn_step_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int32_t* __restrict__ pos_ptr,
    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, float* __restrict__ part, uint32_t* __restrict__ counters,
    uint16_t* __restrict__ out, int rep, int NQ, int NKV, int S, int nsplit, float eps, float scale_log2) {
    constexpr int HD = LPR * 8;
    constexpr int HALF = HD / 2;
    __shared__ float s_state[kAttnWaves][REP][HD + 2];
    __shared__ __attribute__((aligned(16))) uint16_t s_q[REP][HD];
    __shared__ __attribute__((aligned(16))) uint16_t s_kv[2][HD];
    __shared__ float s_w[kCombineMaxSplits];
    __shared__ float s_red[kAttnWaves];
    __shared__ int s_last;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kvh = blockIdx.x, split = blockIdx.y;
    const int p = ldg(pos_ptr);
    const bool pvalid = p >= 0 && p < S;
    const int L = p < 0 ? 1 : (p >= S ? S : p + 1);
    int tps, ns;
    split_plan(L, NKV, kWave / LPR * kAttnWaves, tps, ns);
    if (split >= ns) return;  // inactive split: no partial state, no arrival
    const int t0 = split * tps;
    const int t1 = min(L, t0 + tps);
    const bool has_new = pvalid && p >= t0 && p < t1;
    const int prow = pvalid ? p : (p < 0 ? 0 : S - 1);  // RoPE table row

    // issue the first K/V rows of this split now (they do not depend on q); row p is patched from LDS later
    const int u = lane % LPR;
    u32x4 k_first, v_first;
    {
        constexpr int RPI = kWave / LPR;
        const int t = t0 + wave * RPI + lane / LPR;
        const int tl = t < t1 ? t : t1 - 1;
        k_first = ldg(reinterpret_cast<const u32x4*>(kc + (static_cast<int64_t>(kvh) * S + tl) * HD) + u);
        v_first = ldg(reinterpret_cast<const u32x4*>(vc + (static_cast<int64_t>(kvh) * S + tl) * HD) + u);
    }

    // q heads kvh*rep + hh (and, in the split holding p, the new k): wave w takes heads w, w+4, ...
    // Lane l reduces elements l, l+64, ... in that order (the order of qk_norm_rope_append).
    const int nh = rep + (has_new ? 1 : 0);
    for (int hh = wave; hh < nh; hh += kAttnWaves) {
        const bool isk = hh == rep;
        const uint16_t* src = qkv + static_cast<int64_t>(isk ? NQ + kvh : kvh * rep + hh) * HD;
        const uint16_t* wn = isk ? k_norm : q_norm;
        uint16_t* dst = isk ? s_kv[0] : s_q[hh];
        const float* cr = cos_t + static_cast<int64_t>(prow) * HALF;
        const float* sr = sin_t + static_cast<int64_t>(prow) * HALF;
        if (HALF == kWave) {  // one pair per lane: every operand loaded up front
            const float x1 = f16_bits_to_f32(ldg(src + lane)), x2 = f16_bits_to_f32(ldg(src + lane + HALF));
            const float w1 = f16_bits_to_f32(ldg(wn + lane)), w2 = f16_bits_to_f32(ldg(wn + lane + HALF));
            const float c = ldg(cr + lane), sn = ldg(sr + lane);
            const float inv = rsqrtf(wave_sum_bcast(fmaf(x2, x2, x1 * x1)) / static_cast<float>(HD) + eps);
            const float a = f16_bits_to_f32(f32_to_f16_bits(x1 * inv * w1));
            const float b = f16_bits_to_f32(f32_to_f16_bits(x2 * inv * w2));
            float o1, o2;
            rope_pair(a, b, c, sn, o1, o2);
            dst[lane] = f32_to_f16_bits(o1);
            dst[lane + HALF] = f32_to_f16_bits(o2);
        } else {
            float ss = 0.0f;
            for (int i = lane; i < HD; i += kWave) {
                const float v = f16_bits_to_f32(ldg(src + i));
                ss = fmaf(v, v, ss);
            }
            const float inv = rsqrtf(wave_sum_bcast(ss) / static_cast<float>(HD) + eps);
            for (int i = lane; i < HALF; i += kWave) {
                const float a = f16_bits_to_f32(
                    f32_to_f16_bits(f16_bits_to_f32(ldg(src + i)) * inv * f16_bits_to_f32(ldg(wn + i))));
                const float b = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(ldg(src + i + HALF)) * inv *
                                                                f16_bits_to_f32(ldg(wn + i + HALF))));
                const float c = ldg(cr + i), sn = ldg(sr + i);
                float o1, o2;
                rope_pair(a, b, c, sn, o1, o2);
                dst[i] = f32_to_f16_bits(o1);
                dst[i + HALF] = f32_to_f16_bits(o2);
            }
        }
    }
    if (has_new) {
        const uint16_t* vsrc = qkv + static_cast<int64_t>(NQ + NKV + kvh) * HD;
        for (int i = threadIdx.x; i < HD; i += kAttnThreads) s_kv[1][i] = ldg(vsrc + i);
    }
    __syncthreads();
    if (has_new) {  // append k, v at p
        uint16_t* kd = kc + (static_cast<int64_t>(kvh) * S + p) * HD;
        uint16_t* vd = vc + (static_cast<int64_t>(kvh) * S + p) * HD;
        for (int i = threadIdx.x; i < HD; i += kAttnThreads) {
            stg(kd + i, s_kv[0][i]);
            stg(vd + i, s_kv[1][i]);
        }
    }
    f16x2 qv[REP][4];
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        const u32x4 t = reinterpret_cast<const u32x4*>(s_q[hh < rep ? hh : 0])[u];
        qv[hh][0] = as_f16x2(t.x);
        qv[hh][1] = as_f16x2(t.y);
        qv[hh][2] = as_f16x2(t.z);
        qv[hh][3] = as_f16x2(t.w);
    }
    attn_core<LPR, REP>(qv, rep, kvh, split, t0, t1, S, kc, vc, part, nsplit, scale_log2, has_new ? p : -1,
                        reinterpret_cast<const u32x4*>(s_kv[0]), reinterpret_cast<const u32x4*>(s_kv[1]), s_state,
                        &k_first, &v_first);

    // arrival: the last of the ns active splits of this KV head combines its query heads
    arrive_release();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(counters + kvh, 1u);
        const bool last = prev + 1 == static_cast<uint32_t>(ns);
        if (last) atomicExch(counters + kvh, 0u);
        s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the other splits' partial states
    for (int hh = 0; hh < rep; ++hh)
        combine_head<kAttnThreads>(part, out, kvh * rep + hh, HD, nsplit, ns, s_w, s_red);
}

// General shapes: one wave per query head, lanes over dims, online softmax.
__global__ __launch_bounds__(64) void attn_simple_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                                          const uint16_t* __restrict__ vc, uint16_t* __restrict__ out,
                                                          int rep, int S, int hd, int L_arg,
                                                          const int32_t* __restrict__ pos, float scale_log2) {
    const int h = blockIdx.x, lane = threadIdx.x;
    const int L = cur_len_of(L_arg, pos, S);
    const int kvh = h / rep;
    const uint16_t* kb = kc + static_cast<int64_t>(kvh) * S * hd;
    const uint16_t* vb = vc + static_cast<int64_t>(kvh) * S * hd;
    const uint16_t* qh = q + static_cast<int64_t>(h) * hd;
    constexpr int kMaxPer = 16;  // head_dim <= 1024
    float accd[kMaxPer];
    float qd[kMaxPer];
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int d = lane + 64 * i;
        accd[i] = 0.0f;
        qd[i] = d < hd ? f16_bits_to_f32(qh[d]) : 0.0f;
    }
    float m = kNegBig, l = 0.0f;
    for (int t = 0; t < L; ++t) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int d = lane + 64 * i;
            if (d < hd) part = fmaf(qd[i], f16_bits_to_f32(kb[static_cast<int64_t>(t) * hd + d]), part);
        }
        const float sc = wave_sum_bcast(part) * scale_log2;
        const float mn = fmaxf(m, sc);
        const float corr = fast_exp2(m - mn), p = fast_exp2(sc - mn);
        l = fmaf(l, corr, p);
#pragma unroll
        for (int i = 0; i < kMaxPer; ++i) {
            const int d = lane + 64 * i;
            if (d < hd) accd[i] = fmaf(accd[i], corr, p * f16_bits_to_f32(vb[static_cast<int64_t>(t) * hd + d]));
        }
        m = mn;
    }
#pragma unroll
    for (int i = 0; i < kMaxPer; ++i) {
        const int d = lane + 64 * i;
        if (d < hd) out[static_cast<int64_t>(h) * hd + d] = f32_to_f16_bits(accd[i] / l);
    }
}

struct AttnPlan {
    bool fast;
    int lpr, rep_t, step, tps, nsplit;
    int cap;  // the most splits any length <= the planned one can need (device-position grids)
};

// L: the context length to plan for; with a device position, the largest one (max_seq).
static AttnPlan plan_attention(int64_t NQ, int64_t NKV, int64_t hd, int64_t L) {
    AttnPlan p{false, 0, 0, 0, 0, 0, 0};
    const int64_t rep = NQ / NKV;
    const int64_t lpr = hd / 8;
    const bool pow2 = lpr >= 1 && (lpr & (lpr - 1)) == 0;
    if (hd % 8 == 0 && pow2 && lpr <= 64 && rep <= 8) {
        p.fast = true;
        p.lpr = static_cast<int>(lpr);
        p.rep_t = rep <= 1 ? 1 : rep <= 2 ? 2 : rep <= 4 ? 4 : 8;
        p.step = static_cast<int>((kWave / lpr) * kAttnWaves);  // timesteps per workgroup iteration
        split_plan(L, NKV, p.step, p.tps, p.nsplit);
        const int64_t by_len = ceil_div64(L, p.step), by_heads = ceil_div64(256, NKV);
        p.cap = static_cast<int>(by_len < by_heads ? by_len : by_heads);
        if (p.cap < p.nsplit) p.cap = p.nsplit;
    }
    return p;
}

static int launch_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                            int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim, int64_t cur_len,
                            const int32_t* pos, float scale, void* workspace, size_t workspace_bytes, hipStream_t st,
                            const char* what) {
    const float scale_log2 = scale * kLog2e;
    const int rep = static_cast<int>(NQ / NKV);
    // host length: plan for cur_len; device position: grid for every length up to max_seq, plan at run time
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, pos ? max_seq : cur_len);
    const bool aligned = aligned16(q) && aligned16(k_cache) && aligned16(v_cache);
    if (!p.fast || !aligned) {
        hipLaunchKernelGGL(attn_simple_kernel, dim3(static_cast<unsigned>(NQ)), dim3(64), 0, st, q, k_cache, v_cache,
                           out, rep, static_cast<int>(max_seq), static_cast<int>(head_dim),
                           static_cast<int>(cur_len), pos, scale_log2);
        return launch_status(what);
    }
    const int nsplit = pos ? p.cap : p.nsplit;
    const size_t need = static_cast<size_t>(NQ) * nsplit * (head_dim + 2) * sizeof(float);
    if (!workspace || workspace_bytes < need) {
        set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    float* part = static_cast<float*>(workspace);
    const dim3 grid(static_cast<unsigned>(NKV), static_cast<unsigned>(nsplit));
    const int S = static_cast<int>(max_seq), L = static_cast<int>(cur_len);
#define SOI_A(LL, RR)                                                                                              \
    hipLaunchKernelGGL((attn_split_kernel<LL, RR>), grid, dim3(kAttnThreads), 0, st, q, k_cache, v_cache, part, rep, \
                       S, L, pos, p.tps, nsplit, scale_log2)
#define SOI_AR(LL)                       \
    switch (p.rep_t) {                   \
        case 1: SOI_A(LL, 1); break;     \
        case 2: SOI_A(LL, 2); break;     \
        case 4: SOI_A(LL, 4); break;     \
        default: SOI_A(LL, 8); break;    \
    }
    switch (p.lpr) {
        case 1: SOI_AR(1); break;
        case 2: SOI_AR(2); break;
        case 4: SOI_AR(4); break;
        case 8: SOI_AR(8); break;
        case 16: SOI_AR(16); break;
        case 32: SOI_AR(32); break;
        default: SOI_AR(64); break;
    }
#undef SOI_AR
#undef SOI_A
    int s = launch_status(what);
    if (s) return s;
    hipLaunchKernelGGL(attn_combine_kernel, dim3(static_cast<unsigned>(NQ)), dim3(kCombineThreads), 0, st, part, out,
                       static_cast<int>(head_dim), nsplit, static_cast<int>(NKV), p.step, pos, S);
    return launch_status(what);
}

static int check_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                           int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim, const char* what) {
    SOI_REQUIRE(NQ >= 1 && NKV >= 1 && NQ % NKV == 0, "%s: num_q_heads must be a positive multiple of num_kv_heads",
                what);
    SOI_REQUIRE(head_dim >= 1 && head_dim <= 1024, "%s: head_dim must be in [1, 1024]", what);
    SOI_REQUIRE(max_seq >= 1 && max_seq <= (int64_t(1) << 30), "%s: max_seq_len out of range", what);
    SOI_REQUIRE(NQ <= 65535, "%s: too many heads", what);
    SOI_REQUIRE(q && k_cache && v_cache && out, "%s: null pointer", what);
    return SOI_OK;
}

}  // namespace soi

using namespace soi;

extern "C" size_t soi_decode_attention_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t cur_len) {
    if (NQ <= 0 || NKV <= 0 || head_dim <= 0 || cur_len <= 0 || NQ % NKV) return 0;
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, cur_len);  // covers the device form with max_seq = cur_len
    if (!p.fast) return 0;
    return static_cast<size_t>(NQ) * p.cap * (head_dim + 2) * sizeof(float);
}

extern "C" int soi_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    uint16_t* out, int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim,
                                    int64_t cur_len, float scale, void* workspace, size_t workspace_bytes,
                                    void* stream) {
    const char* what = "soi_decode_attention";
    int st = check_attention(q, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, what);
    if (st) return st;
    SOI_REQUIRE(cur_len >= 1 && cur_len <= max_seq, "%s: cur_len out of range for max_seq_len", what);
    return launch_attention(q, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, cur_len, nullptr, scale, workspace,
                            workspace_bytes, as_stream(stream), what);
}

extern "C" int soi_decode_attention_at(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                       uint16_t* out, int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim,
                                       const int32_t* pos, float scale, void* workspace, size_t workspace_bytes,
                                       void* stream) {
    const char* what = "soi_decode_attention_at";
    int st = check_attention(q, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, what);
    if (st) return st;
    SOI_REQUIRE(pos, "%s: null position pointer", what);
    return launch_attention(q, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, max_seq, pos, scale, workspace,
                            workspace_bytes, as_stream(stream), what);
}

namespace soi {
constexpr size_t kStepCounterBytes = 256;  // NKV <= 64 counters

static size_t step_partial_bytes(int64_t NQ, int64_t hd, const AttnPlan& p) {
    const size_t b = static_cast<size_t>(NQ) * p.cap * (hd + 2) * sizeof(float);
    return (b + 255) & ~static_cast<size_t>(255);
}
}  // namespace soi

extern "C" size_t soi_decode_attention_step_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim,
                                                            int64_t max_seq) {
    if (NQ <= 0 || NKV <= 0 || NKV > 64 || head_dim <= 0 || max_seq <= 0 || NQ % NKV) return 0;
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, max_seq);
    if (!p.fast) return 0;
    return step_partial_bytes(NQ, head_dim, p) + kStepCounterBytes;
}

extern "C" int soi_decode_attention_step(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                                         const float* cos_table, const float* sin_table, const int32_t* pos,
                                         uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, int64_t NQ,
                                         int64_t NKV, int64_t max_seq, int64_t head_dim, float eps, float scale,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "soi_decode_attention_step";
    int st = check_attention(qkv, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, what);
    if (st) return st;
    SOI_REQUIRE(q_norm && k_norm && cos_table && sin_table && pos, "%s: null pointer", what);
    SOI_REQUIRE(NKV <= 64, "%s: at most 64 KV heads", what);
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, max_seq);
    if (!p.fast || !aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache)) {
        set_last_error("%s: head_dim %lld / GQA ratio %lld / alignment not supported by the one-launch form", what,
                       (long long)head_dim, (long long)(NQ / NKV));
        return SOI_ERR_UNSUPPORTED;
    }
    const size_t pb = step_partial_bytes(NQ, head_dim, p);
    if (!workspace || workspace_bytes < pb + kStepCounterBytes || !aligned16(workspace)) {
        set_last_error("%s: 16-byte aligned workspace of %zu bytes required, got %zu", what, pb + kStepCounterBytes,
                       workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    float* part = static_cast<float*>(workspace);
    uint32_t* counters = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + pb);
    const float scale_log2 = scale * kLog2e;
    const int rep = static_cast<int>(NQ / NKV);
    const dim3 grid(static_cast<unsigned>(NKV), static_cast<unsigned>(p.cap));
    hipStream_t s = as_stream(stream);
    const int nq = static_cast<int>(NQ), nkv = static_cast<int>(NKV), S = static_cast<int>(max_seq);
#define SOI_S(LL, RR)                                                                                           \
    hipLaunchKernelGGL((attn_step_kernel<LL, RR>), grid, dim3(kAttnThreads), 0, s, qkv, q_norm, k_norm, cos_table, \
                       sin_table, pos, k_cache, v_cache, part, counters, out, rep, nq, nkv, S, p.cap, eps,             \
                       scale_log2)
#define SOI_SR(LL)                    \
    switch (p.rep_t) {                \
        case 1: SOI_S(LL, 1); break;  \
        case 2: SOI_S(LL, 2); break;  \
        case 4: SOI_S(LL, 4); break;  \
        default: SOI_S(LL, 8); break; \
    }
    switch (p.lpr) {
        case 1: SOI_SR(1); break;
        case 2: SOI_SR(2); break;
        case 4: SOI_SR(4); break;
        case 8: SOI_SR(8); break;
        case 16: SOI_SR(16); break;
        case 32: SOI_SR(32); break;
        default: SOI_SR(64); break;
    }
#undef SOI_SR
#undef SOI_S
    return launch_status(what);
}
