// Batch-1 GQA decode attention on gfx950.
//
// Restates csrc/kernels/decode_attention.cu:17-55 (binding scale =
// 1/sqrt(head_dim), bindings.cpp:482): for each query head h with KV head
// kvh = h / (NQ/NKV), out[h] = sum_t softmax_t(scale * q_h . k_t) v_t over
// t < cur_len, fp32 softmax state, fp16 output.
//
// The reference runs one block per query head and two block barriers per
// timestep. Here (fast path, head_dim a power of two in [8, 256], <= 8 query
// heads per KV head) ONE kernel serves every form (host length, device
// position, and the decode engine's fused step with q/k norm, RoPE and the KV
// append in front):
//   * workgroup (kvh, split) = 8 waves streaming one KV head over a
//     contiguous range of timesteps; every query head that shares the KV head
//     is processed from the same K/V loads (each K/V byte is read once);
//   * a timestep row of head_dim fp16 is read by head_dim/8 lanes with 16-byte
//     loads, so one wave instruction reads 64*16 contiguous bytes; all the
//     rows of up to 8 passes of the workgroup are requested at kernel start,
//     before anything that depends on q, so they arrive in one memory round
//     trip;
//   * scores: v_dot2 over the lane's 8 dims, then a butterfly over the row's
//     lanes; softmax runs in the log2 domain (scores pre-multiplied by
//     scale*log2(e), v_exp_f32) with the online max/sum recurrence of the
//     reference (m0 = -1e30) taken one chunk of passes at a time: the
//     chunk's scores first, one rescale, then its rows enter the sums; the
//     lane groups of a wave share one running max (a wave max per chunk);
//   * so a wave's lane groups are merged by plain sums (a reduce-scatter of
//     lane swaps), then the waves (in wave order) with the standard
//     (m, l, acc) rescaling;
//   * short contexts (at most 8 passes: 256 timesteps at head_dim 128) run
//     ONE workgroup per KV head, which writes the output itself; longer ones
//     split the timesteps (64 or 128 workgroups), each split writes its state
//     to the workspace and the last split of a KV head to arrive (a device
//     counter) combines them in split order; or (host length, and the
//     deferred step whose states the o projection combines) the splits only
//     write their states and a later launch combines them with the same
//     arithmetic. Fixed order throughout:
//     deterministic, and all forms give identical bytes for the same length.
// Other shapes use a simple one-wave-per-head kernel with the same math.
#include "soi_device.h"
#include "soi_host.h"
#include "soi_int4_tile.h"
#include "soi_attn_plan.h"

namespace soi {

constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr float kNegBig = -1e30f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Context length: the host value, or (device form) pos[0] + 1 clamped to [1, S].
__device__ __forceinline__ int cur_len_of(int L_arg, const int32_t* pos, int S) {
    if (!pos) return L_arg;
    const int p = ldg(pos);
    return p < 0 ? 1 : (p >= S ? S : p + 1);
}


// Sum over the LPR lanes of a row group, every lane of the group gets it. Up to
// 16 lanes this is DPP inside a 16-lane row (a few cycles per step, against
// ~100 for an LDS-crossbar shuffle): rotations by 8 and 4 (or the 8-lane
// mirror), then the two quad exchanges; each step doubles the lanes summed.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    if (LPR >= 16) {
        v += dpp_f<0x128>(v);  // row_ror:8
        v += dpp_f<0x124>(v);  // row_ror:4
    } else if (LPR == 8) {
        v += dpp_f<0x141>(v);  // row_half_mirror: lane i <-> 7-i
    }
    if (LPR >= 4) v += dpp_f<0x4e>(v);  // quad_perm [2,3,0,1]
    if (LPR >= 2) v += dpp_f<0xb1>(v);  // quad_perm [1,0,3,2]
    if (LPR == 32) v += xor_lanes<16>(v);
    return v;
}

template <int LPR, int REP>
struct AttnState {
    float m[REP], l[REP], acc[REP][8];
};

// Score of the lane's row (K kk) for every query head, pre-multiplied by scale * log2(e): v_dot2 over the
// lane's 8 dims, then a sum over the row's lanes (every lane of the group takes part); -inf for a row past the
// range. Heads past rep (rep not a power of two) are computed on head 0's q and never written.
template <int LPR, int REP>
__device__ __forceinline__ void attn_scores(float (&sc)[REP], const f16x2 (&qv)[REP][4], bool valid, const u32x4& kk,
                                            float scale_log2) {
    const f16x2 k0 = as_f16x2(kk.x), k1 = as_f16x2(kk.y), k2 = as_f16x2(kk.z), k3 = as_f16x2(kk.w);
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        float part_s = dot2(qv[hh][0], k0, 0.0f);
        part_s = dot2(qv[hh][1], k1, part_s);
        part_s = dot2(qv[hh][2], k2, part_s);
        part_s = dot2(qv[hh][3], k3, part_s);
        const float sc_h = group_sum<LPR>(part_s) * scale_log2;
        sc[hh] = valid ? sc_h : -__builtin_inff();
    }
}

// The lane's row (V vv) with weight 2^(sc - m) enters every query head's sum (m already covers sc).
template <int LPR, int REP>
__device__ __forceinline__ void attn_accumulate(AttnState<LPR, REP>& st, const float (&sc)[REP], const u32x4& vv) {
    const uint32_t vw[4] = {vv.x, vv.y, vv.z, vv.w};
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const f16x2 v2 = as_f16x2(vw[e]);
        v[2 * e] = static_cast<float>(v2.x);
        v[2 * e + 1] = static_cast<float>(v2.y);
    }
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        const float p = fast_exp2(sc[hh] - st.m[hh]);
        st.l[hh] += p;
#pragma unroll
        for (int d = 0; d < 8; ++d) st.acc[hh][d] = fmaf(p, v[d], st.acc[hh][d]);
    }
}

// a + b of lane pairs swapped across 16-lane rows (ROWS = 16) or wave halves (ROWS = 32) by
// v_permlane16_swap / v_permlane32_swap on two values (swap16 / swap32: the upper row of each pair of VDST
// trades places with the lower row of VSRC0): with vdst = x, vsrc = y, lanes of the lower row of each pair end
// with x of both rows, lanes of the upper row with y of both, summed in row order.
template <int ROWS>
__device__ __forceinline__ float swap_sum(float x, float y) {
    float a = x, b = y;
    if constexpr (ROWS == 16) {
        swap16(a, b);
    } else {
        swap32(a, b);
    }
    return a + b;
}

// Max over the lane groups of a wave (lane exchanges across masks LPR .. 32; the lanes of a group hold the
// same value): every lane gets it.
template <int LPR>
__device__ __forceinline__ float groups_max(float v) {
    if constexpr (LPR <= 1) v = fmaxf(v, xor_lanes<1>(v));
    if constexpr (LPR <= 2) v = fmaxf(v, xor_lanes<2>(v));
    if constexpr (LPR <= 4) v = fmaxf(v, xor_lanes<4>(v));
    if constexpr (LPR <= 8) v = fmaxf(v, xor_lanes<8>(v));
    if constexpr (LPR <= 16) {
        float a = v, b = v;
        swap16(a, b);
        v = fmaxf(a, b);
    }
    float a = v, b = v;
    swap32(a, b);
    return fmaxf(a, b);
}

// The wave's state into s_row (= s_state[wave]): its lane groups share the running max, so l and acc are plain
// sums over the groups. Groups inside a 16-lane row are summed by lane exchanges first (LPR < 16); the rows
// are then summed by a reduce-scatter of swap_sum: level 16 leaves row r with dims (2i + (r & 1)) of its 8,
// level 32 with dims r and 4 + r, each summed over the 4 rows in a fixed order (wave halves: dims 2i + half).
template <int LPR, int REP, int HD>
__device__ __forceinline__ void attn_wave_state(AttnState<LPR, REP>& st, float (*s_row)[HD + 2], int lane) {
    if constexpr (LPR < 16) {
#pragma unroll
        for (int mask = LPR; mask < 16; mask *= 2) {
#pragma unroll
            for (int hh = 0; hh < REP; ++hh) {
                if (mask == 1) st.l[hh] += xor_lanes<1>(st.l[hh]);
                if (mask == 2) st.l[hh] += xor_lanes<2>(st.l[hh]);
                if (mask == 4) st.l[hh] += xor_lanes<4>(st.l[hh]);
                if (mask == 8) st.l[hh] += xor_lanes<8>(st.l[hh]);
#pragma unroll
                for (int d = 0; d < 8; ++d) {
                    if (mask == 1) st.acc[hh][d] += xor_lanes<1>(st.acc[hh][d]);
                    if (mask == 2) st.acc[hh][d] += xor_lanes<2>(st.acc[hh][d]);
                    if (mask == 4) st.acc[hh][d] += xor_lanes<4>(st.acc[hh][d]);
                    if (mask == 8) st.acc[hh][d] += xor_lanes<8>(st.acc[hh][d]);
                }
            }
        }
    }
    const int u = lane % LPR;
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        if constexpr (LPR <= 16) {
            const float l2 = swap_sum<16>(st.l[hh], st.l[hh]);
            const float l4 = swap_sum<32>(l2, l2);
            float b[4], c[2];
#pragma unroll
            for (int i = 0; i < 4; ++i) b[i] = swap_sum<16>(st.acc[hh][2 * i], st.acc[hh][2 * i + 1]);
#pragma unroll
            for (int i = 0; i < 2; ++i) c[i] = swap_sum<32>(b[2 * i], b[2 * i + 1]);
            const int r = lane >> 4;
            if ((lane & 15) < LPR) {
                s_row[hh][2 + 8 * u + r] = c[0];
                s_row[hh][2 + 8 * u + 4 + r] = c[1];
            }
            if (lane == 0) {
                s_row[hh][0] = st.m[hh];
                s_row[hh][1] = l4;
            }
        } else {  // LPR == 32: two groups, the wave halves
            const float l2 = swap_sum<32>(st.l[hh], st.l[hh]);
            const int half = lane >> 5;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                s_row[hh][2 + 8 * u + 2 * i + half] = swap_sum<32>(st.acc[hh][2 * i], st.acc[hh][2 * i + 1]);
            if (lane == 0) {
                s_row[hh][0] = st.m[hh];
                s_row[hh][1] = l2;
            }
        }
    }
}

// The K/V rows of a chunk of up to kAttnPassMax passes, requested together.
// Pass i of wave w reads timestep tb0 + i*kAttnWaves*RPI + (lane / LPR) with
// tb0 = t0 + w*RPI; rows at or past t1 are clamped to t1 - 1 (a legal
// address) and masked out of the softmax.
template <int LPR>
struct AttnRows {
    u32x4 k[kAttnPassMax], v[kAttnPassMax];
    __device__ __forceinline__ void load(const uint16_t* kbase, const uint16_t* vbase, int tb0, int t1, int npass) {
        constexpr int HD = LPR * 8;
        constexpr int RPI = kWave / LPR;
        const int lane = threadIdx.x & 63;
        const int g = lane / LPR, u = lane % LPR;
        // pairs of passes past npass are not requested (one wave-uniform branch per pair, as the pass loop
        // takes them): a clamped request would repeat row t1 - 1, and repeated loads of one address queue
        // behind each other
#pragma unroll
        for (int i = 0; i < kAttnPassMax; i += 2) {
            if (i < npass) {
#pragma unroll
                for (int j = i; j < i + 2; ++j) {
                    const int t = tb0 + j * kAttnWaves * RPI + g;
                    const int tl = (j < npass && t < t1) ? t : t1 - 1;
                    k[j] = ldg(reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(tl) * HD) + u);
                    v[j] = ldg(reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(tl) * HD) + u);
                }
            }
        }
    }
};

// The waves' states of query head hh combined: M = the largest m, w[s] = 2^(m_s - M) (wave order).
template <int REP, int HD>
__device__ __forceinline__ float wave_weights(const float (*s_state)[REP][HD + 2], int hh, float (&w)[kAttnWaves]) {
    float M = kNegBig;
#pragma unroll
    for (int s = 0; s < kAttnWaves; ++s) M = fmaxf(M, s_state[s][hh][0]);
#pragma unroll
    for (int s = 0; s < kAttnWaves; ++s) w[s] = fast_exp2(s_state[s][hh][0] - M);
    return M;
}

// sum_s w[s] * (state element e of wave s), e = 1: l, e = 2 + d: acc[d]; in wave order.
template <int REP, int HD>
__device__ __forceinline__ float wave_sum(const float (*s_state)[REP][HD + 2], int hh, int e,
                                          const float (&w)[kAttnWaves]) {
    float v = 0.0f;
#pragma unroll
    for (int s = 0; s < kAttnWaves; ++s) v = fmaf(s_state[s][hh][e], w[s], v);
    return v;
}

// out[h,d] = (sum_s acc_s[d] 2^(m_s-M)) / (sum_s l_s 2^(m_s-M)) over the ns
// split states of the KV head's query heads h0 .. h0+rep-1, M = max_s m_s.
// Thread o takes output (o / HD, o % HD). Its first B split values are
// requested before the (m, l) pairs, which go to LDS, so both arrive in one
// memory round trip (more only past B splits or 512 outputs); every sum runs
// over the splits in ascending order: deterministic. B = 8, 16 or 32, the
// smallest that holds ns (a wave-uniform choice): a batch longer than ns
// repeats split 0's loads, and repeated loads of one address queue behind
// each other.
constexpr int kCombineMaxSplits = kAttnTargetGroups;  // nsplit <= kAttnTargetGroups by construction of the plan
constexpr int kCombineBatch = 32;

// COHERENT: the states were written device-coherent in this launch by workgroups that may run on other XCDs
// (the in-launch combine after the arrival), so they are read device-coherent too; across a launch boundary
// plain loads see them.
template <bool COHERENT>
__device__ __forceinline__ float part_load(const float* p) {
    if constexpr (COHERENT)
        return ld_agent(p);
    else
        return ldg(p);
}

template <int NT, int HD, bool COHERENT, int B>
__device__ __forceinline__ void combine_kv_b(const float* __restrict__ part, uint16_t* __restrict__ out, int h0,
                                             int rep, int nsplit, int ns, float* s_m, float* s_l) {
    constexpr int stride = HD + 2;
    const int tid = threadIdx.x;
    const int nout = rep * HD;
    float v[B];
    {
        const int o = tid < nout ? tid : 0;
        const float* po = part + static_cast<int64_t>(h0 + o / HD) * nsplit * stride + 2 + o % HD;
#pragma unroll
        for (int s = 0; s < B; ++s) v[s] = part_load<COHERENT>(po + static_cast<int64_t>(s < ns ? s : 0) * stride);
    }
    for (int i = tid; i < rep * ns; i += NT) {
        const int hh = i / ns, sp = i % ns;
        const float* ps = part + (static_cast<int64_t>(h0 + hh) * nsplit + sp) * stride;
        s_m[hh * kCombineMaxSplits + sp] = part_load<COHERENT>(ps);
        s_l[hh * kCombineMaxSplits + sp] = part_load<COHERENT>(ps + 1);
    }
    __syncthreads();  // (m, l) of every split in LDS
    for (int o = tid; o < nout; o += NT) {
        const int hh = o / HD;
        const float* sm = s_m + hh * kCombineMaxSplits;
        const float* sl = s_l + hh * kCombineMaxSplits;
        const float* po = part + static_cast<int64_t>(h0 + hh) * nsplit * stride + 2 + o % HD;
        float M = kNegBig;
        for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, sm[sp]);
        float lsum = 0.0f, acc = 0.0f;
        for (int b0 = 0; b0 < ns; b0 += B) {
            if (o != tid || b0 > 0) {  // the first batch of the first output is already in v
#pragma unroll
                for (int s = 0; s < B; ++s)
                    v[s] = part_load<COHERENT>(po + static_cast<int64_t>(b0 + s < ns ? b0 + s : 0) * stride);
            }
#pragma unroll
            for (int s = 0; s < B; ++s) {
                if (b0 + s >= ns) break;
                const float w = fast_exp2(sm[b0 + s] - M);
                lsum = fmaf(sl[b0 + s], w, lsum);
                acc = fmaf(v[s], w, acc);
            }
        }
        stg(out + static_cast<int64_t>(h0 + hh) * HD + o % HD, f32_to_f16_bits(acc / lsum));
    }
}

template <int NT, int HD, bool COHERENT = false>
__device__ __forceinline__ void combine_kv(const float* __restrict__ part, uint16_t* __restrict__ out, int h0, int rep,
                                           int nsplit, int ns, float* s_m, float* s_l) {
    if (ns <= 8)
        combine_kv_b<NT, HD, COHERENT, 8>(part, out, h0, rep, nsplit, ns, s_m, s_l);
    else if (ns <= 16)
        combine_kv_b<NT, HD, COHERENT, 16>(part, out, h0, rep, nsplit, ns, s_m, s_l);
    else
        combine_kv_b<NT, HD, COHERENT, kCombineBatch>(part, out, h0, rep, nsplit, ns, s_m, s_l);
}

struct AttnArgs {
    // PRE = false: q [NQ, hd]; PRE = true: qkv [q | k | v], q_norm, k_norm, cos/sin tables [S, hd/2]
    const uint16_t* q;
    const uint16_t* q_norm;
    const uint16_t* k_norm;
    const float* cos_t;
    const float* sin_t;
    const int32_t* pos;  // null: host length L_arg
    uint16_t* kc;
    uint16_t* vc;
    float* part;
    uint32_t* counters;
    uint16_t* out;
    int rep, NQ, NKV, S, L_arg, nsplit;
    int defer;       // 1: a split context leaves its states in the workspace (no arrival, no combine, out unwritten)
    int head_split;  // 1: workgroup x takes query head x / NKV of KV head x % NKV alone (grid NQ x splits)
    float eps, scale_log2;
};

// PRE (the decode engine's step): per workgroup, q/k RMSNorm + RoPE of the
// fused projection at position p = pos[0] (the rounding points of
// qk_norm_rope_append), the KV append of k, v at p by the workgroup whose
// range holds p (which also takes timestep p from LDS, not from the cache it
// is writing). counters[kvh] must be 0 before the launch; the last split
// resets it.
template <int LPR, int REP, bool PRE>
__global__ __launch_bounds__(kAttnThreads) void attn_kernel(const AttnArgs a) {
    constexpr int HD = LPR * 8;
    constexpr int HALF = HD / 2;
    constexpr int RPI = kWave / LPR;  // timesteps per wave instruction
    constexpr int STEP = RPI * kAttnWaves;
    __shared__ float s_state[kAttnWaves][REP][HD + 2];
    __shared__ __attribute__((aligned(16))) uint16_t s_q[PRE ? REP : 1][HD];
    __shared__ __attribute__((aligned(16))) uint16_t s_kv[2][HD];
    __shared__ float s_cm[REP * kCombineMaxSplits], s_cl[REP * kCombineMaxSplits];
    __shared__ int s_last;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane / LPR, u = lane % LPR;
    const int split = blockIdx.y;
    const int rep = a.rep, S = a.S;
    // the query heads of this workgroup: kvh * rep + hq0 + hh, hh < nhq. With head_split the rep workgroups of a
    // KV head are NKV apart in x, so (NKV a multiple of 8) they run on one XCD and share the K/V rows in its L2
    const int gx = blockIdx.x;
    const int kvh = a.head_split ? gx % a.NKV : gx;
    const int hq0 = a.head_split ? gx / a.NKV : 0;
    const int nhq = a.head_split ? 1 : rep;
    int p = -1;
    int L;
    // PRE: the position is requested first (a scalar load), then the operands of the wave's first head (a query
    // head, or the new k), which do not depend on it, so its RMSNorm does not wait for the position. The RoPE
    // table rows and the K/V rows follow once it is known. (Requesting split 0's first K/V rows before the
    // position as well measured slower: loads return in order, so the table rows then wait for the K/V rows.)
    if (PRE) p = ldg(a.pos);
    const uint16_t* kbase = a.kc + static_cast<int64_t>(kvh) * S * HD;  // this KV head's cache
    const uint16_t* vbase = a.vc + static_cast<int64_t>(kvh) * S * HD;
    auto head_src = [&](int hh) {
        return a.q + static_cast<int64_t>(hh == nhq ? a.NQ + kvh : kvh * rep + hq0 + hh) * HD;
    };
    uint16_t f_x1 = 0, f_x2 = 0, f_w1 = 0, f_w2 = 0;
    float f_c = 0.0f, f_sn = 0.0f;
    if (PRE && HALF == kWave && wave <= nhq) {  // wave-uniform; wave nhq's new k is used only next to p
        const int fh = wave;
        const uint16_t* src = head_src(fh);
        const uint16_t* wn = fh == nhq ? a.k_norm : a.q_norm;
        f_x1 = ldg(src + lane);
        f_x2 = ldg(src + lane + HALF);
        f_w1 = ldg(wn + lane);
        f_w2 = ldg(wn + lane + HALF);
    }
    if (PRE) {
        L = p < 0 ? 1 : (p >= S ? S : p + 1);
    } else {
        L = cur_len_of(a.L_arg, a.pos, S);
    }
    int tps, ns;
    split_plan(L, a.NKV, STEP, tps, ns);
    if (split >= ns) return;  // inactive split: no state, no arrival
    const int t0 = split * tps;
    const int t1 = min(L, t0 + tps);
    const bool pvalid = PRE && p >= 0 && p < S;
    const bool has_new = pvalid && p >= t0 && p < t1;
    const int tnew = has_new ? p : -1;

    const int tb0 = t0 + wave * RPI;
    const int npass_all = (t1 - t0 + STEP - 1) / STEP;
    // PRE: q heads kvh*rep + hq0 + hh (and, in the workgroup holding p, the new k) are normed and rotated; wave w
    // takes heads w, w+8, ... With head_dim 128 (one pair per lane) the operands of the wave's first head are
    // in flight already (above), and the table rows are requested before the K/V rows, so its RMSNorm and RoPE
    // run while the rows are.
    const int prow = pvalid ? p : (p < 0 ? 0 : S - 1);  // RoPE table row
    const int nh = PRE ? nhq + (has_new ? 1 : 0) : 0;
    if (PRE && HALF == kWave && wave < nh) {  // wave-uniform
        f_c = ldg(a.cos_t + static_cast<int64_t>(prow) * HALF + lane);
        f_sn = ldg(a.sin_t + static_cast<int64_t>(prow) * HALF + lane);
    }
    // without PRE the query heads are requested first: loads return in order, and the first pass's scores need
    // them, so they do not wait behind every pass's K/V rows
    u32x4 qraw[REP];
    if (!PRE) {
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            const int h = kvh * rep + hq0 + (hh < nhq ? hh : 0);
            qraw[hh] = ldg(reinterpret_cast<const u32x4*>(a.q + static_cast<int64_t>(h) * HD) + u);
        }
    }
    // the K/V rows of the first chunk: they do not depend on q (row p is patched from LDS later)
    AttnRows<LPR> rows;
    rows.load(kbase, vbase, tb0, t1, npass_all < kAttnPassMax ? npass_all : kAttnPassMax);
    // the operands pass through an empty asm here, so no conversion of them (and no wait for them) is placed
    // above the row requests
    if constexpr (PRE && HALF == kWave)
        asm volatile("" : "+v"(f_x1), "+v"(f_x2), "+v"(f_w1), "+v"(f_w2), "+v"(f_c), "+v"(f_sn));

    f16x2 qv[REP][4];
    if (PRE) {
        // Lane l reduces elements l, l+64, ... in that order (the order of qk_norm_rope_append).
        for (int hh = wave; hh < nh; hh += kAttnWaves) {
            const bool isk = hh == nhq;
            const uint16_t* src = head_src(hh);
            const uint16_t* wn = isk ? a.k_norm : a.q_norm;
            uint16_t* dst = isk ? s_kv[0] : s_q[hh];
            const float* cr = a.cos_t + static_cast<int64_t>(prow) * HALF;
            const float* sr = a.sin_t + static_cast<int64_t>(prow) * HALF;
            if (HALF == kWave) {  // one pair per lane
                if (hh != wave) {  // a later head of this wave (rep 8 with the new k): its operands now
                    f_x1 = ldg(src + lane);
                    f_x2 = ldg(src + lane + HALF);
                    f_w1 = ldg(wn + lane);
                    f_w2 = ldg(wn + lane + HALF);
                    f_c = ldg(cr + lane);
                    f_sn = ldg(sr + lane);
                }
                const float x1 = f16_bits_to_f32(f_x1), x2 = f16_bits_to_f32(f_x2);
                const float w1 = f16_bits_to_f32(f_w1), w2 = f16_bits_to_f32(f_w2);
                const float inv = rsqrtf(wave_sum_bcast(fmaf(x2, x2, x1 * x1)) / static_cast<float>(HD) + a.eps);
                const float xa = f16_bits_to_f32(f32_to_f16_bits(x1 * inv * w1));
                const float xb = f16_bits_to_f32(f32_to_f16_bits(x2 * inv * w2));
                float o1, o2;
                rope_pair(xa, xb, f_c, f_sn, o1, o2);
                dst[lane] = f32_to_f16_bits(o1);
                dst[lane + HALF] = f32_to_f16_bits(o2);
            } else {
                float ss = 0.0f;
                for (int i = lane; i < HD; i += kWave) {
                    const float v = f16_bits_to_f32(ldg(src + i));
                    ss = fmaf(v, v, ss);
                }
                const float inv = rsqrtf(wave_sum_bcast(ss) / static_cast<float>(HD) + a.eps);
                for (int i = lane; i < HALF; i += kWave) {
                    const float xa = f16_bits_to_f32(
                        f32_to_f16_bits(f16_bits_to_f32(ldg(src + i)) * inv * f16_bits_to_f32(ldg(wn + i))));
                    const float xb = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(ldg(src + i + HALF)) * inv *
                                                                     f16_bits_to_f32(ldg(wn + i + HALF))));
                    const float c = ldg(cr + i), sn = ldg(sr + i);
                    float o1, o2;
                    rope_pair(xa, xb, c, sn, o1, o2);
                    dst[i] = f32_to_f16_bits(o1);
                    dst[i + HALF] = f32_to_f16_bits(o2);
                }
            }
        }
        if (has_new) {
            const uint16_t* vsrc = a.q + static_cast<int64_t>(a.NQ + a.NKV + kvh) * HD;
            for (int i = tid; i < HD; i += kAttnThreads) s_kv[1][i] = ldg(vsrc + i);
        }
        __syncthreads();
        if (has_new && hq0 == 0) {  // append k, v at p (one workgroup per KV head)
            uint16_t* kd = a.kc + (static_cast<int64_t>(kvh) * S + p) * HD;
            uint16_t* vd = a.vc + (static_cast<int64_t>(kvh) * S + p) * HD;
            for (int i = tid; i < HD; i += kAttnThreads) {
                stg(kd + i, s_kv[0][i]);
                stg(vd + i, s_kv[1][i]);
            }
        }
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            const u32x4 t = reinterpret_cast<const u32x4*>(s_q[hh < nhq ? hh : 0])[u];
            qv[hh][0] = as_f16x2(t.x);
            qv[hh][1] = as_f16x2(t.y);
            qv[hh][2] = as_f16x2(t.z);
            qv[hh][3] = as_f16x2(t.w);
        }
    } else {
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            const u32x4 t = qraw[hh];
            qv[hh][0] = as_f16x2(t.x);
            qv[hh][1] = as_f16x2(t.y);
            qv[hh][2] = as_f16x2(t.z);
            qv[hh][3] = as_f16x2(t.w);
        }
    }

    AttnState<LPR, REP> st;
#pragma unroll
    for (int hh = 0; hh < REP; ++hh) {
        st.m[hh] = kNegBig;
        st.l[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < 8; ++d) st.acc[hh][d] = 0.0f;
    }
    // the new timestep's K / V (PRE, the workgroup holding p): taken from LDS instead of the rows read before
    // the append
    u32x4 knew = u32x4{0u, 0u, 0u, 0u}, vnew = knew;
    if (PRE && has_new) {  // workgroup-uniform
        knew = reinterpret_cast<const u32x4*>(s_kv[0])[u];
        vnew = reinterpret_cast<const u32x4*>(s_kv[1])[u];
    }
    // Per chunk of up to kAttnPassMax passes: the scores of every pass first (independent of each other), then
    // the running max moves once to cover them all (acc, l rescaled once), then the rows enter the sums. The
    // online-softmax recurrence of the reference with the chunk's rows as one step. Passes go in pairs: one
    // uniform branch per pair; the second pass of a pair past the chunk scores -inf.
    for (int c0 = 0; c0 < npass_all; c0 += kAttnPassMax) {
        const int left = npass_all - c0;
        const int np = left < kAttnPassMax ? left : kAttnPassMax;
        if (c0 > 0) rows.load(kbase, vbase, tb0 + c0 * STEP, t1, np);
        float sc[kAttnPassMax][REP];
#pragma unroll
        for (int i = 0; i < kAttnPassMax; i += 2) {
            if (i < np) {
#pragma unroll
                for (int j = i; j < i + 2; ++j) {
                    const int t = tb0 + (c0 + j) * STEP + g;
                    const u32x4 kk = (PRE && t == tnew) ? knew : rows.k[j];
                    attn_scores<LPR, REP>(sc[j], qv, j < np && t < t1, kk, a.scale_log2);
                }
            } else {
#pragma unroll
                for (int j = i; j < i + 2; ++j)
#pragma unroll
                    for (int hh = 0; hh < REP; ++hh) sc[j][hh] = -__builtin_inff();
            }
        }
#pragma unroll
        for (int hh = 0; hh < REP; ++hh) {
            float mn = st.m[hh];
#pragma unroll
            for (int j = 0; j < kAttnPassMax; ++j) mn = fmaxf(mn, sc[j][hh]);
            mn = groups_max<LPR>(mn);  // one running max for all the wave's lane groups
            const float corr = fast_exp2(st.m[hh] - mn);
            st.l[hh] *= corr;
#pragma unroll
            for (int d = 0; d < 8; ++d) st.acc[hh][d] *= corr;
            st.m[hh] = mn;
        }
#pragma unroll
        for (int i = 0; i < kAttnPassMax; i += 2) {
            if (i < np) {
#pragma unroll
                for (int j = i; j < i + 2; ++j) {
                    const int t = tb0 + (c0 + j) * STEP + g;
                    const u32x4 vv = (PRE && t == tnew) ? vnew : rows.v[j];
                    attn_accumulate<LPR, REP>(st, sc[j], vv);
                }
            }
        }
    }

    // the wave's state (its lane groups summed) into LDS
    attn_wave_state<LPR, REP, HD>(st, s_state[wave], lane);
    __syncthreads();

    if (ns == 1) {  // one workgroup holds the whole context: out = acc / l (the split combine with one state)
        for (int i = tid; i < nhq * HD; i += kAttnThreads) {
            const int hh = i / HD, d = i % HD;
            float w[kAttnWaves];
            wave_weights<REP, HD>(s_state, hh, w);
            const float lsum = wave_sum<REP, HD>(s_state, hh, 1, w);
            const float acc = wave_sum<REP, HD>(s_state, hh, 2 + d, w);
            stg(a.out + static_cast<int64_t>(kvh * rep + hq0 + hh) * HD + d, f32_to_f16_bits(acc / lsum));
        }
        return;
    }
    for (int i = tid; i < nhq * (HD + 2); i += kAttnThreads) {  // the split's state: [M, l, acc] per query head
        const int hh = i / (HD + 2), e = i % (HD + 2);
        float w[kAttnWaves];
        const float M = wave_weights<REP, HD>(s_state, hh, w);
        const float v = e == 0 ? M : wave_sum<REP, HD>(s_state, hh, e, w);
        float* dst = a.part + (static_cast<int64_t>(kvh * rep + hq0 + hh) * a.nsplit + split) * (HD + 2) + e;
        if (a.defer)
            stg(dst, v);  // read by the next launch
        else
            st_agent(dst, v);  // read in this launch by the last split, possibly on another XCD
    }
    if (a.defer) return;  // the consumer combines the states (gemv_attn_combine_kernel)
    // arrival: the last of the ns splits of this workgroup's heads combines them (one counter per x); the states
    // go out and come back device-coherent, so no L2 write-back or invalidate is needed (arrive_coherent)
    arrive_coherent();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(a.counters + gx, 1u);
        const bool last = prev + 1 == static_cast<uint32_t>(ns);
        if (last) atomicExch(a.counters + gx, 0u);
        s_last = last ? 1 : 0;
    }
    __syncthreads();
    if (!s_last) return;
    combine_kv<kAttnThreads, HD, true>(a.part, a.out, kvh * rep + hq0, nhq, a.nsplit, ns, s_cm, s_cl);
}

// Second launch of the host-length form: workgroup kvh combines the split states of its query heads with
// combine_kv (the arithmetic of the in-launch combine), after an attn_kernel launch with defer set; ns is the
// host's plan. An unsplit context wrote out itself. Across the launch boundary the states need no device fence
// or arrival counter.
template <int HD>
__global__ __launch_bounds__(kAttnThreads) void attn_combine_kernel(const float* __restrict__ part,
                                                                    uint16_t* __restrict__ out, int rep, int nsplit,
                                                                    int ns) {
    __shared__ float s_cm[8 * kCombineMaxSplits], s_cl[8 * kCombineMaxSplits];
    if (ns == 1) return;  // uniform
    combine_kv<kAttnThreads, HD>(part, out, static_cast<int>(blockIdx.x) * rep, rep, nsplit, ns, s_cm, s_cl);
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
    bool head_split;  // one query head per workgroup (grid x = NQ); else a KV head's query heads (x = NKV)
    int gx;
};

// L: the context length to plan for; with a device position, the largest one (max_seq).
static AttnPlan plan_attention(int64_t NQ, int64_t NKV, int64_t hd, int64_t L) {
    AttnPlan p{false, 0, 0, 0, 0, 0, 0, false, 0};
    const int64_t rep = NQ / NKV;
    const int64_t lpr = hd / 8;
    const bool pow2 = lpr >= 1 && (lpr & (lpr - 1)) == 0;
    if (hd % 8 == 0 && pow2 && lpr <= 32 && rep <= 8 && L * NKV < (int64_t(1) << 31)) {
        p.fast = true;
        p.lpr = static_cast<int>(lpr);
        p.gx = static_cast<int>(NKV);
        p.rep_t = rep <= 1 ? 1 : rep <= 2 ? 2 : rep <= 4 ? 4 : 8;
        p.step = static_cast<int>((kWave / lpr) * kAttnWaves);  // timesteps per workgroup pass
        split_plan(L, NKV, p.step, p.tps, p.nsplit);
        const int64_t by_len = ceil_div64(L, p.step), by_heads = ceil_div64(kAttnTargetGroups, NKV);
        p.cap = static_cast<int>(by_len < by_heads ? by_len : by_heads);
        if (p.cap < p.nsplit) p.cap = p.nsplit;
        if (p.cap < 1) p.cap = 1;
    }
    return p;
}

// A workgroup per query head (grid x = NQ): the query heads of a KV head share its K/V rows through L2 instead
// of one workgroup's registers, and each workgroup's passes do 1/rep of the score and sum work (the attention
// step at L = 192: 5.5 -> 4.7 us). Used where the split combine is not in the launch (the deferred step, the
// host-length form's second launch) or not needed; the in-launch combine keeps a workgroup per KV head, whose
// arrival and combine cost twice as much with twice the workgroups (10.2 -> 12.0 us at L = 2048, measured).
// Each query head's arithmetic does not depend on the layout, so both give the same bytes.
static void use_head_split(AttnPlan& p, int64_t NQ, int64_t NKV) {
    if (!p.fast || NQ == NKV) return;
    p.head_split = true;
    p.gx = static_cast<int>(NQ);
    p.rep_t = 1;
}

// Workspace: the split states [NQ, cap, hd + 2] fp32 (256-byte aligned), then
// one arrival counter per workgroup column, at most NQ (zero before the first
// call; every call leaves them zero).
static size_t attn_partial_bytes(int64_t NQ, int64_t hd, const AttnPlan& p) {
    const size_t b = static_cast<size_t>(NQ) * p.cap * (hd + 2) * sizeof(float);
    return (b + 255) & ~static_cast<size_t>(255);
}
static size_t attn_counter_bytes(int64_t NQ) {
    return (static_cast<size_t>(NQ) * sizeof(uint32_t) + 255) & ~static_cast<size_t>(255);
}

static int launch_attn_kernel(const AttnPlan& p, bool pre, dim3 grid, hipStream_t st, const AttnArgs& a) {
#define SOI_A(LL, RR)                                                                                        \
    do {                                                                                                     \
        if (pre)                                                                                             \
            hipLaunchKernelGGL((attn_kernel<LL, RR, true>), grid, dim3(kAttnThreads), 0, st, a);             \
        else                                                                                                 \
            hipLaunchKernelGGL((attn_kernel<LL, RR, false>), grid, dim3(kAttnThreads), 0, st, a);            \
    } while (0)
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
        default: SOI_AR(32); break;
    }
#undef SOI_AR
#undef SOI_A
    return SOI_OK;
}

static int launch_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                            int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim, int64_t cur_len,
                            const int32_t* pos, float scale, void* workspace, size_t workspace_bytes, hipStream_t st,
                            const char* what) {
    const float scale_log2 = scale * kLog2e;
    const int rep = static_cast<int>(NQ / NKV);
    // host length: plan for cur_len; device position: grid for every length up to max_seq, plan at run time
    AttnPlan p = plan_attention(NQ, NKV, head_dim, pos ? max_seq : cur_len);
    if (!pos) use_head_split(p, NQ, NKV);  // the host length combines in a second launch
    const bool aligned = aligned16(q) && aligned16(k_cache) && aligned16(v_cache);
    if (!p.fast || !aligned) {
        hipLaunchKernelGGL(attn_simple_kernel, dim3(static_cast<unsigned>(NQ)), dim3(64), 0, st, q, k_cache, v_cache,
                           out, rep, static_cast<int>(max_seq), static_cast<int>(head_dim),
                           static_cast<int>(cur_len), pos, scale_log2);
        return launch_status(what);
    }
    const int nsplit = pos ? p.cap : p.nsplit;
    const size_t pb = attn_partial_bytes(NQ, head_dim, p);
    const size_t need = pb + attn_counter_bytes(NQ);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) {
        set_last_error("%s: 16-byte aligned workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    AttnArgs a{};
    a.head_split = p.head_split ? 1 : 0;
    a.q = q;
    a.pos = pos;
    a.kc = const_cast<uint16_t*>(k_cache);  // read only in this form
    a.vc = const_cast<uint16_t*>(v_cache);
    a.part = static_cast<float*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + pb);
    a.out = out;
    a.rep = rep;
    a.NQ = static_cast<int>(NQ);
    a.NKV = static_cast<int>(NKV);
    a.S = static_cast<int>(max_seq);
    a.L_arg = static_cast<int>(cur_len);
    a.nsplit = nsplit;
    a.scale_log2 = scale_log2;
    // a host length that splits: the splits leave their states and a second launch combines them (cheaper at
    // long contexts than the device-scope release, arrival counter and acquire of the in-launch combine: 9.2
    // against 10.3 us at L = 2048). A device position keeps the in-launch combine: its grid can split at any
    // length, and a second launch would cost ~1.4 us at the unsplit lengths too.
    a.defer = (!pos && nsplit > 1) ? 1 : 0;
    launch_attn_kernel(p, false, dim3(static_cast<unsigned>(p.gx), static_cast<unsigned>(nsplit)), st, a);
    if (a.defer) {
#define SOI_AC(LL)                                                                                             \
    hipLaunchKernelGGL(attn_combine_kernel<LL * 8>, dim3(static_cast<unsigned>(NKV)), dim3(kAttnThreads), 0, st, \
                       a.part, out, rep, nsplit, nsplit)
        switch (p.lpr) {
            case 1: SOI_AC(1); break;
            case 2: SOI_AC(2); break;
            case 4: SOI_AC(4); break;
            case 8: SOI_AC(8); break;
            case 16: SOI_AC(16); break;
            default: SOI_AC(32); break;
        }
#undef SOI_AC
    }
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


// ---- o projection that finishes a deferred attention step ----
// With AttnArgs::defer a split context leaves out unwritten and its per-split
// states [m, l, acc] in the workspace; the INT4 GEMV that consumes the
// attention output (the o projection) combines them while its weight rows
// load. Workgroup = 8 waves, 1 row per wave; thread t owns x[4t .. 4t+3]
// (K = NQ * hd <= 2048, one query head per thread): it requests the states of
// its head (the first 8 or 16 splits: the smaller batch that holds the
// context's splits, since a longer batch repeats split 0's loads and repeated
// loads of one address queue behind each other) before the tile's weight loads,
// combines them with the arithmetic of combine_kv (M over all splits, then l
// and acc summed in split order, x = fp16(acc / l)) into LDS, and every wave
// reads its x chunks from there. An unsplit context (ns = 1) wrote out
// itself, and x is that vector. So y equals the plain GEMV of the attention
// output bit for bit.
constexpr int kOcWaves = 8;
constexpr int kOcThreads = kOcWaves * kWave;
constexpr int kOcRows = 1;  // 8 rows per workgroup: 256 workgroups (one per CU) for a 2048-row projection
constexpr int kOcBatch = 16;
constexpr int kOcMaxK = 4 * kOcThreads;

struct OcArgs {
    const float* part;         // [NQ, nsplit, hd + 2]
    const uint16_t* attn_out;  // [K] (written by an unsplit step)
    const int32_t* pos;
    int HD, NKV, S, step, nsplit;
};

__device__ __forceinline__ int attn_splits(const OcArgs& a, int L) {
    int tps, ns;
    split_plan(L, a.NKV, a.step, tps, ns);
    return ns;
}

// The split states of thread t's four x elements (ns > 1), combined into the LDS copy of x by finish(); the
// first B splits are held in registers.
template <int B>
struct AttnCombineState {
    int ns;   // splits of the current context
    int i0;   // first x element of the thread (clamped to K - 4; live = 4t < K)
    bool live;
    f32x2 ml[B];  // (m, l) of each split
    f32x4 va[B];  // acc[d0 .. d0+3] of each split

    __device__ __forceinline__ const float* rec(const OcArgs& a, int s) const {
        const int h = i0 / a.HD;
        return a.part + (static_cast<int64_t>(h) * a.nsplit + (s < ns ? s : 0)) * (a.HD + 2);
    }
    // Unconditional loads (clamped addresses): a branch around them would make the wave wait at its end.
    __device__ __forceinline__ void prefetch(const OcArgs& a, int K, int nsplits) {
        ns = nsplits;
        const int t4 = 4 * static_cast<int>(threadIdx.x);
        live = t4 < K;
        i0 = live ? t4 : K - 4;
        const int d0 = i0 % a.HD;
#pragma unroll
        for (int s = 0; s < B; ++s) {
            const float* r = rec(a, s);
            ml[s] = ldg(reinterpret_cast<const f32x2*>(r));
            const f32x2 a01 = ldg(reinterpret_cast<const f32x2*>(r + 2 + d0));  // 8-byte aligned only
            const f32x2 a23 = ldg(reinterpret_cast<const f32x2*>(r + 4 + d0));
            va[s] = f32x4{a01.x, a01.y, a23.x, a23.y};
        }
        __builtin_amdgcn_sched_barrier(0);  // every state load requested before the first use
    }
    // x[i0 .. i0+3] into s_x, then a workgroup barrier.
    __device__ __forceinline__ void finish(const OcArgs& a, uint16_t* s_x) const {
        float M = kNegBig;  // max is exact: any order gives combine_kv's M
#pragma unroll
        for (int s = 0; s < B; ++s)
            if (s < ns) M = fmaxf(M, ml[s].x);
        for (int s = B; s < ns; ++s) M = fmaxf(M, ldg(rec(a, s)));
        float lsum = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        const int d0 = i0 % a.HD;
#pragma unroll
        for (int s = 0; s < B; ++s) {
            if (s < ns) {
                const float w = fast_exp2(ml[s].x - M);
                lsum = fmaf(ml[s].y, w, lsum);
                acc[0] = fmaf(va[s].x, w, acc[0]);
                acc[1] = fmaf(va[s].y, w, acc[1]);
                acc[2] = fmaf(va[s].z, w, acc[2]);
                acc[3] = fmaf(va[s].w, w, acc[3]);
            }
        }
        for (int s = B; s < ns; ++s) {  // long contexts with few KV heads: further splits
            const float* r = rec(a, s);
            const float w = fast_exp2(ldg(r) - M);
            lsum = fmaf(ldg(r + 1), w, lsum);
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = fmaf(ldg(r + 2 + d0 + j), w, acc[j]);
        }
        u32x2 xo;
        xo.x = static_cast<uint32_t>(f32_to_f16_bits(acc[0] / lsum)) |
               (static_cast<uint32_t>(f32_to_f16_bits(acc[1] / lsum)) << 16);
        xo.y = static_cast<uint32_t>(f32_to_f16_bits(acc[2] / lsum)) |
               (static_cast<uint32_t>(f32_to_f16_bits(acc[3] / lsum)) << 16);
        if (live) *reinterpret_cast<u32x2*>(s_x + i0) = xo;
        __syncthreads();
    }
};

// The context's split states combined into the LDS copy of x (ns > 1; the batch choice is wave-uniform). The
// two branches start with different (empty) asm statements: with identical first instructions the compiler
// hoists split 0's loads above the branch and waits for them there, a round trip before the other loads.
__device__ __forceinline__ void attn_combine_into(const OcArgs& a, int K, int ns, uint16_t* s_x) {
    if (ns <= 8) {
        asm volatile("; combine batch 8" ::: "memory");
        AttnCombineState<8> st;
        st.prefetch(a, K, ns);
        st.finish(a, s_x);
    } else {
        asm volatile("; combine batch 16" ::: "memory");
        AttnCombineState<kOcBatch> st;
        st.prefetch(a, K, ns);
        st.finish(a, s_x);
    }
}

// x chunk c (32 elements) from the LDS copy of x (zeros for a chunk past K).
template <bool FULL>
__device__ __forceinline__ void lds_x_chunk(const uint16_t* s_x, int c, bool cv, f16x2 xv[16]) {
    const bool ok = FULL || cv;
    const u32x4* p = reinterpret_cast<const u32x4*>(s_x + 32 * (ok ? c : 0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u32x4 t = p[i];
        if (!ok) t = u32x4{0u, 0u, 0u, 0u};
        xv[4 * i + 0] = as_f16x2(t.x);
        xv[4 * i + 1] = as_f16x2(t.y);
        xv[4 * i + 2] = as_f16x2(t.z);
        xv[4 * i + 3] = as_f16x2(t.w);
    }
}

// General form (several passes, or K < 2048): x is final in LDS before the tile starts.
struct AttnLdsX {
    static constexpr bool kSinglePass = false;
    const uint16_t* s_x;
    const uint16_t* b;
    __device__ __forceinline__ const uint16_t* base() const { return b; }
    template <bool VEC, bool FULL>
    __device__ __forceinline__ void load(int, int c, bool cv, f16x2 xv[16]) const {
        lds_x_chunk<FULL>(s_x, c, cv, xv);
    }
};

// One-pass form (K == 2048, lane l's chunk is x[32l .. 32l+31]): the position and the lane's chunk of the
// step's out are requested before the tile's weight loads; load() runs after them: an unsplit context takes
// the chunk as x, a split one requests its states then (held by value: they stay in registers), combines
// them into LDS and reads the chunk from there.
struct AttnOnePassX {
    static constexpr bool kSinglePass = true;
    OcArgs oa;
    uint16_t* s_x;
    int p;        // pos[0]
    u32x4 xc[4];  // x[32l .. 32l+31] of out
    __device__ __forceinline__ const uint16_t* base() const { return oa.attn_out; }
    template <bool VEC, bool FULL>
    __device__ __forceinline__ void load(int K, int c, bool cv, f16x2 xv[16]) const {
        const int L = p < 0 ? 1 : (p >= oa.S ? oa.S : p + 1);  // cur_len_of
        const int ns = attn_splits(oa, L);
        if (ns == 1) {  // uniform over the grid
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[4 * i + 0] = as_f16x2(xc[i].x);
                xv[4 * i + 1] = as_f16x2(xc[i].y);
                xv[4 * i + 2] = as_f16x2(xc[i].z);
                xv[4 * i + 3] = as_f16x2(xc[i].w);
            }
            return;
        }
        attn_combine_into(oa, K, ns, s_x);
        lds_x_chunk<FULL>(s_x, c, cv, xv);
    }
};

template <bool ONEPASS, bool CS, bool FULL, class EP>
__global__ __launch_bounds__(kOcThreads) void gemv_attn_combine_kernel(DenseRows rows, int64_t N, OcArgs oa, EP ep,
                                                                       int K, int gs) {
    __shared__ __attribute__((aligned(16))) uint16_t s_x[kOcMaxK];
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kOcWaves + (threadIdx.x >> 6)) * kOcRows;
    if constexpr (ONEPASS) {
        AttnOnePassX xs;
        xs.oa = oa;
        xs.s_x = s_x;
        xs.p = ldg(oa.pos);
        const u32x4* o4 = reinterpret_cast<const u32x4*>(oa.attn_out) + 4 * (threadIdx.x & (kWave - 1));
#pragma unroll
        for (int i = 0; i < 4; ++i) xs.xc[i] = ldg(o4 + i);
        gemv_int4_tile<kOcRows, 1, true, CS, true, FULL>(rows, N, xs, ep, K, gs, row0);
    } else {
        const int ns = attn_splits(oa, cur_len_of(0, oa.pos, oa.S));
        if (ns == 1) {  // the step wrote out itself (uniform over the grid): the plain GEMV of it
            gemv_int4_tile<kOcRows, 1, true, CS, true, FULL>(rows, N, PlainX{oa.attn_out}, ep, K, gs, row0);
            return;
        }
        attn_combine_into(oa, K, ns, s_x);
        gemv_int4_tile<kOcRows, 1, true, CS, true, FULL>(rows, N, AttnLdsX{s_x, oa.attn_out}, ep, K, gs, row0);
    }
}

template <class EP>
static int launch_attn_combine(const uint8_t* Wq, const float* scale, const void* workspace, size_t workspace_bytes,
                               const uint16_t* attn_out, const int32_t* pos, int64_t NQ, int64_t NKV,
                               int64_t head_dim, int64_t max_seq, const EP& ep, int64_t N, int64_t group_size,
                               int64_t num_groups, void* stream, const char* what) {
    SOI_REQUIRE(NQ >= 1 && NKV >= 1 && NQ % NKV == 0, "%s: num_q_heads must be a positive multiple of num_kv_heads",
                what);
    SOI_REQUIRE(max_seq >= 1 && max_seq <= (int64_t(1) << 30), "%s: max_seq_len out of range", what);
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, max_seq);
    SOI_REQUIRE(p.fast, "%s: head_dim %lld / GQA ratio %lld not supported by the deferred attention step", what,
                (long long)head_dim, (long long)(NQ / NKV));
    const int64_t K = NQ * head_dim;
    SOI_REQUIRE(K % 32 == 0 && K <= kOcMaxK, "%s: num_q_heads * head_dim must be a multiple of 32 and at most %d",
                what, kOcMaxK);
    SOI_REQUIRE(group_size >= 8 && group_size % 8 == 0, "%s: group_size must be a positive multiple of 8", what);
    SOI_REQUIRE(num_groups == ceil_div64(K, group_size), "%s: num_groups must be ceil(K / group_size)", what);
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    SOI_REQUIRE(Wq && scale && workspace && attn_out && pos, "%s: null pointer", what);
    SOI_REQUIRE(aligned16(Wq) && aligned16(attn_out) && aligned16(workspace),
                "%s: Wq, attn_out and workspace must be 16-byte aligned", what);
    const size_t need = attn_partial_bytes(NQ, head_dim, p);
    if (workspace_bytes < need) {
        set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    if (N == 0) return SOI_OK;
    OcArgs oa{static_cast<const float*>(workspace), attn_out, pos, static_cast<int>(head_dim),
              static_cast<int>(NKV), static_cast<int>(max_seq), p.step, p.cap};
    const DenseRows rows{Wq, scale, (K / 8) * 4, num_groups};
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, kOcWaves * kOcRows)));
    hipStream_t st = as_stream(stream);
    const bool one = K == 32 * kWave, cs = group_size % 32 == 0;  // one 64-chunk pass
    const bool full = N % (kOcWaves * kOcRows) == 0 && K % (32 * kWave) == 0;
    const int Ki = static_cast<int>(K), gi = static_cast<int>(group_size);
#define SOI_OC(O, C, F) \
    hipLaunchKernelGGL((gemv_attn_combine_kernel<O, C, F, EP>), grid, dim3(kOcThreads), 0, st, rows, N, oa, ep, Ki, gi)
    if (one && cs && full) SOI_OC(true, true, true);
    else if (cs && full) SOI_OC(false, true, true);
    else if (cs) SOI_OC(false, true, false);
    else SOI_OC(false, false, false);
#undef SOI_OC
    return launch_status(what);
}

}  // namespace soi

using namespace soi;

extern "C" size_t soi_decode_attention_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t cur_len) {
    if (NQ <= 0 || NKV <= 0 || head_dim <= 0 || cur_len <= 0 || NQ % NKV) return 0;
    const AttnPlan p = plan_attention(NQ, NKV, head_dim, cur_len);  // covers the device form with max_seq = cur_len
    if (!p.fast) return 0;
    return attn_partial_bytes(NQ, head_dim, p) + attn_counter_bytes(NQ);
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

extern "C" size_t soi_decode_attention_step_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim,
                                                            int64_t max_seq) {
    return soi_decode_attention_workspace_bytes(NQ, NKV, head_dim, max_seq);
}

static int attention_step(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                          const float* cos_table, const float* sin_table, const int32_t* pos, uint16_t* k_cache,
                          uint16_t* v_cache, uint16_t* out, int64_t NQ, int64_t NKV, int64_t max_seq,
                          int64_t head_dim, float eps, float scale, void* workspace, size_t workspace_bytes,
                          void* stream, bool defer, const char* what) {
    int st = check_attention(qkv, k_cache, v_cache, out, NQ, NKV, max_seq, head_dim, what);
    if (st) return st;
    SOI_REQUIRE(q_norm && k_norm && cos_table && sin_table && pos, "%s: null pointer", what);
    AttnPlan p = plan_attention(NQ, NKV, head_dim, max_seq);
    if (defer) use_head_split(p, NQ, NKV);  // the o projection combines the split states
    if (!p.fast || !aligned16(qkv) || !aligned16(k_cache) || !aligned16(v_cache)) {
        set_last_error("%s: head_dim %lld / GQA ratio %lld / alignment not supported by the one-launch form", what,
                       (long long)head_dim, (long long)(NQ / NKV));
        return SOI_ERR_UNSUPPORTED;
    }
    const size_t pb = attn_partial_bytes(NQ, head_dim, p);
    const size_t need = pb + attn_counter_bytes(NQ);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) {
        set_last_error("%s: 16-byte aligned workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    AttnArgs a{};
    a.head_split = p.head_split ? 1 : 0;
    a.q = qkv;
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.cos_t = cos_table;
    a.sin_t = sin_table;
    a.pos = pos;
    a.kc = k_cache;
    a.vc = v_cache;
    a.part = static_cast<float*>(workspace);
    a.counters = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + pb);
    a.out = out;
    a.rep = static_cast<int>(NQ / NKV);
    a.NQ = static_cast<int>(NQ);
    a.NKV = static_cast<int>(NKV);
    a.S = static_cast<int>(max_seq);
    a.nsplit = p.cap;
    a.defer = defer ? 1 : 0;
    a.eps = eps;
    a.scale_log2 = scale * kLog2e;
    launch_attn_kernel(p, true, dim3(static_cast<unsigned>(p.gx), static_cast<unsigned>(p.cap)), as_stream(stream), a);
    return launch_status(what);
}

extern "C" int soi_decode_attention_step(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                                         const float* cos_table, const float* sin_table, const int32_t* pos,
                                         uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, int64_t NQ,
                                         int64_t NKV, int64_t max_seq, int64_t head_dim, float eps, float scale,
                                         void* workspace, size_t workspace_bytes, void* stream) {
    return attention_step(qkv, q_norm, k_norm, cos_table, sin_table, pos, k_cache, v_cache, out, NQ, NKV, max_seq,
                          head_dim, eps, scale, workspace, workspace_bytes, stream, false, "soi_decode_attention_step");
}

extern "C" int soi_decode_attention_step_deferred(const uint16_t* qkv, const uint16_t* q_norm,
                                                  const uint16_t* k_norm, const float* cos_table,
                                                  const float* sin_table, const int32_t* pos, uint16_t* k_cache,
                                                  uint16_t* v_cache, uint16_t* out, int64_t NQ, int64_t NKV,
                                                  int64_t max_seq, int64_t head_dim, float eps, float scale,
                                                  void* workspace, size_t workspace_bytes, void* stream) {
    return attention_step(qkv, q_norm, k_norm, cos_table, sin_table, pos, k_cache, v_cache, out, NQ, NKV, max_seq,
                          head_dim, eps, scale, workspace, workspace_bytes, stream, true,
                          "soi_decode_attention_step_deferred");
}

extern "C" int soi_gemv_w4a16_attn_combine(const uint8_t* Wq, const float* scale, const void* workspace,
                                           size_t workspace_bytes, const uint16_t* attn_out, const int32_t* pos,
                                           int64_t NQ, int64_t NKV, int64_t head_dim, int64_t max_seq, uint16_t* y,
                                           const uint16_t* res, uint16_t* res_out, int64_t N, int64_t group_size,
                                           int64_t num_groups, void* stream) {
    const char* what = "soi_gemv_w4a16_attn_combine";
    SOI_REQUIRE(y, "%s: null pointer", what);
    SOI_REQUIRE(!res == !res_out, "%s: res and res_out go together", what);
    if (res)
        return launch_attn_combine(Wq, scale, workspace, workspace_bytes, attn_out, pos, NQ, NKV, head_dim, max_seq,
                                   StoreYAdd{y, res, res_out}, N, group_size, num_groups, stream, what);
    return launch_attn_combine(Wq, scale, workspace, workspace_bytes, attn_out, pos, NQ, NKV, head_dim, max_seq,
                               StoreY{y}, N, group_size, num_groups, stream, what);
}
