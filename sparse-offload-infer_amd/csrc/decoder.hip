// Decoder-step glue for batch-1 decode on gfx950: RMSNorm (optionally fused
// with the residual add), RoPE, KV-cache append, the fp16 GEMV of the LM
// head, argmax, SiLU gating, embedding lookup and the device-resident
// position counter.
//
// Restated from the reference's decode step (python/soinfer/runtime/
// generate.py:141-182, 276-310, 429-463) and its kernels (rmsnorm.cu:9-48,
// rope.cu:5-25, kv_cache.cu:7-27, gemv_fp16.cu:60-95). The engine forms read
// the token and the position from device memory, so one captured HIP graph
// replays every decode step with no host round trip.
//
// Rounding points follow the reference: every op writes binary16; the
// residual add is a binary16 add (fp32 sum of two binary16 values rounded to
// binary16, which equals the correctly rounded binary16 sum); RMSNorm,
// RoPE, SiLU and the GEMV compute in fp32.
#include "soi_device.h"
#include "soi_host.h"

namespace soi {

constexpr int kNormThreads = 256;
constexpr int kNormWaves = kNormThreads / kWave;

// Sum over a 256-thread workgroup in a fixed order (DPP inside each wave,
// then waves in order). Every thread gets the total.
__device__ __forceinline__ float block_sum_256(float v, float* s_red) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    v = wave_sum_bcast(v);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < kNormWaves; ++w) t += s_red[w];
    return t;
}

// One workgroup per row. ADD: the row is v = x + delta (binary16), x is
// replaced by v, and the normalised row is computed from v. Both passes read
// the original x and delta (the update is written in the second pass), so no
// thread reads memory written in the same launch. VEC: hidden % 8 == 0 and
// all pointers 16-byte aligned.
template <bool ADD, bool VEC>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ delta,
                                                               const uint16_t* __restrict__ w,
                                                               uint16_t* __restrict__ out, int hidden, float eps,
                                                               int32_t* __restrict__ advance_pos) {
    // engine form: the last op of a decode step also moves the device position (no kernel of this
    // launch reads it; every earlier launch on the stream has completed)
    if (advance_pos && blockIdx.x == 0 && threadIdx.x == 0) stg(advance_pos, ldg(advance_pos) + 1);
    __shared__ float s_red[kNormWaves];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * hidden;
    uint16_t* xr = x + base;
    uint16_t* orow = out + base;
    float ss = 0.0f;
    if (VEC) {
        const u32x4* x4 = reinterpret_cast<const u32x4*>(xr);
        const u32x4* d4 = ADD ? reinterpret_cast<const u32x4*>(delta + base) : nullptr;
        for (int c = threadIdx.x; c < (hidden >> 3); c += kNormThreads) {
            u32x4 v = ldg(x4 + c);
            if (ADD) {
                const u32x4 d = ldg(d4 + c);
                v.x = add_f16x2(v.x, d.x);
                v.y = add_f16x2(v.y, d.y);
                v.z = add_f16x2(v.z, d.z);
                v.w = add_f16x2(v.w, d.w);
            }
            ss += sumsq_f16x2(v.x) + sumsq_f16x2(v.y) + sumsq_f16x2(v.z) + sumsq_f16x2(v.w);
        }
    } else {
        for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
            float v = f16_bits_to_f32(ldg(xr + i));
            if (ADD) v = f16_bits_to_f32(f32_to_f16_bits(v + f16_bits_to_f32(ldg(delta + base + i))));
            ss = fmaf(v, v, ss);
        }
    }
    const float total = block_sum_256(ss, s_red);
    const float inv = rsqrtf(total / static_cast<float>(hidden) + eps);
    if (VEC) {
        u32x4* x4 = reinterpret_cast<u32x4*>(xr);
        const u32x4* d4 = ADD ? reinterpret_cast<const u32x4*>(delta + base) : nullptr;
        const u32x4* w4 = reinterpret_cast<const u32x4*>(w);
        u32x4* o4 = reinterpret_cast<u32x4*>(orow);
        for (int c = threadIdx.x; c < (hidden >> 3); c += kNormThreads) {
            u32x4 v = ldg(x4 + c);
            const u32x4 g = ldg(w4 + c);
            if (ADD) {
                const u32x4 d = ldg(d4 + c);
                v.x = add_f16x2(v.x, d.x);
                v.y = add_f16x2(v.y, d.y);
                v.z = add_f16x2(v.z, d.z);
                v.w = add_f16x2(v.w, d.w);
            }
            u32x4 r;
            r.x = norm_f16x2(v.x, g.x, inv);
            r.y = norm_f16x2(v.y, g.y, inv);
            r.z = norm_f16x2(v.z, g.z, inv);
            r.w = norm_f16x2(v.w, g.w, inv);
            stg(o4 + c, r);
            if (ADD) stg(x4 + c, v);
        }
    } else {
        for (int i = threadIdx.x; i < hidden; i += kNormThreads) {
            float v = f16_bits_to_f32(ldg(xr + i));
            if (ADD) v = f16_bits_to_f32(f32_to_f16_bits(v + f16_bits_to_f32(ldg(delta + base + i))));
            stg(orow + i, f32_to_f16_bits(v * inv * f16_bits_to_f32(ldg(w + i))));
            if (ADD) stg(xr + i, f32_to_f16_bits(v));
        }
    }
}

// RoPE, rotate-half convention, in place: for i < hd/2,
//   x[i] <- x[i] c_i - x[i+hd/2] s_i,  x[i+hd/2] <- x[i+hd/2] c_i + x[i] s_i
// (rounded as fma(x[i], c, -(x[i+hd/2] s)) and fma(x[i+hd/2], c, x[i] s)).
// One workgroup per head, one thread per pair.
__global__ void rope_kernel(uint16_t* __restrict__ x, const float* __restrict__ cs, const float* __restrict__ sn,
                            int head_dim) {
    const int half = head_dim >> 1;
    const int i = threadIdx.x;
    if (i >= half) return;
    uint16_t* row = x + static_cast<int64_t>(blockIdx.x) * head_dim;
    const float c = ldg(cs + i), s = ldg(sn + i);
    const float x1 = f16_bits_to_f32(ldg(row + i)), x2 = f16_bits_to_f32(ldg(row + i + half));
    float o1, o2;
    rope_pair(x1, x2, c, s, o1, o2);
    stg(row + i, f32_to_f16_bits(o1));
    stg(row + i + half, f32_to_f16_bits(o2));
}

// KV append at a host position (pos >= 0) or at pos_ptr[0] (device form).
__global__ void kv_append_kernel(const uint16_t* __restrict__ k_new, const uint16_t* __restrict__ v_new,
                                 uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int max_seq, int head_dim,
                                 int pos_arg, const int32_t* __restrict__ pos_ptr) {
    const int pos = pos_ptr ? ldg(pos_ptr) : pos_arg;
    if (pos < 0 || pos >= max_seq) return;
    const int h = blockIdx.x;
    const uint16_t* ks = k_new + static_cast<int64_t>(h) * head_dim;
    const uint16_t* vs = v_new + static_cast<int64_t>(h) * head_dim;
    uint16_t* kd = kc + (static_cast<int64_t>(h) * max_seq + pos) * head_dim;
    uint16_t* vd = vc + (static_cast<int64_t>(h) * max_seq + pos) * head_dim;
    for (int i = threadIdx.x; i < head_dim; i += blockDim.x) {
        stg(kd + i, ldg(ks + i));
        stg(vd + i, ldg(vs + i));
    }
}

// Engine form of the attention prologue of one layer, one workgroup per head:
// q heads -> RMSNorm(q_norm) -> RoPE -> q_out; k heads -> RMSNorm(k_norm) ->
// RoPE -> k_cache[kvh, pos]; v heads -> v_cache[kvh, pos]. qkv holds the
// fused projection [q (NQ*hd) | k (NKV*hd) | v (NKV*hd)]. The normalised
// values are rounded to binary16 before RoPE, as the separate ops do. RoPE
// angles come from tables cos/sin [max_seq, hd/2] at row pos.
__global__ __launch_bounds__(kNormThreads) void qk_norm_rope_append_kernel(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, const int32_t* __restrict__ pos_ptr,
    uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int NQ, int NKV,
    int max_seq, int head_dim, float eps) {
    const int pos = ldg(pos_ptr);
    if (pos < 0 || pos >= max_seq) return;  // uniform over the workgroup
    const int h = blockIdx.x;
    const int half = head_dim >> 1;
    const uint16_t* src = qkv + static_cast<int64_t>(h) * head_dim;
    if (h >= NQ + NKV) {  // v head: copy into the cache
        const int kvh = h - NQ - NKV;
        uint16_t* vd = vc + (static_cast<int64_t>(kvh) * max_seq + pos) * head_dim;
        for (int i = threadIdx.x; i < head_dim; i += kNormThreads) stg(vd + i, ldg(src + i));
        return;
    }
    const uint16_t* wn = h < NQ ? q_norm : k_norm;
    // every wave computes the same mean square (lanes stride 64 over the head), the reduction order of
    // the one-launch attention step, so the two forms give identical values
    const int lane = threadIdx.x & 63;
    float ss = 0.0f;
    for (int i = lane; i < head_dim; i += kWave) {
        const float v = f16_bits_to_f32(ldg(src + i));
        ss = fmaf(v, v, ss);
    }
    const float inv = rsqrtf(wave_sum_bcast(ss) / static_cast<float>(head_dim) + eps);
    uint16_t* dst = h < NQ ? q_out + static_cast<int64_t>(h) * head_dim
                           : kc + (static_cast<int64_t>(h - NQ) * max_seq + pos) * head_dim;
    const float* cr = cos_t + static_cast<int64_t>(pos) * half;
    const float* sr = sin_t + static_cast<int64_t>(pos) * half;
    for (int i = threadIdx.x; i < half; i += kNormThreads) {
        const float a = f16_bits_to_f32(
            f32_to_f16_bits(f16_bits_to_f32(ldg(src + i)) * inv * f16_bits_to_f32(ldg(wn + i))));
        const float b = f16_bits_to_f32(f32_to_f16_bits(f16_bits_to_f32(ldg(src + i + half)) * inv *
                                                        f16_bits_to_f32(ldg(wn + i + half))));
        const float c = ldg(cr + i), s = ldg(sr + i);
        float o1, o2;
        rope_pair(a, b, c, s, o1, o2);
        stg(dst + i, f32_to_f16_bits(o1));
        stg(dst + i + half, f32_to_f16_bits(o2));
    }
}

// fp16 GEMV y[N] = W[N,K] x[K], fp32 accumulation (LM head). Same work
// layout as the INT4 GEMV: R rows per wave, lane owns 16-byte chunk l of each
// 64-chunk pass, PU passes loaded before the arithmetic, transposed row
// reduction. VEC: K % 8 == 0 and 16-byte aligned W and x.
template <int R, int PU, bool FULL>
__global__ __launch_bounds__(64) void gemv_f16_kernel(const uint16_t* __restrict__ W, const uint16_t* __restrict__ x,
                                                      uint16_t* __restrict__ y, int64_t N, int K) {
    const int lane = threadIdx.x;
    const int chunks = K >> 3;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
    const u32x4* z = reinterpret_cast<const u32x4*>(g_zero16);
    const u32x4* x4 = reinterpret_cast<const u32x4*>(x);
    const u32x4* wr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (FULL || row0 + r < N) ? row0 + r : N - 1;
        wr[r] = reinterpret_cast<const u32x4*>(W + row * K);
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += kWave * PU) {
        u32x4 wv[PU][R], xv[PU];
#pragma unroll
        for (int p = 0; p < PU; ++p) {
            const int c = c0 + p * kWave + lane;
            const bool ok = FULL || c < chunks;
            xv[p] = ldg(ok ? x4 + c : z);
#pragma unroll
            for (int r = 0; r < R; ++r) wv[p][r] = ldg_stream(ok ? wr[r] + c : z);
        }
#pragma unroll
        for (int p = 0; p < PU; ++p) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float a = acc[r];
                a = dot2(as_f16x2(wv[p][r].x), as_f16x2(xv[p].x), a);
                a = dot2(as_f16x2(wv[p][r].y), as_f16x2(xv[p].y), a);
                a = dot2(as_f16x2(wv[p][r].z), as_f16x2(xv[p].z), a);
                a = dot2(as_f16x2(wv[p][r].w), as_f16x2(xv[p].w), a);
                acc[r] = a;
            }
        }
    }
    const float total = reduce_rows<R>(acc);
    const int r = reduce_rows_row<R>(static_cast<uint32_t>(lane));
    if ((lane & (64 / R - 1)) == 0 && (FULL || row0 + r < N)) stg(y + row0 + r, f32_to_f16_bits(total));
}

// Any K / alignment: one wave per row, lanes stride over k.
__global__ __launch_bounds__(64) void gemv_f16_simple_kernel(const uint16_t* __restrict__ W,
                                                             const uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ y, int K) {
    const int64_t row = blockIdx.x;
    const uint16_t* wr = W + row * K;
    float a = 0.0f;
    for (int k = threadIdx.x; k < K; k += kWave) a = fmaf(f16_bits_to_f32(ldg(wr + k)), f16_bits_to_f32(ldg(x + k)), a);
    a = wave_sum_bcast(a);
    if (threadIdx.x == 0) stg(y + row, f32_to_f16_bits(a));
}

// h[i] = fp16(silu(g_i) * u_i) with g = gate_W x and u = up_W x summed in fp32 over fp16 products. Both matrices'
// rows i stream through one wave, which reads each x chunk once for both; the SiLU and the product run on the
// reduced sums, so only h is written. R rows of each matrix per wave: R = 2 keeps 4 weight rows in flight, the
// same as the fp16 GEMV's 4-row tile, so the register footprint (and occupancy) matches it.
template <int R, int PU, bool FULL>
__global__ __launch_bounds__(64) void swiglu_gate_up_kernel(const uint16_t* __restrict__ Wg,
                                                            const uint16_t* __restrict__ Wu,
                                                            const uint16_t* __restrict__ x,
                                                            uint16_t* __restrict__ h, int64_t I, int H) {
    const int lane = threadIdx.x;
    const int chunks = H >> 3;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * R;
    const u32x4* z = reinterpret_cast<const u32x4*>(g_zero16);
    const u32x4* x4 = reinterpret_cast<const u32x4*>(x);
    const u32x4 *gr[R], *ur[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = (FULL || row0 + r < I) ? row0 + r : I - 1;
        gr[r] = reinterpret_cast<const u32x4*>(Wg + row * H);
        ur[r] = reinterpret_cast<const u32x4*>(Wu + row * H);
    }
    float ga[R], ua[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ga[r] = ua[r] = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += kWave * PU) {
        u32x4 gv[PU][R], uv[PU][R], xv[PU];
#pragma unroll
        for (int p = 0; p < PU; ++p) {
            const int c = c0 + p * kWave + lane;
            const bool ok = FULL || c < chunks;
            xv[p] = ldg(ok ? x4 + c : z);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                gv[p][r] = ldg_stream(ok ? gr[r] + c : z);
                uv[p][r] = ldg_stream(ok ? ur[r] + c : z);
            }
        }
#pragma unroll
        for (int p = 0; p < PU; ++p) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float a = ga[r], b = ua[r];
                a = dot2(as_f16x2(gv[p][r].x), as_f16x2(xv[p].x), a);
                b = dot2(as_f16x2(uv[p][r].x), as_f16x2(xv[p].x), b);
                a = dot2(as_f16x2(gv[p][r].y), as_f16x2(xv[p].y), a);
                b = dot2(as_f16x2(uv[p][r].y), as_f16x2(xv[p].y), b);
                a = dot2(as_f16x2(gv[p][r].z), as_f16x2(xv[p].z), a);
                b = dot2(as_f16x2(uv[p][r].z), as_f16x2(xv[p].z), b);
                a = dot2(as_f16x2(gv[p][r].w), as_f16x2(xv[p].w), a);
                b = dot2(as_f16x2(uv[p][r].w), as_f16x2(xv[p].w), b);
                ga[r] = a;
                ua[r] = b;
            }
        }
    }
    const float g = reduce_rows<R>(ga);
    const float u = reduce_rows<R>(ua);
    const int r = reduce_rows_row<R>(static_cast<uint32_t>(lane));
    if ((lane & (64 / R - 1)) == 0 && (FULL || row0 + r < I)) stg(h + row0 + r, f32_to_f16_bits(silu_f32(g) * u));
}

// Any H / alignment: one wave per row, lanes stride over k.
__global__ __launch_bounds__(64) void swiglu_gate_up_simple_kernel(const uint16_t* __restrict__ Wg,
                                                                   const uint16_t* __restrict__ Wu,
                                                                   const uint16_t* __restrict__ x,
                                                                   uint16_t* __restrict__ h, int H) {
    const int64_t row = blockIdx.x;
    const uint16_t* g = Wg + row * H;
    const uint16_t* u = Wu + row * H;
    float a = 0.0f, b = 0.0f;
    for (int k = threadIdx.x; k < H; k += kWave) {
        const float xk = f16_bits_to_f32(ldg(x + k));
        a = fmaf(f16_bits_to_f32(ldg(g + k)), xk, a);
        b = fmaf(f16_bits_to_f32(ldg(u + k)), xk, b);
    }
    a = wave_sum_bcast(a);
    b = wave_sum_bcast(b);
    if (threadIdx.x == 0) stg(h + row, f32_to_f16_bits(silu_f32(a) * b));
}

// argmax with torch.argmax's order: NaN above every number, ties -> lowest index.
__device__ __forceinline__ bool arg_better(float av, int ai, float bv, int bi) {
    const bool an = av != av, bn = bv != bv;
    if (an != bn) return an;
    if (!an && av != bv) return av > bv;
    return ai < bi;
}

__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        const float ov = __shfl_xor(v, m, kWave);
        const int oi = __shfl_xor(i, m, kWave);
        if (arg_better(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
}

constexpr int kArgmaxThreads = 256;
constexpr int kArgmaxPerBlock = 2048;  // one 16-byte load (8 values) per thread

__device__ __forceinline__ void block_argmax(float& v, int& i, float* s_v, int* s_i) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    wave_argmax(v, i);
    if (lane == 0) {
        s_v[wave] = v;
        s_i[wave] = i;
    }
    __syncthreads();
    v = s_v[0];
    i = s_i[0];
#pragma unroll
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
        if (arg_better(s_v[w], s_i[w], v, i)) {
            v = s_v[w];
            i = s_i[w];
        }
}

// Stage 1: workgroup b reduces [b*2048, (b+1)*2048) to one (value, index);
// VEC (n % 8 == 0, 16-byte aligned x): one 16-byte load per thread.
template <bool VEC>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_partial_kernel(const uint16_t* __restrict__ x, int n,
                                                                        float* __restrict__ pv,
                                                                        int* __restrict__ pi) {
    __shared__ float s_v[kArgmaxThreads / kWave];
    __shared__ int s_i[kArgmaxThreads / kWave];
    const int b0 = blockIdx.x * kArgmaxPerBlock;
    const int b1 = min(n, b0 + kArgmaxPerBlock);
    float v = -__builtin_inff();
    int i = 0x7fffffff;
    if (VEC) {
        const int j0 = b0 + 8 * threadIdx.x;
        if (j0 < b1) {
            const u32x4 t = ldg(reinterpret_cast<const u32x4*>(x + j0));
            const uint32_t wds[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const f16x2 h = as_f16x2(wds[e]);
                const float lo = static_cast<float>(h.x), hi = static_cast<float>(h.y);
                if (arg_better(lo, j0 + 2 * e, v, i)) {
                    v = lo;
                    i = j0 + 2 * e;
                }
                if (arg_better(hi, j0 + 2 * e + 1, v, i)) {
                    v = hi;
                    i = j0 + 2 * e + 1;
                }
            }
        }
    } else {
        for (int j = b0 + threadIdx.x; j < b1; j += kArgmaxThreads) {
            const float t = f16_bits_to_f32(ldg(x + j));
            if (arg_better(t, j, v, i)) {
                v = t;
                i = j;
            }
        }
    }
    block_argmax(v, i, s_v, s_i);
    if (threadIdx.x == 0) {
        stg(pv + blockIdx.x, v);
        stg(pi + blockIdx.x, i);
    }
}

// Stage 2: one workgroup reduces the partials; writes the index to out[0]
// and, when given, appends it to log[*log_len] and increments *log_len
// (log capacity log_cap; a full log is left unchanged).
__global__ __launch_bounds__(kArgmaxThreads) void argmax_final_kernel(const float* __restrict__ pv,
                                                                      const int* __restrict__ pi, int nb,
                                                                      int32_t* __restrict__ out,
                                                                      int32_t* __restrict__ log,
                                                                      int32_t* __restrict__ log_len, int log_cap) {
    __shared__ float s_v[kArgmaxThreads / kWave];
    __shared__ int s_i[kArgmaxThreads / kWave];
    float v = -__builtin_inff();
    int i = 0x7fffffff;
    for (int j = threadIdx.x; j < nb; j += kArgmaxThreads) {
        const float t = ldg(pv + j);
        const int ti = ldg(pi + j);
        if (arg_better(t, ti, v, i)) {
            v = t;
            i = ti;
        }
    }
    block_argmax(v, i, s_v, s_i);
    if (threadIdx.x == 0) {
        stg(out, static_cast<int32_t>(i));
        if (log && log_len) {
            const int at = ldg(log_len);
            if (at >= 0 && at < log_cap) {
                stg(log + at, static_cast<int32_t>(i));
                stg(log_len, at + 1);
            }
        }
    }
}

// dense: gate = gu[0, n), up = gu[up_offset, up_offset + n) of one buffer or two
__global__ void silu_mul_kernel(const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
                                uint16_t* __restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    stg(out + i, f32_to_f16_bits(silu_f32(f16_bits_to_f32(ldg(gate + i))) * f16_bits_to_f32(ldg(up + i))));
}

// DIP: out[j] = fp16(silu(gate[idx[j]]) * u_sel[j]); an index outside [0, n_gate) gives NaN
__global__ void silu_mul_indexed_kernel(const uint16_t* __restrict__ gate, const int32_t* __restrict__ idx,
                                        const uint16_t* __restrict__ u_sel, uint16_t* __restrict__ out, int k,
                                        int n_gate) {
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= k) return;
    const int c = ldg(idx + j);
    if (c < 0 || c >= n_gate) {
        stg(out + j, uint16_t(0x7e00u));
        return;
    }
    stg(out + j, f32_to_f16_bits(silu_f32(f16_bits_to_f32(ldg(gate + c))) * f16_bits_to_f32(ldg(u_sel + j))));
}

// out[:] = table[token[0], :] (zeros for a token outside [0, rows))
__global__ void embed_kernel(const uint16_t* __restrict__ table, int64_t rows, int hidden,
                             const int32_t* __restrict__ token, uint16_t* __restrict__ out) {
    const int t = ldg(token);
    const bool ok = t >= 0 && t < rows;
    const uint16_t* src = table + (ok ? static_cast<int64_t>(t) : 0) * hidden;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        stg(out + i, ok ? ldg(src + i) : uint16_t(0));
}

__global__ void advance_kernel(int32_t* __restrict__ pos, int32_t delta) {
    if (threadIdx.x == 0) stg(pos, ldg(pos) + delta);
}

static bool vec_ok(int64_t n, std::initializer_list<const void*> ps) {
    if (n % 8) return false;
    for (const void* p : ps)
        if (!aligned16(p)) return false;
    return true;
}

}  // namespace soi

using namespace soi;

extern "C" int soi_rmsnorm(const uint16_t* x, const uint16_t* weight, uint16_t* out, int64_t rows, int64_t hidden,
                           float eps, void* stream) {
    const char* what = "soi_rmsnorm";
    SOI_REQUIRE(rows >= 0 && rows <= (int64_t(1) << 31) - 1, "%s: rows out of range", what);
    SOI_REQUIRE(hidden >= 1 && hidden <= (int64_t(1) << 24), "%s: hidden must be in [1, 2^24]", what);
    if (rows == 0) return SOI_OK;
    SOI_REQUIRE(x && weight && out, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    uint16_t* xm = const_cast<uint16_t*>(x);  // not written without the residual add
    const int h = static_cast<int>(hidden);
    if (vec_ok(hidden, {x, weight, out}))
        hipLaunchKernelGGL((rmsnorm_kernel<false, true>), dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, st,
                           xm, nullptr, weight, out, h, eps, nullptr);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<false, false>), dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0,
                           st, xm, nullptr, weight, out, h, eps, nullptr);
    return launch_status(what);
}

static int residual_rmsnorm(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* out, int64_t rows,
                            int64_t hidden, float eps, int32_t* advance_pos, void* stream, const char* what) {
    SOI_REQUIRE(rows >= 0 && rows <= (int64_t(1) << 31) - 1, "%s: rows out of range", what);
    SOI_REQUIRE(hidden >= 1 && hidden <= (int64_t(1) << 24), "%s: hidden must be in [1, 2^24]", what);
    if (rows == 0) return SOI_OK;
    SOI_REQUIRE(x && delta && weight && out, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    const int h = static_cast<int>(hidden);
    if (vec_ok(hidden, {x, delta, weight, out}))
        hipLaunchKernelGGL((rmsnorm_kernel<true, true>), dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, st,
                           x, delta, weight, out, h, eps, advance_pos);
    else
        hipLaunchKernelGGL((rmsnorm_kernel<true, false>), dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, st,
                           x, delta, weight, out, h, eps, advance_pos);
    return launch_status(what);
}

extern "C" int soi_residual_rmsnorm(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* out,
                                    int64_t rows, int64_t hidden, float eps, void* stream) {
    return residual_rmsnorm(x, delta, weight, out, rows, hidden, eps, nullptr, stream, "soi_residual_rmsnorm");
}

extern "C" int soi_final_norm_advance(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* out,
                                      int64_t hidden, float eps, int32_t* pos, void* stream) {
    const char* what = "soi_final_norm_advance";
    SOI_REQUIRE(pos, "%s: null position pointer", what);
    return residual_rmsnorm(x, delta, weight, out, 1, hidden, eps, pos, stream, what);
}

extern "C" int soi_rope_apply(uint16_t* x, const float* cos_vals, const float* sin_vals, int64_t num_heads,
                              int64_t head_dim, void* stream) {
    const char* what = "soi_rope_apply";
    SOI_REQUIRE(num_heads >= 0 && num_heads <= (int64_t(1) << 31) - 1, "%s: num_heads out of range", what);
    SOI_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 2048, "%s: head_dim must be even, in [2, 2048]",
                what);
    if (num_heads == 0) return SOI_OK;
    SOI_REQUIRE(x && cos_vals && sin_vals, "%s: null pointer", what);
    hipLaunchKernelGGL(rope_kernel, dim3(static_cast<unsigned>(num_heads)), dim3(static_cast<unsigned>(head_dim / 2)),
                       0, as_stream(stream), x, cos_vals, sin_vals, static_cast<int>(head_dim));
    return launch_status(what);
}

extern "C" int soi_kv_cache_append(const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                                   int64_t num_kv_heads, int64_t max_seq, int64_t head_dim, int64_t pos,
                                   void* stream) {
    const char* what = "soi_kv_cache_append";
    SOI_REQUIRE(num_kv_heads >= 1 && num_kv_heads <= 65535, "%s: num_kv_heads out of range", what);
    SOI_REQUIRE(max_seq >= 1 && max_seq <= (int64_t(1) << 30) && head_dim >= 1 && head_dim <= 65536,
                "%s: size out of range", what);
    SOI_REQUIRE(pos >= 0 && pos < max_seq, "%s: pos out of range for max_seq_len", what);
    SOI_REQUIRE(k_new && v_new && k_cache && v_cache, "%s: null pointer", what);
    hipLaunchKernelGGL(kv_append_kernel, dim3(static_cast<unsigned>(num_kv_heads)), dim3(head_dim < 256 ? head_dim : 256),
                       0, as_stream(stream), k_new, v_new, k_cache, v_cache, static_cast<int>(max_seq),
                       static_cast<int>(head_dim), static_cast<int>(pos), nullptr);
    return launch_status(what);
}

extern "C" int soi_qk_norm_rope_append(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                                       const float* cos_table, const float* sin_table, const int32_t* pos,
                                       uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t max_seq, int64_t head_dim, float eps,
                                       void* stream) {
    const char* what = "soi_qk_norm_rope_append";
    SOI_REQUIRE(num_q_heads >= 1 && num_kv_heads >= 1 && num_q_heads + 2 * num_kv_heads <= 65535,
                "%s: head counts out of range", what);
    SOI_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 4096, "%s: head_dim must be even, in [2, 4096]",
                what);
    SOI_REQUIRE(max_seq >= 1 && max_seq <= (int64_t(1) << 30), "%s: max_seq_len out of range", what);
    SOI_REQUIRE(qkv && q_norm && k_norm && cos_table && sin_table && pos && q_out && k_cache && v_cache,
                "%s: null pointer", what);
    hipLaunchKernelGGL(qk_norm_rope_append_kernel, dim3(static_cast<unsigned>(num_q_heads + 2 * num_kv_heads)),
                       dim3(kNormThreads), 0, as_stream(stream), qkv, q_norm, k_norm, cos_table, sin_table, pos,
                       q_out, k_cache, v_cache, static_cast<int>(num_q_heads), static_cast<int>(num_kv_heads),
                       static_cast<int>(max_seq), static_cast<int>(head_dim), eps);
    return launch_status(what);
}

extern "C" int soi_gemv_f16(const uint16_t* W, const uint16_t* x, uint16_t* y, int64_t N, int64_t K, void* stream) {
    const char* what = "soi_gemv_f16";
    SOI_REQUIRE(N >= 0 && N <= (int64_t(1) << 31) - 1, "%s: N out of range", what);
    SOI_REQUIRE(K >= 1 && K <= (int64_t(1) << 30), "%s: K must be in [1, 2^30]", what);
    if (N == 0) return SOI_OK;
    SOI_REQUIRE(W && x && y, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    const int Ki = static_cast<int>(K);
    if (!vec_ok(K, {W, x})) {
        hipLaunchKernelGGL(gemv_f16_simple_kernel, dim3(static_cast<unsigned>(N)), dim3(64), 0, st, W, x, y, Ki);
        return launch_status(what);
    }
    // one row per wave (151936 single-wave workgroups for the LM head): 90.2-91.5 us for the 622.6 MB head against
    // 92.9-93.5 us with 2 rows and 94.1-95.6 us with 4 (4 passes each, back to back on cold copies, bit-identical)
    constexpr int R = 1;
    const int64_t chunks = K / 8;
    const int64_t passes = ceil_div64(chunks, kWave);
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, R)));
    if (passes >= 4 && N % R == 0 && chunks % (4 * kWave) == 0)
        hipLaunchKernelGGL((gemv_f16_kernel<R, 4, true>), grid, dim3(64), 0, st, W, x, y, N, Ki);
    else if (passes >= 2)
        hipLaunchKernelGGL((gemv_f16_kernel<R, 2, false>), grid, dim3(64), 0, st, W, x, y, N, Ki);
    else
        hipLaunchKernelGGL((gemv_f16_kernel<R, 1, false>), grid, dim3(64), 0, st, W, x, y, N, Ki);
    return launch_status(what);
}

extern "C" int soi_swiglu_gate_up(const uint16_t* gate_W, const uint16_t* up_W, const uint16_t* x, uint16_t* h,
                                  int64_t I, int64_t H, void* stream) {
    const char* what = "soi_swiglu_gate_up";
    SOI_REQUIRE(I >= 0 && I <= (int64_t(1) << 31) - 1, "%s: I out of range", what);
    SOI_REQUIRE(H >= 1 && H <= (int64_t(1) << 30), "%s: H must be in [1, 2^30]", what);
    if (I == 0) return SOI_OK;
    SOI_REQUIRE(gate_W && up_W && x && h, "%s: null pointer", what);
    hipStream_t st = as_stream(stream);
    const int Hi = static_cast<int>(H);
    if (!vec_ok(H, {gate_W, up_W, x})) {
        hipLaunchKernelGGL(swiglu_gate_up_simple_kernel, dim3(static_cast<unsigned>(I)), dim3(64), 0, st, gate_W,
                           up_W, x, h, Hi);
        return launch_status(what);
    }
    constexpr int R = 2;
    const int64_t chunks = H / 8;
    const int64_t passes = ceil_div64(chunks, kWave);
    const dim3 grid(static_cast<unsigned>(ceil_div64(I, R)));
    if (passes >= 4 && I % R == 0 && chunks % (4 * kWave) == 0)
        hipLaunchKernelGGL((swiglu_gate_up_kernel<R, 4, true>), grid, dim3(64), 0, st, gate_W, up_W, x, h, I, Hi);
    else if (passes >= 2)
        hipLaunchKernelGGL((swiglu_gate_up_kernel<R, 2, false>), grid, dim3(64), 0, st, gate_W, up_W, x, h, I, Hi);
    else
        hipLaunchKernelGGL((swiglu_gate_up_kernel<R, 1, false>), grid, dim3(64), 0, st, gate_W, up_W, x, h, I, Hi);
    return launch_status(what);
}

extern "C" size_t soi_argmax_workspace_bytes(int64_t n) {
    if (n <= 0) return 0;
    return static_cast<size_t>(ceil_div64(n, kArgmaxPerBlock)) * (sizeof(float) + sizeof(int));
}

extern "C" int soi_argmax_f16(const uint16_t* x, int64_t n, int32_t* out_index, int32_t* log, int32_t* log_len,
                              int64_t log_cap, void* workspace, size_t workspace_bytes, void* stream) {
    const char* what = "soi_argmax_f16";
    SOI_REQUIRE(n >= 1 && n <= (int64_t(1) << 31) - 1, "%s: n must be in [1, 2^31)", what);
    SOI_REQUIRE(x && out_index, "%s: null pointer", what);
    SOI_REQUIRE((log == nullptr) == (log_len == nullptr), "%s: log and log_len go together", what);
    SOI_REQUIRE(log_cap >= 0 && log_cap <= (int64_t(1) << 31) - 1, "%s: log_cap out of range", what);
    const int64_t nb = ceil_div64(n, kArgmaxPerBlock);
    const size_t need = soi_argmax_workspace_bytes(n);
    if (!workspace || workspace_bytes < need) {
        set_last_error("%s: workspace of %zu bytes required, got %zu", what, need, workspace_bytes);
        return SOI_ERR_WORKSPACE;
    }
    float* pv = static_cast<float*>(workspace);
    int* pi = reinterpret_cast<int*>(pv + nb);
    hipStream_t st = as_stream(stream);
    if (n % 8 == 0 && aligned16(x))
        hipLaunchKernelGGL(argmax_partial_kernel<true>, dim3(static_cast<unsigned>(nb)), dim3(kArgmaxThreads), 0, st, x,
                           static_cast<int>(n), pv, pi);
    else
        hipLaunchKernelGGL(argmax_partial_kernel<false>, dim3(static_cast<unsigned>(nb)), dim3(kArgmaxThreads), 0, st,
                           x, static_cast<int>(n), pv, pi);
    int s = launch_status(what);
    if (s) return s;
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(kArgmaxThreads), 0, st, pv, pi, static_cast<int>(nb),
                       out_index, log, log_len, static_cast<int>(log_cap));
    return launch_status(what);
}

extern "C" int soi_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, void* stream) {
    const char* what = "soi_silu_mul";
    SOI_REQUIRE(n >= 0 && n <= (int64_t(1) << 31) - 1, "%s: n out of range", what);
    if (n == 0) return SOI_OK;
    SOI_REQUIRE(gate && up && out, "%s: null pointer", what);
    hipLaunchKernelGGL(silu_mul_kernel, dim3(static_cast<unsigned>(ceil_div64(n, 256))), dim3(256), 0,
                       as_stream(stream), gate, up, out, static_cast<int>(n));
    return launch_status(what);
}

extern "C" int soi_silu_mul_indexed(const uint16_t* gate, int64_t n_gate, const int32_t* idx, const uint16_t* u_sel,
                                    uint16_t* out, int64_t k, void* stream) {
    const char* what = "soi_silu_mul_indexed";
    SOI_REQUIRE(k >= 0 && k <= (int64_t(1) << 31) - 1 && n_gate >= 0 && n_gate <= (int64_t(1) << 31) - 1,
                "%s: size out of range", what);
    if (k == 0) return SOI_OK;
    SOI_REQUIRE(gate && idx && u_sel && out, "%s: null pointer", what);
    hipLaunchKernelGGL(silu_mul_indexed_kernel, dim3(static_cast<unsigned>(ceil_div64(k, 256))), dim3(256), 0,
                       as_stream(stream), gate, idx, u_sel, out, static_cast<int>(k), static_cast<int>(n_gate));
    return launch_status(what);
}

extern "C" int soi_embed_lookup(const uint16_t* table, int64_t rows, int64_t hidden, const int32_t* token,
                                uint16_t* out, void* stream) {
    const char* what = "soi_embed_lookup";
    SOI_REQUIRE(rows >= 1 && hidden >= 1 && hidden <= (int64_t(1) << 30), "%s: size out of range", what);
    SOI_REQUIRE(table && token && out, "%s: null pointer", what);
    const int blocks = static_cast<int>(ceil_div64(hidden, 256) < 64 ? ceil_div64(hidden, 256) : 64);
    hipLaunchKernelGGL(embed_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), table, rows,
                       static_cast<int>(hidden), token, out);
    return launch_status(what);
}

extern "C" int soi_advance_position(int32_t* pos, int32_t delta, void* stream) {
    const char* what = "soi_advance_position";
    SOI_REQUIRE(pos, "%s: null pointer", what);
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, as_stream(stream), pos, delta);
    return launch_status(what);
}
