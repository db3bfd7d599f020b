/*
 * soi_oracle.c -- CPU restatement of sparse-offload-infer's quantized decode
 * hot path, used ONLY as a test checker and as the bench's CPU baseline.
 *
 * This file is test infrastructure. Nothing in the product (the HIP library,
 * the soinfer._C extension, the soinfer Python package) links, imports or
 * calls it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load it, and only as the checker / reported baseline.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root). Pinning of each function (which golden
 * vector, closed form or invariant checks it) is listed in the test file
 * tests/test_oracle_cpu.py; functions are grouped below as they are there.
 *
 * Numeric formats: fp16 values cross this interface as raw uint16 bit
 * patterns; conversion is written here from the IEEE-754 binary16 definition.
 */
#include <fenv.h>
#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* IEEE-754 binary16 <-> binary32                                             */
/* ------------------------------------------------------------------------- */

EXPORT float soi_ref_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    float out;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in binary32 */
        out = (float)m * (1.0f / 16777216.0f);
        return sign ? -out : out;
    }
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e - 15u + 127u) << 23) | (m << 13);
    }
    memcpy(&out, &bits, 4);
    return out;
}

/* round-to-nearest-even binary32 -> binary16 */
EXPORT uint16_t soi_ref_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                  /* below 2^-14: half subnormal range */
        float v;
        memcpy(&v, &ax, 4);
        float scaled = v * 16777216.0f; /* exact power-of-two scaling, in [0, 1024) */
        float fl = floorf(scaled);
        float frac = scaled - fl;
        uint32_t r = (uint32_t)fl;
        if (frac > 0.5f || (frac == 0.5f && (r & 1u))) r += 1u;
        return (uint16_t)(sign | r); /* r == 1024 encodes the smallest normal, as required */
    }
    uint32_t mant = ax & 0x7fffffu;
    uint32_t e = (ax >> 23) - 127u + 15u;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
    return (uint16_t)(sign | h);
}

EXPORT void soi_ref_f16_to_f32_array(const uint16_t* h, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = soi_ref_f16_to_f32(h[i]);
}

EXPORT void soi_ref_f32_to_f16_array(const float* f, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = soi_ref_f32_to_f16(f[i]);
}

static uint16_t f64_to_f16(double d) {
    /* Round a double to binary16 via binary32. Double rounding is avoided by
     * rounding to odd first: a binary32 with the sticky bit folded into its
     * last place keeps enough information for a correct RNE to binary16. */
    float f = (float)d;
    double back = (double)f;
    if (back != d && isfinite(f)) {
        uint32_t b;
        memcpy(&b, &f, 4);
        /* truncate toward zero then set the lsb (round-to-odd) */
        if (fabs(back) > fabs(d)) b -= 1u;
        b |= 1u;
        memcpy(&f, &b, 4);
    }
    return soi_ref_f32_to_f16(f);
}

EXPORT void soi_ref_f64_to_f16_array(const double* d, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = f64_to_f16(d[i]);
}

/* ------------------------------------------------------------------------- */
/* R2: symmetric group quantizer (min_max scale)                               */
/*   python/soinfer/quant/formats.py:55-65 (_amax_per_group), :77-110         */
/*   (quantize, group branch), python/soinfer/quant/calibrate.py:19,22-27     */
/*   (min_max: scale = max(amax/qmax, FLT_MIN)).                               */
/* Division is IEEE binary32 division (the reference quantizes on the CPU,    */
/* where torch divides exactly); rounding is round-half-to-even (torch.round). */
/* ------------------------------------------------------------------------- */

static float rne_f32(float v) {
    /* round half to even, independent of the current rounding mode */
    float fl = floorf(v);
    float diff = v - fl; /* exact for |v| < 2^23 */
    if (fabsf(v) >= 8388608.0f) return v;
    if (diff > 0.5f) return fl + 1.0f;
    if (diff < 0.5f) return fl;
    return (fmodf(fl, 2.0f) == 0.0f) ? fl : fl + 1.0f;
}

EXPORT void soi_ref_quantize_group(const float* w, int64_t N, int64_t K, int64_t gs, int bits, int8_t* q_out,
                                   float* scale_out) {
    const int qmax = (1 << (bits - 1)) - 1;
    const int64_t G = (K + gs - 1) / gs;
    const int64_t Kp = G * gs;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t g = 0; g < G; ++g) {
            float amax = 0.0f;
            for (int64_t i = 0; i < gs; ++i) {
                int64_t k = g * gs + i;
                float v = (k < K) ? w[n * K + k] : 0.0f;
                float a = fabsf(v);
                if (a > amax || isnan(a)) amax = a;
            }
            float s = amax / (float)qmax;
            if (s < FLT_MIN) s = FLT_MIN; /* clamp(min=tiny); NaN passes through */
            scale_out[n * G + g] = s;
            for (int64_t i = 0; i < gs; ++i) {
                int64_t k = g * gs + i;
                float v = (k < K) ? w[n * K + k] : 0.0f;
                float r = rne_f32(v / s);
                if (r > (float)qmax) r = (float)qmax;
                if (r < -(float)qmax) r = -(float)qmax;
                q_out[n * Kp + k] = (int8_t)r;
            }
        }
    }
}

/* per-tensor / per-channel branches (formats.py:88-99), used by the INT8 GEMV
 * parity cases. granularity 0 = per_tensor, 1 = per_channel. */
EXPORT void soi_ref_quantize_simple(const float* w, int64_t N, int64_t K, int bits, int granularity, int8_t* q_out,
                                    float* scale_out) {
    const int qmax = (1 << (bits - 1)) - 1;
    if (granularity == 0) {
        float amax = 0.0f;
        for (int64_t i = 0; i < N * K; ++i) {
            float a = fabsf(w[i]);
            if (a > amax) amax = a;
        }
        float s = amax / (float)qmax;
        if (s < FLT_MIN) s = FLT_MIN;
        scale_out[0] = s;
        for (int64_t i = 0; i < N * K; ++i) {
            float r = rne_f32(w[i] / s);
            if (r > qmax) r = (float)qmax;
            if (r < -qmax) r = -(float)qmax;
            q_out[i] = (int8_t)r;
        }
        return;
    }
    for (int64_t n = 0; n < N; ++n) {
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(w[n * K + k]);
            if (a > amax) amax = a;
        }
        float s = amax / (float)qmax;
        if (s < FLT_MIN) s = FLT_MIN;
        scale_out[n] = s;
        for (int64_t k = 0; k < K; ++k) {
            float r = rne_f32(w[n * K + k] / s);
            if (r > qmax) r = (float)qmax;
            if (r < -qmax) r = -(float)qmax;
            q_out[n * K + k] = (int8_t)r;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* R1: INT4 AWQ-order packing                                                  */
/*   csrc/include/layout.h:19-45,73-74; python/soinfer/quant/pack.py:31-69.   */
/*   byte0 = v0|v2<<4, byte1 = v4|v6<<4, byte2 = v1|v3<<4, byte3 = v5|v7<<4;  */
/*   K zero-padded to a multiple of 8.                                         */
/* ------------------------------------------------------------------------- */

EXPORT void soi_ref_pack_int4(const int8_t* q, int64_t N, int64_t K, uint8_t* out) {
    const int64_t words = (K + 7) / 8;
    static const int order[8] = {0, 2, 4, 6, 1, 3, 5, 7};
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t w = 0; w < words; ++w) {
            for (int b = 0; b < 4; ++b) {
                int lo_src = order[2 * b], hi_src = order[2 * b + 1];
                int64_t klo = w * 8 + lo_src, khi = w * 8 + hi_src;
                int lo = (klo < K) ? (q[n * K + klo] & 0xf) : 0;
                int hi = (khi < K) ? (q[n * K + khi] & 0xf) : 0;
                out[n * words * 4 + w * 4 + b] = (uint8_t)(lo | (hi << 4));
            }
        }
    }
}

/* signed value of logical element k of a packed row (sign-extended nibble) */
static inline int int4_at(const uint8_t* row, int64_t k) {
    static const int byte_of[8] = {0, 2, 0, 2, 1, 3, 1, 3};
    static const int shift_of[8] = {0, 0, 4, 4, 0, 0, 4, 4};
    int64_t w = k >> 3;
    int j = (int)(k & 7);
    int nib = (row[w * 4 + byte_of[j]] >> shift_of[j]) & 0xf;
    return nib >= 8 ? nib - 16 : nib;
}

EXPORT void soi_ref_unpack_int4(const uint8_t* packed, int64_t N, int64_t K, int8_t* q_out) {
    const int64_t row_bytes = ((K + 7) / 8) * 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) q_out[n * K + k] = (int8_t)int4_at(packed + n * row_bytes, k);
}

/* ------------------------------------------------------------------------- */
/* R3/R4: INT4 group dequant-GEMV                                              */
/*   csrc/kernels/gemv_w4a16_group.cu:23-70 (naive), :77-127 (lop3);          */
/*   y[n] = sum_k s[n, k/gs] * q[n,k] * x[k].                                   */
/* Two accumulations: binary64 (the precision oracle) and binary32 in plain   */
/* ascending-k order (the reference's fp32 arithmetic, one term at a time).   */
/* ------------------------------------------------------------------------- */

EXPORT void soi_ref_gemv_w4_f64(const uint8_t* Wq, const float* scale, const uint16_t* x, int64_t N, int64_t K,
                                int64_t gs, int64_t G, double* y) {
    const int64_t row_bytes = ((K + 7) / 8) * 4;
    float* xf = (float*)malloc(sizeof(float) * (size_t)K);
    for (int64_t k = 0; k < K; ++k) xf[k] = soi_ref_f16_to_f32(x[k]);
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* row = Wq + n * row_bytes;
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double s = (double)scale[n * G + k / gs];
            acc += s * (double)int4_at(row, k) * (double)xf[k];
        }
        y[n] = acc;
    }
    free(xf);
}

/* The same GEMV with its rows split over `threads` POSIX threads (contiguous row ranges). Every row is
 * still summed in ascending k by one thread, so the output equals soi_ref_gemv_w4_f64 exactly; this form
 * exists only to time the CPU baseline on several host cores. */
typedef struct {
    const uint8_t* Wq;
    const float* scale;
    const uint16_t* x;
    int64_t n0, n1, K, gs, G;
    double* y;
} soi_gemv_w4_job;

static void* soi_gemv_w4_worker(void* arg) {
    const soi_gemv_w4_job* j = (const soi_gemv_w4_job*)arg;
    const int64_t row_bytes = ((j->K + 7) / 8) * 4;
    soi_ref_gemv_w4_f64(j->Wq + j->n0 * row_bytes, j->scale + j->n0 * j->G, j->x, j->n1 - j->n0, j->K, j->gs, j->G,
                        j->y + j->n0);
    return NULL;
}

EXPORT void soi_ref_gemv_w4_f64_mt(const uint8_t* Wq, const float* scale, const uint16_t* x, int64_t N, int64_t K,
                                   int64_t gs, int64_t G, double* y, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    if ((int64_t)threads > N) threads = (int)(N > 0 ? N : 1);
    pthread_t tid[64];
    soi_gemv_w4_job job[64];
    for (int t = 0; t < threads; ++t) {
        job[t] = (soi_gemv_w4_job){Wq, scale, x, N * t / threads, N * (t + 1) / threads, K, gs, G, y};
    }
    int started = 0;
    for (int t = 1; t < threads; ++t, ++started)
        if (pthread_create(&tid[t], NULL, soi_gemv_w4_worker, &job[t]) != 0) break;
    soi_gemv_w4_worker(&job[0]);
    for (int t = 1; t <= started; ++t) pthread_join(tid[t], NULL);
    for (int t = started + 1; t < threads; ++t) soi_gemv_w4_worker(&job[t]); /* threads that failed to start */
}

EXPORT void soi_ref_gemv_w4_f32(const uint8_t* Wq, const float* scale, const uint16_t* x, int64_t N, int64_t K,
                                int64_t gs, int64_t G, float* y) {
    const int64_t row_bytes = ((K + 7) / 8) * 4;
    for (int64_t n = 0; n < N; ++n) {
        const uint8_t* row = Wq + n * row_bytes;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float s = scale[n * G + k / gs];
            acc = fmaf(s * (float)int4_at(row, k), soi_ref_f16_to_f32(x[k]), acc);
        }
        y[n] = acc;
    }
}

/* dequantized matrix in binary32: W[n,k] = fl(q * s) -- the value the
 * reference's basis-vector test compares against (formats.py:113-123). */
EXPORT void soi_ref_dequant_int4(const uint8_t* Wq, const float* scale, int64_t N, int64_t K, int64_t gs, int64_t G,
                                 float* W) {
    const int64_t row_bytes = ((K + 7) / 8) * 4;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k)
            W[n * K + k] = (float)int4_at(Wq + n * row_bytes, k) * scale[n * G + k / gs];
}

/* ------------------------------------------------------------------------- */
/* R5: INT8 dequant-GEMV (csrc/kernels/gemv_w8a16.cu:22-62)                    */
/*   scale row stride 0 = per-tensor broadcast; element k uses                */
/*   scale[row*stride + k/gs].                                                 */
/* ------------------------------------------------------------------------- */

EXPORT void soi_ref_gemv_w8_f64(const int8_t* Wq, const float* scale, const uint16_t* x, int64_t N, int64_t K,
                                int64_t gs, int64_t scale_row_stride, double* y) {
    for (int64_t n = 0; n < N; ++n) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) {
            double s = (double)scale[n * scale_row_stride + k / gs];
            acc += s * (double)Wq[n * K + k] * (double)soi_ref_f16_to_f32(x[k]);
        }
        y[n] = acc;
    }
}

/* ------------------------------------------------------------------------- */
/* R7: topk_threshold_select (csrc/kernels/topk_select.cu:10-96)              */
/*   Rule A (the reference): total_max = max(0, max v) (:19-23);             */
/*   lo = 0, hi = fl(total_max + 1e-3f) (:24-27); 24 times                     */
/*   { mid = fl(0.5f * fl(lo + hi)); if count(v >= mid) >= k lo = mid        */
/*     else hi = mid } (:37-61); then the first k indices in ascending order */
/*   with v >= lo (:85-95). Returns the number written.                       */
/* Rule B: exact top-k by value, ties broken by the lower index, output in    */
/*   ascending index order (the BASELINE config-3 wording).                   */
/* ------------------------------------------------------------------------- */

EXPORT float soi_ref_topk_tau_rule_a(const float* v, int64_t n, int64_t k) {
    float total_max = 0.0f;
    for (int64_t i = 0; i < n; ++i) total_max = fmaxf(total_max, v[i]);
    volatile float lo = 0.0f;
    volatile float hi = total_max + 1e-3f;
    for (int iter = 0; iter < 24; ++iter) {
        volatile float sum = lo + hi;
        volatile float mid = 0.5f * sum;
        int64_t count = 0;
        for (int64_t i = 0; i < n; ++i)
            if (v[i] >= mid) ++count;
        if (count >= k)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

EXPORT int64_t soi_ref_topk_rule_a(const float* v, int64_t n, int64_t k, int32_t* out_idx) {
    const float tau = soi_ref_topk_tau_rule_a(v, n, k);
    int64_t pos = 0;
    for (int64_t i = 0; i < n && pos < k; ++i)
        if (v[i] >= tau) out_idx[pos++] = (int32_t)i;
    return pos;
}

static const float* g_sort_vals;
static int cmp_desc_then_index(const void* a, const void* b) {
    int32_t ia = *(const int32_t*)a, ib = *(const int32_t*)b;
    float va = g_sort_vals[ia], vb = g_sort_vals[ib];
    if (va > vb) return -1;
    if (va < vb) return 1;
    return (ia < ib) ? -1 : (ia > ib);
}
static int cmp_int32(const void* a, const void* b) {
    int32_t ia = *(const int32_t*)a, ib = *(const int32_t*)b;
    return (ia < ib) ? -1 : (ia > ib);
}

EXPORT int64_t soi_ref_topk_rule_b(const float* v, int64_t n, int64_t k, int32_t* out_idx) {
    int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (size_t)n);
    for (int64_t i = 0; i < n; ++i) order[i] = (int32_t)i;
    g_sort_vals = v;
    qsort(order, (size_t)n, sizeof(int32_t), cmp_desc_then_index);
    qsort(order, (size_t)k, sizeof(int32_t), cmp_int32);
    memcpy(out_idx, order, sizeof(int32_t) * (size_t)k);
    free(order);
    return k;
}

/* ------------------------------------------------------------------------- */
/* R8: gather_rows (csrc/kernels/gather_rows.cu:6-21)                          */
/*   dst[j,:] = matrix[idx[j],:], byte copy.                                   */
/* ------------------------------------------------------------------------- */

EXPORT void soi_ref_gather_rows(const uint8_t* matrix, const int64_t* idx, int64_t k, int64_t row_nbytes,
                                uint8_t* dst) {
    for (int64_t j = 0; j < k; ++j) memcpy(dst + j * row_nbytes, matrix + idx[j] * row_nbytes, (size_t)row_nbytes);
}

/* ------------------------------------------------------------------------- */
/* R11/R14: sparse down accumulate (csrc/kernels/gemv_sparse_accumulate.cu:  */
/*   10-38; fused form gemv_dip_fused.cu:116-154)                              */
/*   y[c] = sum_{j<k} h_j * s[j, c/gs] * q[j, c]                               */
/* Row j of the weights/scales is taken from the descriptor when desc != NULL */
/* (top bit set: staging row desc&0x7fffffff, else cache slot), otherwise     */
/* row j of (cache_Wq, cache_scale).                                          */
/* ------------------------------------------------------------------------- */

static void row_ptrs(const int32_t* desc, int64_t j, const uint8_t* cWq, const float* cS, const uint8_t* sWq,
                     const float* sS, int64_t row_bytes, int64_t G, const uint8_t** wrow, const float** srow) {
    if (!desc) {
        *wrow = cWq + j * row_bytes;
        *srow = cS + j * G;
        return;
    }
    uint32_t d = (uint32_t)desc[j];
    int64_t off = (int64_t)(d & 0x7fffffffu);
    if (d >> 31) {
        *wrow = sWq + off * row_bytes;
        *srow = sS + off * G;
    } else {
        *wrow = cWq + off * row_bytes;
        *srow = cS + off * G;
    }
}

EXPORT void soi_ref_sparse_accumulate_f64(const uint8_t* cWq, const float* cS, const uint8_t* sWq, const float* sS,
                                          const int32_t* desc, const uint16_t* h, int64_t k, int64_t H, int64_t gs,
                                          int64_t G, double* y) {
    const int64_t row_bytes = ((H + 7) / 8) * 4;
    for (int64_t c = 0; c < H; ++c) y[c] = 0.0;
    for (int64_t j = 0; j < k; ++j) {
        const uint8_t* wrow;
        const float* srow;
        row_ptrs(desc, j, cWq, cS, sWq, sS, row_bytes, G, &wrow, &srow);
        double hj = (double)soi_ref_f16_to_f32(h[j]);
        for (int64_t c = 0; c < H; ++c) y[c] += hj * (double)srow[c / gs] * (double)int4_at(wrow, c);
    }
}

/* up direction with descriptors (gemv_dip_fused.cu:48-102): y[j] = row_j . x */
EXPORT void soi_ref_fused_up_f64(const uint8_t* cWq, const float* cS, const uint8_t* sWq, const float* sS,
                                 const int32_t* desc, const uint16_t* x, int64_t k, int64_t K, int64_t gs, int64_t G,
                                 double* y) {
    const int64_t row_bytes = ((K + 7) / 8) * 4;
    for (int64_t j = 0; j < k; ++j) {
        const uint8_t* wrow;
        const float* srow;
        row_ptrs(desc, j, cWq, cS, sWq, sS, row_bytes, G, &wrow, &srow);
        double acc = 0.0;
        for (int64_t kk = 0; kk < K; ++kk)
            acc += (double)srow[kk / gs] * (double)int4_at(wrow, kk) * (double)soi_ref_f16_to_f32(x[kk]);
        y[j] = acc;
    }
}

/* ------------------------------------------------------------------------- */
/* R12: build_dip_descriptors (csrc/kernels/gemv_dip_fused.cu:17-42)           */
/*   desc_j = slot_of[sel_j] if >= 0, else (miss position | 1<<31);           */
/*   misses numbered in ascending j (the reference numbers them in atomicAdd  */
/*   order, which is a race; ascending j is the deterministic instance).      */
/* ------------------------------------------------------------------------- */

EXPORT int32_t soi_ref_build_dip_descriptors(const int32_t* sel, int64_t k, const int32_t* slot_of, int32_t* desc,
                                             int32_t* miss_channels) {
    int32_t mc = 0;
    for (int64_t j = 0; j < k; ++j) {
        int32_t ch = sel[j];
        int32_t slot = slot_of[ch];
        if (slot >= 0) {
            desc[j] = slot;
        } else {
            miss_channels[mc] = ch;
            desc[j] = (int32_t)((uint32_t)mc | 0x80000000u);
            ++mc;
        }
    }
    return mc;
}

/* ------------------------------------------------------------------------- */
/* R16: decode attention (csrc/kernels/decode_attention.cu:17-55; binding     */
/*   scale = 1/sqrt(head_dim), bindings.cpp:482). GQA: kv head = qh / (NQ/NKV).*/
/*   Softmax evaluated in binary64 (exact max subtraction).                   */
/* ------------------------------------------------------------------------- */

EXPORT void soi_ref_decode_attention_f64(const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t NQ,
                                         int64_t NKV, int64_t S, int64_t hd, int64_t L, double* out) {
    const int64_t rep = NQ / NKV;
    const double scale = 1.0 / sqrt((double)hd);
    double* sc = (double*)malloc(sizeof(double) * (size_t)L);
    for (int64_t h = 0; h < NQ; ++h) {
        const int64_t kvh = h / rep;
        const uint16_t* K = kc + kvh * S * hd;
        const uint16_t* V = vc + kvh * S * hd;
        double m = -INFINITY;
        for (int64_t t = 0; t < L; ++t) {
            double d = 0.0;
            for (int64_t i = 0; i < hd; ++i)
                d += (double)soi_ref_f16_to_f32(q[h * hd + i]) * (double)soi_ref_f16_to_f32(K[t * hd + i]);
            sc[t] = d * scale;
            if (sc[t] > m) m = sc[t];
        }
        double l = 0.0;
        for (int64_t t = 0; t < L; ++t) {
            sc[t] = exp(sc[t] - m);
            l += sc[t];
        }
        for (int64_t i = 0; i < hd; ++i) {
            double a = 0.0;
            for (int64_t t = 0; t < L; ++t) a += sc[t] * (double)soi_ref_f16_to_f32(V[t * hd + i]);
            out[h * hd + i] = a / l;
        }
    }
    free(sc);
}
