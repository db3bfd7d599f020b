// Device-side primitives shared by every soinfer HIP kernel (gfx950, wave64).
//
// Numeric conventions used throughout the library:
//   * weights are symmetric integers (INT4 in [-8,7], INT8 in [-128,127]) with
//     fp32 per-group scales; activations are IEEE binary16;
//   * dequantisation produces EXACT small integers in binary16 (no rounding),
//     products of two binary16 values are exact in binary32, and every sum is
//     accumulated in binary32 in a fixed order, so every kernel is
//     deterministic run to run;
//   * the order of a reduction is part of a kernel's contract: kernels that
//     must agree bit-for-bit (dense vs. descriptor-driven) share the same
//     accumulation templates below.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace soi {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// 16 zero bytes: the load target of lanes / rows that have nothing to read,
// so loads can be issued unconditionally (no branch, no serialising wait)
// and contribute exact zeros.
// (Never written; one private copy per code object. 16-byte aligned: it is
// the target of dwordx4 loads.)
__device__ __attribute__((aligned(16))) uint32_t g_zero16[4] = {0u, 0u, 0u, 0u};

// Loads through the global address space (global_load_*, not flat_load_*):
// pointers read from memory or chosen by a select lose the address-space
// information the compiler needs, so the kernels cast explicitly.
template <class T>
__device__ __forceinline__ T ldg(const T* p) {
    typedef const __attribute__((address_space(1))) T gT;
    return *(gT*)(p);
}
template <class T>
__device__ __forceinline__ void stg(T* p, T v) {
    typedef __attribute__((address_space(1))) T gT;
    *(gT*)(p) = v;
}
// Same, marked non-temporal (streamed once: weights).
template <class T>
__device__ __forceinline__ T ldg_stream(const T* p) {
    typedef const __attribute__((address_space(1))) T gT;
    return __builtin_nontemporal_load((gT*)(p));
}

// A pointer known to be the same in every lane, moved to scalar registers.
template <class T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v >> 32));
    return reinterpret_cast<T*>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ f16x2 as_f16x2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }

// ---------------------------------------------------------------------------
// INT4 (AWQ nibble order) -> binary16, two methods with identical results.
//
// Word layout: nibble i (bits 4i..4i+3) of a little-endian uint32 holds
// logical element AWQ[i] with AWQ = [0,2,4,6,1,3,5,7]; each nibble is a
// two's-complement signed 4-bit value. Both methods return the four pairs
// (v0,v1), (v2,v3), (v4,v5), (v6,v7) as packed binary16, i.e. consecutive
// k elements, matching a contiguous load of x.
// ---------------------------------------------------------------------------

// Method "bitfield": IEEE-754 binary16 exponent-bias construction. A value u
// in [0,15] placed in the low mantissa bits of 0x6400 (= 1024.0, where the
// binary16 spacing is exactly 1) encodes 1024+u; placed in mantissa bits 4..7
// it encodes 1024+16u. XOR 0x8 on each nibble maps a signed nibble n to
// u = n+8 (offset binary). Then
//   (1024+u)       - 1032       = n   (one packed add)
//   (1024+16u)/16  - 72         = n   (one packed fma; /16 is exact)
// All intermediate values are integers below 2048, hence exact in binary16.
// The mask/xor/or step is one three-input bitwise op (v_bitop3_b32) per pair.
// Since the mask bits and the 0x6400 bits are disjoint,
// ((w ^ 0x8..) & m) | 0x6400.. == (w & m) ^ (0x6400.. | 0x8 at the nibble),
// a single v_bitop3_b32 with truth table 0x6A = (a & b) ^ c.
__device__ __forceinline__ uint32_t and_xor(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x6A);
}

__device__ __forceinline__ void dequant_int4x8_bitfield(uint32_t w, f16x2 out[4]) {
    const uint32_t w8 = w >> 8;
    const uint32_t p0 = and_xor(w, 0x000f000fu, 0x64086408u);   // nibbles 0,4 -> v0, v1
    const uint32_t p1 = and_xor(w, 0x00f000f0u, 0x64806480u);   // nibbles 1,5 -> v2, v3 (x16)
    const uint32_t p2 = and_xor(w8, 0x000f000fu, 0x64086408u);  // nibbles 2,6 -> v4, v5
    const uint32_t p3 = and_xor(w8, 0x00f000f0u, 0x64806480u);  // nibbles 3,7 -> v6, v7 (x16)
    const f16x2 bias = {(f16)-1032.0f, (f16)-1032.0f};
    const f16x2 sixteenth = {(f16)0.0625f, (f16)0.0625f};
    const f16x2 bias16 = {(f16)-72.0f, (f16)-72.0f};
    out[0] = as_f16x2(p0) + bias;
    out[1] = __builtin_elementwise_fma(as_f16x2(p1), sixteenth, bias16);
    out[2] = as_f16x2(p2) + bias;
    out[3] = __builtin_elementwise_fma(as_f16x2(p3), sixteenth, bias16);
}

// Method used by the dot-product kernels: offset-binary nibbles as binary16
// SUBNORMALS. With u = n + 8 in [0,15], the half with bit pattern u encodes
// exactly u * 2^-24 and the pattern u<<4 encodes 16u * 2^-24, so no bias
// subtraction is needed per value: one v_bitop3 ((w & mask) ^ 0x8..) per pair.
//   lo[0] = (u0, u1) * 2^-24     hi[0] = (u2, u3) * 2^-20
//   lo[1] = (u4, u5) * 2^-24     hi[1] = (u6, u7) * 2^-20
// A dot product then recovers sum q*x = 2^24 * sum(lo.x) + 2^20 * sum(hi.x)
// - 8 * sum(x): the products u * 2^-24 * x are exact in binary32 (binary16
// denormals are preserved by the dot instructions), the power-of-two
// rescales are exact, and sum(x) is shared by every row of a tile.
__device__ __forceinline__ void int4x8_subnormal_bitfield(uint32_t w, f16x2 lo[2], f16x2 hi[2]) {
    const uint32_t w8 = w >> 8;
    lo[0] = as_f16x2(and_xor(w, 0x000f000fu, 0x00080008u));
    hi[0] = as_f16x2(and_xor(w, 0x00f000f0u, 0x00800080u));
    lo[1] = as_f16x2(and_xor(w8, 0x000f000fu, 0x00080008u));
    hi[1] = as_f16x2(and_xor(w8, 0x00f000f0u, 0x00800080u));
}

// Same bit patterns built nibble by nibble (bitfield extract, xor, shift, or):
// the independent second derivation, bit-identical to the above.
__device__ __forceinline__ void int4x8_subnormal_scalar(uint32_t w, f16x2 lo[2], f16x2 hi[2]) {
    // nibble index holding logical element j (AWQ order)
    constexpr int nib[8] = {0, 4, 1, 5, 2, 6, 3, 7};
    uint32_t u[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) u[j] = __builtin_amdgcn_ubfe(w, 4 * nib[j], 4) ^ 8u;
    lo[0] = as_f16x2(u[0] | (u[1] << 16));
    hi[0] = as_f16x2((u[2] << 4) | (u[3] << 20));
    lo[1] = as_f16x2(u[4] | (u[5] << 16));
    hi[1] = as_f16x2((u[6] << 4) | (u[7] << 20));
}

// INT8 -> binary16: four signed bytes b0..b3 of a word become (b0,b1),(b2,b3).
// XOR 0x80 maps b to u = b+128; 0x6400|u encodes 1024+u exactly; subtracting
// 1152 returns b exactly.
__device__ __forceinline__ void dequant_int8x4(uint32_t w, f16x2 out[2]) {
    const uint32_t t = w ^ 0x80808080u;
    const uint32_t p0 = (t & 0xffu) | ((t & 0xff00u) << 8) | 0x64006400u;
    const uint32_t p1 = ((t >> 16) & 0xffu) | ((t >> 8) & 0xff0000u) | 0x64006400u;
    const f16x2 bias = {(f16)-1152.0f, (f16)-1152.0f};
    out[0] = as_f16x2(p0) + bias;
    out[1] = as_f16x2(p1) + bias;
}

// a.x*b.x + a.y*b.y + c, products exact in binary32 (v_dot2c_f32_f16).
__device__ __forceinline__ float dot2(f16x2 a, f16x2 b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// ---------------------------------------------------------------------------
// Wave64 reductions with DPP. Fixed order: within quads, then 8 lanes, then
// 16-lane rows, then rows (1+0), (3+2), then (3+2)+(1+0). Result valid in
// lane 63; wave_sum_bcast returns it to every lane.
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf,
                                                                 false));
}

// The value of lane (l ^ MASK) in lane l, without the LDS crossbar where a VALU
// form exists: masks 16 / 32 by v_permlane16_swap / v_permlane32_swap (with
// both operands v, lane l's partner is in the first result when bit MASK of l
// is set, else in the second), 8 by DPP row_ror:8 ((i + 8) mod 16 = i ^ 8
// inside a 16-lane row), 2 and 1 by quad permutes, 4 by __shfl_xor.
template <int MASK>
__device__ __forceinline__ float xor_lanes(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const unsigned lane = threadIdx.x & 63;
    if constexpr (MASK == 32) {
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        return __builtin_bit_cast(float, (lane & 32) ? r[0] : r[1]);
    } else if constexpr (MASK == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
    } else if constexpr (MASK == 8) {
        return dpp_f<0x128>(v);
    } else if constexpr (MASK == 2) {
        return dpp_f<0x4e>(v);
    } else if constexpr (MASK == 1) {
        return dpp_f<0xb1>(v);
    } else {
        return __shfl_xor(v, MASK, 64);
    }
}

__device__ __forceinline__ float wave_sum_lane63(float v) {
    v += dpp_f<0xb1>(v);        // quad_perm [1,0,3,2]
    v += dpp_f<0x4e>(v);        // quad_perm [2,3,0,1]
    v += dpp_f<0x124>(v);       // row_ror:4
    v += dpp_f<0x128>(v);       // row_ror:8  -> every lane holds its 16-lane row sum
    v += dpp_f<0x142, 0xa>(v);  // row_bcast:15 into rows 1,3
    v += dpp_f<0x143, 0xc>(v);  // row_bcast:31 into rows 2,3
    return v;
}

__device__ __forceinline__ float wave_sum_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_sum_lane63(v)), 63));
}

__device__ __forceinline__ float wave_max_bcast(float v) {
    v = fmaxf(v, dpp_f<0xb1>(v));
    v = fmaxf(v, dpp_f<0x4e>(v));
    v = fmaxf(v, dpp_f<0x124>(v));
    v = fmaxf(v, dpp_f<0x128>(v));
    // cross-row: rows 1,3 take max with lane 15/47, then rows 2,3 with lane 31
    {
        float o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                        __builtin_bit_cast(int, v), 0x142, 0xa, 0xf,
                                                                        false));
        v = fmaxf(v, o);
        o = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                  __builtin_bit_cast(int, v), 0x143, 0xc, 0xf, false));
        v = fmaxf(v, o);
    }
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// ---------------------------------------------------------------------------
// Transposed reduction of R per-lane partials (R rows) across the wave, R in
// {1,2,4,8}: each exchange step halves the number of live values per lane
// (v_permlane32_swap / v_permlane16_swap / DPP row_ror:8 move the halves a
// lane gives away), then an 8-lane DPP sum finishes. Every lane ends with the
// full sum of row reduce_rows_row<R>(lane); the order of additions is fixed.
// kSwapUpperToVdst: v_permlane{32,16}_swap exchange the upper half of VDST
// with the lower half of VSRC0 (measured on gfx950).
// ---------------------------------------------------------------------------
constexpr bool kSwapUpperToVdst = true;

// The swaps are written as inline asm with both registers as read-write
// operands: through the two-result builtins the compiler was observed to read
// the second result from the first register.
__device__ __forceinline__ void swap32(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap16(float& a, float& b) {
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// sum over the 8 lanes of each aligned 8-lane group, result in every lane
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141>(v);  // row_half_mirror: lane i <- 7-i within each 8 lanes
    return v;
}

template <int R>
__device__ __forceinline__ float reduce_rows(float a[R]) {
    const uint32_t lane = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
    if (R == 8) {
        float b[4], c[2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float hi = a[j + 4], lo = a[j];
            swap32(hi, lo);
            b[j] = hi + lo;
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float hi = b[j + 2], lo = b[j];
            swap16(hi, lo);
            c[j] = hi + lo;
        }
        const bool e = lane & 8u;
        const float keep = e ? c[0] : c[1];
        const float send = e ? c[1] : c[0];
        return sum8(keep + dpp_f<0x128>(send));  // row_ror:8 = lane ^ 8 within 16
    } else if (R == 4) {
        float b[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float hi = a[j + 2], lo = a[j];
            swap32(hi, lo);
            b[j] = hi + lo;
        }
        float hi = b[1], lo = b[0];
        swap16(hi, lo);
        const float c = hi + lo;
        return sum8(c + dpp_f<0x128>(c));
    } else if (R == 2) {
        // Never swap a value with itself: the compiler folds swap(x, x) as if
        // both results were equal. Swapping against zero instead leaves the
        // row totals in the lower 16 lanes of each 32-lane half.
        float hi = a[1], lo = a[0];
        swap32(hi, lo);
        float b = hi + lo, z = 0.0f;
        swap16(b, z);
        const float c = b + z;
        return sum8(c + dpp_f<0x128>(c));
    } else {
        float v = a[0], z = 0.0f;
        swap32(v, z);
        float b = v + z, z2 = 0.0f;
        swap16(b, z2);
        const float c = b + z2;
        return sum8(c + dpp_f<0x128>(c));
    }
}

// which row's total reduce_rows<R> leaves in `lane`
template <int R>
__device__ __forceinline__ int reduce_rows_row(uint32_t lane) {
    const int g = static_cast<int>(lane >> 3);  // 8-lane group 0..7
    if (R == 8) return kSwapUpperToVdst ? 7 - g : g;
    if (R == 4) return kSwapUpperToVdst ? 3 - (g >> 1) : (g >> 1);
    if (R == 2) return kSwapUpperToVdst ? 1 - (g >> 2) : (g >> 2);
    return 0;
}

// Device-coherent (agent scope) 4-byte stores and loads (global_store / global_load with sc1): they reach,
// and read from, the point where the XCDs' accesses are coherent, so data one workgroup writes this way is
// visible to a workgroup on another XCD that reads it this way once the writer's stores have completed
// (s_waitcnt) and the reader has observed the writer's signal (a device-scope atomic). That needs no L2
// write-back (buffer_wbl2) before the signal and no L2 invalidate after it: measured on MI355X, those two
// fences cost about 3-4 us per arrival, more than the round trips they order.
__device__ __forceinline__ void st_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Workgroup arrival for data written with st_agent: every wave waits until its own stores have completed, and
// the barrier makes that true for the whole workgroup; thread 0 then signals with a device-scope atomic.
__device__ __forceinline__ void arrive_coherent() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

// number of set bits of a 64-bit wave mask strictly below this lane
__device__ __forceinline__ uint32_t mask_prefix(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

__device__ __forceinline__ uint64_t ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// binary32 -> binary16, round to nearest even, of a value that has been
// rounded to binary32 first (the reference computes in fp32 and then
// converts). The empty asm keeps the compiler from folding a producing
// multiply into a mixed-precision instruction (v_fma_mixlo_f16) that rounds
// once, straight to binary16: that choice is made per inlined site, so two
// kernels evaluating the same expression could otherwise disagree in the
// last binary16 bit.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    asm("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, static_cast<f16>(v));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) { return static_cast<float>(__builtin_bit_cast(f16, b)); }


// ---------------------------------------------------------------------------
// binary16 element helpers shared by the decode-step kernels
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return static_cast<uint32_t>(f32_to_f16_bits(a)) | (static_cast<uint32_t>(f32_to_f16_bits(b)) << 16);
}

// binary16 add of packed pairs: fp32 sum rounded once to binary16
__device__ __forceinline__ uint32_t add_f16x2(uint32_t a, uint32_t b) {
    const f16x2 x = as_f16x2(a), y = as_f16x2(b);
    return pack_f16x2(static_cast<float>(x.x) + static_cast<float>(y.x),
                      static_cast<float>(x.y) + static_cast<float>(y.y));
}

__device__ __forceinline__ float sumsq_f16x2(uint32_t a) {
    const f16x2 x = as_f16x2(a);
    const float u = static_cast<float>(x.x), v = static_cast<float>(x.y);
    return fmaf(v, v, u * u);
}

__device__ __forceinline__ uint32_t norm_f16x2(uint32_t a, uint32_t w, float inv) {
    const f16x2 x = as_f16x2(a), g = as_f16x2(w);
    return pack_f16x2(static_cast<float>(x.x) * inv * static_cast<float>(g.x),
                      static_cast<float>(x.y) * inv * static_cast<float>(g.y));
}

// RoPE rotation of one (x_i, x_{i+hd/2}) pair with fixed rounding: explicit
// fma so that every kernel applying it rounds identically (free contraction of
// a*c - b*s could fuse either product).
__device__ __forceinline__ void rope_pair(float a, float b, float c, float s, float& o1, float& o2) {
    o1 = fmaf(a, c, -(b * s));
    o2 = fmaf(b, c, a * s);
}

// silu(t) = t / (1 + exp(-t)) in fp32 (SwiGLU gating, generate.py:178)
__device__ __forceinline__ float silu_f32(float t) { return t / (1.0f + expf(-t)); }

}  // namespace soi
