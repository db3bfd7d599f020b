// Row sources for the INT4 kernels. A kernel body is written once against
// `rows.get(j)`; the dense, descriptor-driven (hot cache + staging) and
// index-driven (resident weights) variants only differ in where row j's
// packed bytes and scales live, so they share every arithmetic step and
// return bit-identical results on the same logical rows.
// get() is branch-free (an unresolvable row gets a clamped in-range address
// and ok = false): a branch around a load makes the wave wait for it at the
// merge, which serialised the per-lane row lookups of the sparse down.
// get(j) == resolve(key(j), j): key() is the first load of a lookup (index or
// descriptor), resolve() the rest, so a kernel can issue every row's key
// before any row's dependent loads (loads complete in order).
#pragma once

#include <stdint.h>

namespace soi {

struct RowRef {
    const uint8_t* w;  // packed row (ceil(K/8)*4 bytes)
    const float* s;    // its scale row (num_groups floats)
    bool ok;           // false: unresolvable row (out-of-range offset); the kernel emits NaN, reads nothing
};

// row j of one [N, row_bytes] matrix
struct DenseRows {
    const uint8_t* W;
    const float* S;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return j; }
    __device__ __forceinline__ RowRef resolve(int64_t k, int64_t) const { return {W + k * row_bytes, S + k * G, true}; }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
};

// row j resolved by descriptor: top bit set -> staging row, else cache row
struct DescRows {
    const uint8_t* cW;
    const float* cS;
    int64_t cN;
    const uint8_t* sW;
    const float* sS;
    int64_t sN;
    const int32_t* desc;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return static_cast<uint32_t>(desc[j]); }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
    __device__ __forceinline__ RowRef resolve(int64_t kd, int64_t) const {
        const uint32_t d = static_cast<uint32_t>(kd);
        const int64_t off = static_cast<int64_t>(d & 0x7fffffffu);
        const bool st = (d >> 31) != 0;
        const bool ok = off < (st ? sN : cN);
        const int64_t o = ok ? off : 0;
        return {(st ? sW : cW) + o * row_bytes, (st ? sS : cS) + o * G, ok};
    }
};

// row j = channel idx[j] through a hot-channel cache: slot_of[ch] >= 0 -> cache
// row slot_of[ch], else row ch of the full matrix (usually a device mapping of
// pinned host memory, read in place) with its scales from the full scale
// matrix. Same logical rows as DescRows over a staging copy of the misses, so
// the GEMV results are identical; a channel outside [0, fN) or a slot outside
// [0, cN) is unresolvable.
struct SlotRows {
    const uint8_t* cW;
    const float* cS;
    int64_t cN;
    const uint8_t* fW;
    const float* fS;
    int64_t fN;
    const int32_t* idx;
    const int32_t* slot_of;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return idx[j]; }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
    __device__ __forceinline__ RowRef resolve(int64_t ch, int64_t) const {
        const bool cok = ch >= 0 && ch < fN;
        const int64_t c = cok ? ch : 0;
        const int32_t s = slot_of[c];
        const bool hit = s >= 0;
        const bool ok = cok && (!hit || s < cN);
        const int64_t r = hit ? (ok ? s : 0) : c;
        return {(hit ? cW : fW) + r * row_bytes, (hit ? cS : fS) + r * G, ok};
    }
};

// SlotRows with the misses already copied to staging row j (device memory):
// a miss reads row j of stW, its scales still come from row ch of fS.
struct SlotStageRows {
    const uint8_t* cW;
    const float* cS;
    int64_t cN;
    const uint8_t* stW;
    const float* fS;
    int64_t fN;
    const int32_t* idx;
    const int32_t* slot_of;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return idx[j]; }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
    __device__ __forceinline__ RowRef resolve(int64_t ch, int64_t j) const {
        const bool cok = ch >= 0 && ch < fN;
        const int64_t c = cok ? ch : 0;
        const int32_t s = slot_of[c];
        const bool hit = s >= 0;
        const bool ok = cok && (!hit || s < cN);
        const int64_t r = ok ? s : 0;
        return {hit ? cW + r * row_bytes : stW + j * row_bytes, hit ? cS + r * G : fS + c * G, ok};
    }
};

// row j = row idx[j] of a resident [num_rows, row_bytes] matrix
struct IndexRows {
    const uint8_t* W;
    const float* S;
    int64_t nrows;
    const int32_t* idx;
    int64_t row_bytes;
    int64_t G;
    __device__ __forceinline__ int64_t key(int64_t j) const { return idx[j]; }
    __device__ __forceinline__ RowRef get(int64_t j) const { return resolve(key(j), j); }
    __device__ __forceinline__ RowRef resolve(int64_t r, int64_t) const {
        const bool ok = r >= 0 && r < nrows;
        const int64_t rr = ok ? r : 0;
        return {W + rr * row_bytes, S + rr * G, ok};
    }
};

}  // namespace soi
