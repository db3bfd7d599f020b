// Row sources for the INT4 kernels. A kernel body is written once against
// `rows.get(j)`; the dense, descriptor-driven (hot cache + staging) and
// index-driven (resident weights) variants only differ in where row j's
// packed bytes and scales live, so they share every arithmetic step and
// return bit-identical results on the same logical rows.
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
    __device__ __forceinline__ RowRef get(int64_t j) const { return {W + j * row_bytes, S + j * G, true}; }
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
    __device__ __forceinline__ RowRef get(int64_t j) const {
        const uint32_t d = static_cast<uint32_t>(desc[j]);
        const int64_t off = static_cast<int64_t>(d & 0x7fffffffu);
        if (d >> 31) {
            if (off < sN) return {sW + off * row_bytes, sS + off * G, true};
        } else {
            if (off < cN) return {cW + off * row_bytes, cS + off * G, true};
        }
        return {nullptr, nullptr, false};
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
    __device__ __forceinline__ RowRef get(int64_t j) const {
        const int32_t ch = idx[j];
        if (ch < 0 || ch >= fN) return {nullptr, nullptr, false};
        const int32_t s = slot_of[ch];
        if (s >= 0) {
            if (s < cN) return {cW + static_cast<int64_t>(s) * row_bytes, cS + static_cast<int64_t>(s) * G, true};
            return {nullptr, nullptr, false};
        }
        return {fW + static_cast<int64_t>(ch) * row_bytes, fS + static_cast<int64_t>(ch) * G, true};
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
    __device__ __forceinline__ RowRef get(int64_t j) const {
        const int32_t ch = idx[j];
        if (ch < 0 || ch >= fN) return {nullptr, nullptr, false};
        const int32_t s = slot_of[ch];
        if (s >= 0) {
            if (s < cN) return {cW + static_cast<int64_t>(s) * row_bytes, cS + static_cast<int64_t>(s) * G, true};
            return {nullptr, nullptr, false};
        }
        return {stW + j * row_bytes, fS + static_cast<int64_t>(ch) * G, true};
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
    __device__ __forceinline__ RowRef get(int64_t j) const {
        const int32_t r = idx[j];
        if (r >= 0 && r < nrows) return {W + static_cast<int64_t>(r) * row_bytes, S + static_cast<int64_t>(r) * G, true};
        return {nullptr, nullptr, false};
    }
};

}  // namespace soi
