// C-ABI plumbing (status text, per-thread error detail, version) and the
// host-side row gathers from pinned memory.
#include <cstring>

#include "soi_host.h"

namespace soi {

static thread_local char g_last_error[512] = "";

void set_last_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
}

static int check_gather(const uint8_t* matrix, int64_t num_rows, int64_t row_nbytes, const int64_t* indices,
                        int64_t k, const uint8_t* gpu_dst, const char* what) {
    SOI_REQUIRE(num_rows >= 0 && row_nbytes >= 0 && k >= 0, "%s: negative size", what);
    SOI_REQUIRE(k == 0 || row_nbytes == 0 || (matrix && indices && gpu_dst), "%s: null pointer", what);
    for (int64_t j = 0; j < k; ++j) {
        SOI_REQUIRE(indices[j] >= 0 && indices[j] < num_rows, "%s: indices[%lld] = %lld out of range [0, %lld)", what,
                    (long long)j, (long long)indices[j], (long long)num_rows);
    }
    return SOI_OK;
}

}  // namespace soi

using namespace soi;

extern "C" const char* soi_status_string(int status) {
    switch (status) {
        case SOI_OK: return "success";
        case SOI_ERR_INVALID_ARGUMENT: return "invalid argument";
        case SOI_ERR_WORKSPACE: return "workspace missing or too small";
        case SOI_ERR_HIP: return "HIP runtime error";
        case SOI_ERR_UNSUPPORTED: return "unsupported configuration";
        default: return "unknown status";
    }
}

extern "C" const char* soi_last_error(void) { return g_last_error; }

extern "C" const char* soi_version(void) { return "soinfer-amd 0.1.0 (gfx950)"; }

// Host memcpy of each selected row into contiguous pinned staging, then one
// H2D copy (csrc/kernels/gather_rows.cu:6-13).
extern "C" int soi_gather_rows_staged(const uint8_t* matrix, int64_t num_rows, int64_t row_nbytes,
                                      const int64_t* indices, int64_t k, uint8_t* staging, uint8_t* gpu_dst,
                                      void* stream) {
    const char* what = "soi_gather_rows_staged";
    int s = check_gather(matrix, num_rows, row_nbytes, indices, k, gpu_dst, what);
    if (s) return s;
    const size_t bytes = static_cast<size_t>(k) * static_cast<size_t>(row_nbytes);
    if (bytes == 0) return SOI_OK;
    SOI_REQUIRE(staging, "%s: null staging", what);
    for (int64_t j = 0; j < k; ++j)
        std::memcpy(staging + j * row_nbytes, matrix + indices[j] * row_nbytes, static_cast<size_t>(row_nbytes));
    SOI_HIP_TRY(hipMemcpyAsync(gpu_dst, staging, bytes, hipMemcpyHostToDevice, as_stream(stream)), what);
    return SOI_OK;
}

// One H2D copy per selected row (csrc/kernels/gather_rows.cu:15-21).
extern "C" int soi_gather_rows_naive(const uint8_t* matrix, int64_t num_rows, int64_t row_nbytes,
                                     const int64_t* indices, int64_t k, uint8_t* gpu_dst, void* stream) {
    const char* what = "soi_gather_rows_naive";
    int s = check_gather(matrix, num_rows, row_nbytes, indices, k, gpu_dst, what);
    if (s) return s;
    if (row_nbytes == 0) return SOI_OK;
    for (int64_t j = 0; j < k; ++j) {
        SOI_HIP_TRY(hipMemcpyAsync(gpu_dst + j * row_nbytes, matrix + indices[j] * row_nbytes,
                                   static_cast<size_t>(row_nbytes), hipMemcpyHostToDevice, as_stream(stream)),
                    what);
    }
    return SOI_OK;
}
