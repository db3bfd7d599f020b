// soinfer._C -- thin PyTorch-ROCm binding over the C ABI in include/soinfer_amd.h.
//
// Function names, argument order, dtypes, output allocation and the
// validation rules (TORCH_CHECK -> Python RuntimeError) follow the
// reference's operator surface, csrc/bindings.cpp:26-610 (hot-path subset:
// gemv_w8a16 239-262, gemv_w4a16_group{,_lop3} 266-309,
// gemv_w4a16_sparse_accumulate 311-339, build_dip_descriptors 341-359,
// gemv_dip_fused_{up,down} 363-432, decode_attention 468-488,
// topk_threshold_select 507-518, gather_rows_{staged,naive} 522-559).
// Kernels are launched on the current HIP stream of the input's device; a
// C-ABI failure raises RuntimeError carrying the library's error text
// (the reference aborts the process instead, common.cuh:18-26).
#include <torch/extension.h>

#include <ATen/hip/HIPContext.h>
#include <c10/hip/HIPStream.h>

#include <cmath>
#include <tuple>
#include <vector>

#include "../../include/soinfer_amd.h"

namespace {

void* cur_stream(const torch::Tensor& t) {
    return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

void check_status(int status, const char* name) {
    TORCH_CHECK(status == SOI_OK, name, ": ", soi_status_string(status), ": ", soi_last_error());
}

void check_f32_cuda_contiguous(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, ": input must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == torch::kFloat32, name, ": only float32 is supported");
    TORCH_CHECK(t.is_contiguous(), name, ": input must be contiguous");
}

void check_f16_cuda_contiguous(const torch::Tensor& t, const char* name) {
    TORCH_CHECK(t.is_cuda(), name, ": input must be a CUDA tensor");
    TORCH_CHECK(t.scalar_type() == torch::kFloat16, name, ": only float16 is supported");
    TORCH_CHECK(t.is_contiguous(), name, ": input must be contiguous");
}

void check_same_device(const torch::Tensor& a, const torch::Tensor& b, const char* name) {
    TORCH_CHECK(a.device() == b.device(), name, ": all CUDA tensors must be on the same device");
}

const uint16_t* h16(const torch::Tensor& t) { return reinterpret_cast<const uint16_t*>(t.data_ptr<at::Half>()); }
uint16_t* h16m(torch::Tensor& t) { return reinterpret_cast<uint16_t*>(t.data_ptr<at::Half>()); }

int64_t expected_num_groups(int64_t k_dim, int64_t group_size) { return (k_dim + group_size - 1) / group_size; }

// workspaces end (attention) or start (sparse down) with arrival counters that must start at zero
torch::Tensor zeroed_workspace(const torch::Tensor& like, size_t bytes) {
    return torch::zeros({static_cast<int64_t>(bytes > 0 ? bytes : 1)}, like.options().dtype(torch::kUInt8));
}

}  // namespace

// ---------------------------------------------------------------------------
// INT8 / INT4 dense GEMV
// ---------------------------------------------------------------------------

torch::Tensor gemv_w8a16(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x, int64_t group_size) {
    TORCH_CHECK(Wq.is_cuda(), "gemv_w8a16(Wq): must be a CUDA tensor");
    TORCH_CHECK(Wq.scalar_type() == torch::kInt8, "gemv_w8a16(Wq): must be int8");
    TORCH_CHECK(Wq.is_contiguous(), "gemv_w8a16(Wq): must be contiguous");
    TORCH_CHECK(Wq.dim() == 2, "gemv_w8a16(Wq): must be 2D [N, K]");
    check_f16_cuda_contiguous(x, "gemv_w8a16(x)");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == Wq.size(1), "gemv_w8a16: x must be 1D [K] matching Wq's K");
    TORCH_CHECK(group_size >= 1, "gemv_w8a16: group_size must be >= 1");
    check_f32_cuda_contiguous(scale, "gemv_w8a16(scale)");
    const int64_t N = Wq.size(0), K = Wq.size(1);
    TORCH_CHECK(scale.dim() == 2, "gemv_w8a16: scale must be 2D [N or 1, num_groups]");
    TORCH_CHECK(scale.size(0) == N || scale.size(0) == 1,
                "gemv_w8a16: scale.size(0) must be N (per-channel/group) or 1 (per-tensor broadcast)");
    const int64_t num_groups = scale.size(1);
    const int64_t stride = (scale.size(0) == 1) ? 0 : num_groups;
    TORCH_CHECK(num_groups == 1 || group_size % 4 == 0,
                "gemv_w8a16: group_size must be a multiple of 4 when num_groups > 1");
    TORCH_CHECK(num_groups == 1 || num_groups == expected_num_groups(K, group_size),
                "gemv_w8a16: scale's num_groups must be 1 (per-tensor broadcast) or ceil(K/group_size) for the given "
                "K and group_size, got ", num_groups, " but expected ", expected_num_groups(K, group_size));
    check_same_device(Wq, x, "gemv_w8a16");
    check_same_device(Wq, scale, "gemv_w8a16");
    const at::DeviceGuard guard(x.device());
    auto y = torch::empty({N}, x.options());
    check_status(soi_gemv_w8a16(Wq.data_ptr<int8_t>(), scale.data_ptr<float>(), h16(x), h16m(y), N, K, group_size,
                                num_groups, stride, cur_stream(x)),
                 "gemv_w8a16");
    return y;
}

namespace {

using Int4Fn = int (*)(const uint8_t*, const float*, const uint16_t*, uint16_t*, int64_t, int64_t, int64_t, int64_t,
                       void*);

torch::Tensor gemv_w4a16_group_impl(torch::Tensor Wq_packed, torch::Tensor scale, torch::Tensor x, int64_t K,
                                    int64_t group_size, const char* name, Int4Fn fn) {
    TORCH_CHECK(Wq_packed.is_cuda(), name, "(Wq_packed): must be a CUDA tensor");
    TORCH_CHECK(Wq_packed.scalar_type() == torch::kUInt8, name, "(Wq_packed): must be uint8 (AWQ-packed int4)");
    TORCH_CHECK(Wq_packed.is_contiguous(), name, "(Wq_packed): must be contiguous");
    TORCH_CHECK(Wq_packed.dim() == 2, name, "(Wq_packed): must be 2D [N, ceil(K/8)*4]");
    check_f16_cuda_contiguous(x, "x");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == K, name, ": x must be 1D [K]");
    TORCH_CHECK(K >= 1, name, ": K must be >= 1");
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    const int64_t N = Wq_packed.size(0);
    TORCH_CHECK(Wq_packed.size(1) == ((K + 7) / 8) * 4, name, ": Wq_packed.size(1) must be ceil(K/8)*4 for the given K");
    TORCH_CHECK(scale.is_cuda(), name, ": scale must be a CUDA tensor");
    TORCH_CHECK(scale.scalar_type() == torch::kFloat32, name, ": scale must be float32");
    TORCH_CHECK(scale.is_contiguous(), name, ": scale must be contiguous");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == N, name,
                ": scale must be 2D [N, num_groups] (grouped int4 has no per-tensor broadcast)");
    const int64_t num_groups = scale.size(1);
    TORCH_CHECK(num_groups == expected_num_groups(K, group_size), name, ": scale's num_groups must be "
                "ceil(K/group_size) for the given K and group_size, got ", num_groups, " but expected ",
                expected_num_groups(K, group_size));
    check_same_device(Wq_packed, x, name);
    check_same_device(Wq_packed, scale, name);
    const at::DeviceGuard guard(x.device());
    auto y = torch::empty({N}, x.options());
    check_status(fn(Wq_packed.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), h16m(y), N, K, group_size,
                    num_groups, cur_stream(x)),
                 name);
    return y;
}

}  // namespace

torch::Tensor gemv_w4a16_group(torch::Tensor Wq_packed, torch::Tensor scale, torch::Tensor x, int64_t K,
                               int64_t group_size) {
    return gemv_w4a16_group_impl(Wq_packed, scale, x, K, group_size, "gemv_w4a16_group", soi_gemv_w4a16_group);
}

torch::Tensor gemv_w4a16_group_lop3(torch::Tensor Wq_packed, torch::Tensor scale, torch::Tensor x, int64_t K,
                                    int64_t group_size) {
    return gemv_w4a16_group_impl(Wq_packed, scale, x, K, group_size, "gemv_w4a16_group_lop3",
                                 soi_gemv_w4a16_group_lop3);
}

// P same-shape INT4 GEMVs in one launch; pointer tables are int64 device tensors
// of data pointers built (and validated) by soinfer.ops.GemvBatch.
void gemv_w4a16_batched(torch::Tensor Wq_ptrs, torch::Tensor scale_ptrs, torch::Tensor x_ptrs, torch::Tensor y_ptrs,
                        int64_t N, int64_t K, int64_t group_size) {
    const char* name = "gemv_w4a16_batched";
    for (const auto* t : {&Wq_ptrs, &scale_ptrs, &x_ptrs, &y_ptrs}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kInt64 && t->dim() == 1 && t->is_contiguous(), name,
                    ": pointer tables must be contiguous 1D int64 CUDA tensors");
        TORCH_CHECK(t->size(0) == Wq_ptrs.size(0), name, ": pointer tables must have the same length");
        check_same_device(Wq_ptrs, *t, name);
    }
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    const at::DeviceGuard guard(Wq_ptrs.device());
    check_status(soi_gemv_w4a16_batched(reinterpret_cast<const uint8_t* const*>(Wq_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const float* const*>(scale_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const uint16_t* const*>(x_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<uint16_t* const*>(y_ptrs.data_ptr<int64_t>()),
                                        Wq_ptrs.size(0), N, K, group_size, expected_num_groups(K, group_size),
                                        cur_stream(Wq_ptrs)),
                 name);
}

// P same-shape INT8 GEMVs in one launch; pointer tables built (and validated) by soinfer.ops.Int8Batch.
void gemv_w8a16_batched(torch::Tensor Wq_ptrs, torch::Tensor scale_ptrs, torch::Tensor x_ptrs, torch::Tensor y_ptrs,
                        int64_t N, int64_t K, int64_t group_size, int64_t num_groups, int64_t scale_row_stride) {
    const char* name = "gemv_w8a16_batched";
    for (const auto* t : {&Wq_ptrs, &scale_ptrs, &x_ptrs, &y_ptrs}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kInt64 && t->dim() == 1 && t->is_contiguous(), name,
                    ": pointer tables must be contiguous 1D int64 CUDA tensors");
        TORCH_CHECK(t->size(0) == Wq_ptrs.size(0), name, ": pointer tables must have the same length");
        check_same_device(Wq_ptrs, *t, name);
    }
    const at::DeviceGuard guard(Wq_ptrs.device());
    check_status(soi_gemv_w8a16_batched(reinterpret_cast<const int8_t* const*>(Wq_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const float* const*>(scale_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const uint16_t* const*>(x_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<uint16_t* const*>(y_ptrs.data_ptr<int64_t>()),
                                        Wq_ptrs.size(0), N, K, group_size, num_groups, scale_row_stride,
                                        cur_stream(Wq_ptrs)),
                 name);
}

void gemv_w4a16_grouped(torch::Tensor Wq_ptrs, torch::Tensor scale_ptrs, torch::Tensor x_ptrs, torch::Tensor y_ptrs,
                        std::vector<int64_t> class_count, std::vector<int64_t> class_N, std::vector<int64_t> class_K,
                        int64_t group_size) {
    const char* name = "gemv_w4a16_grouped";
    for (const auto* t : {&Wq_ptrs, &scale_ptrs, &x_ptrs, &y_ptrs}) {
        TORCH_CHECK(t->is_cuda() && t->scalar_type() == torch::kInt64 && t->dim() == 1 && t->is_contiguous(), name,
                    ": pointer tables must be contiguous 1D int64 CUDA tensors");
        TORCH_CHECK(t->size(0) == Wq_ptrs.size(0), name, ": pointer tables must have the same length");
        check_same_device(Wq_ptrs, *t, name);
    }
    TORCH_CHECK(class_count.size() == class_N.size() && class_count.size() == class_K.size(), name,
                ": class arrays must have the same length");
    int64_t total = 0;
    for (int64_t c : class_count) total += c;
    TORCH_CHECK(total == Wq_ptrs.size(0), name, ": class counts must add up to the pointer table length");
    const at::DeviceGuard guard(Wq_ptrs.device());
    check_status(soi_gemv_w4a16_grouped(reinterpret_cast<const uint8_t* const*>(Wq_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const float* const*>(scale_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<const uint16_t* const*>(x_ptrs.data_ptr<int64_t>()),
                                        reinterpret_cast<uint16_t* const*>(y_ptrs.data_ptr<int64_t>()),
                                        static_cast<int64_t>(class_count.size()), class_count.data(), class_N.data(),
                                        class_K.data(), group_size, cur_stream(Wq_ptrs)),
                 name);
}

// ---------------------------------------------------------------------------
// sparse down accumulate
// ---------------------------------------------------------------------------

torch::Tensor gemv_w4a16_sparse_accumulate(torch::Tensor Wq_selected, torch::Tensor scale_selected,
                                           torch::Tensor h_selected, int64_t H, int64_t group_size) {
    const char* name = "gemv_w4a16_sparse_accumulate";
    TORCH_CHECK(Wq_selected.is_cuda() && Wq_selected.scalar_type() == torch::kUInt8 && Wq_selected.is_contiguous(),
                name, "(Wq_selected): must be a contiguous CUDA uint8 tensor");
    TORCH_CHECK(Wq_selected.dim() == 2, name, "(Wq_selected): must be 2D [k, ceil(H/8)*4]");
    TORCH_CHECK(H >= 1, name, ": H must be >= 1");
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    const int64_t k = Wq_selected.size(0);
    TORCH_CHECK(Wq_selected.size(1) == ((H + 7) / 8) * 4, name,
                ": Wq_selected.size(1) must be ceil(H/8)*4 for the given H");
    TORCH_CHECK(scale_selected.is_cuda() && scale_selected.scalar_type() == torch::kFloat32 &&
                    scale_selected.is_contiguous(),
                name, "(scale_selected): must be a contiguous CUDA float32 tensor");
    TORCH_CHECK(scale_selected.dim() == 2 && scale_selected.size(0) == k, name,
                ": scale_selected must be 2D [k, num_groups]");
    check_f16_cuda_contiguous(h_selected, "gemv_w4a16_sparse_accumulate(h_selected)");
    TORCH_CHECK(h_selected.dim() == 1 && h_selected.size(0) == k, name, ": h_selected must be 1D [k]");
    const int64_t num_groups = scale_selected.size(1);
    TORCH_CHECK(num_groups == expected_num_groups(H, group_size), name, ": scale_selected's num_groups must be "
                "ceil(H/group_size) for the given H and group_size, got ", num_groups, " but expected ",
                expected_num_groups(H, group_size));
    check_same_device(Wq_selected, h_selected, name);
    check_same_device(Wq_selected, scale_selected, name);
    const at::DeviceGuard guard(h_selected.device());
    auto y = torch::empty({H}, h_selected.options());
    const size_t wsb = soi_sparse_accumulate_workspace_bytes(H, k);
    auto ws = zeroed_workspace(h_selected, wsb);
    check_status(soi_gemv_w4a16_sparse_accumulate(Wq_selected.data_ptr<uint8_t>(), scale_selected.data_ptr<float>(),
                                                  h16(h_selected), h16m(y), H, k, group_size, num_groups,
                                                  ws.data_ptr<uint8_t>(), wsb, cur_stream(h_selected)),
                 name);
    return y;
}

// ---------------------------------------------------------------------------
// hot-cache descriptors and fused GEMVs
// ---------------------------------------------------------------------------

std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> build_dip_descriptors(torch::Tensor selected_indices,
                                                                              torch::Tensor slot_of) {
    const char* name = "build_dip_descriptors";
    TORCH_CHECK(selected_indices.is_cuda() && selected_indices.scalar_type() == torch::kInt32 &&
                    selected_indices.dim() == 1 && selected_indices.is_contiguous(),
                name, "(selected_indices): must be a contiguous 1D int32 CUDA tensor");
    TORCH_CHECK(slot_of.is_cuda() && slot_of.scalar_type() == torch::kInt32 && slot_of.dim() == 1 &&
                    slot_of.is_contiguous(),
                name, "(slot_of): must be a contiguous 1D int32 CUDA tensor");
    check_same_device(selected_indices, slot_of, name);
    const at::DeviceGuard guard(selected_indices.device());
    const int64_t k = selected_indices.size(0);
    auto descriptors = torch::empty({k}, selected_indices.options());
    auto miss_channels = torch::empty({k}, selected_indices.options());
    auto miss_count = torch::empty({1}, selected_indices.options());
    check_status(soi_build_dip_descriptors(selected_indices.data_ptr<int32_t>(), k, slot_of.data_ptr<int32_t>(),
                                           slot_of.size(0), descriptors.data_ptr<int32_t>(),
                                           miss_channels.data_ptr<int32_t>(), miss_count.data_ptr<int32_t>(),
                                           cur_stream(selected_indices)),
                 name);
    return {descriptors, miss_channels, miss_count};
}

namespace {

void check_dip_fused_common(const torch::Tensor& cache_Wq, const torch::Tensor& cache_scale,
                            const torch::Tensor& staging_Wq, const torch::Tensor& staging_scale,
                            const torch::Tensor& descriptors, int64_t row_dim, const char* name) {
    const int64_t expected_bytes = ((row_dim + 7) / 8) * 4;
    TORCH_CHECK(cache_Wq.is_cuda() && cache_Wq.scalar_type() == torch::kUInt8 && cache_Wq.dim() == 2 &&
                    cache_Wq.is_contiguous() && cache_Wq.size(1) == expected_bytes,
                name, "(cache_Wq): must be a contiguous 2D uint8 CUDA tensor [C, ceil(row_dim/8)*4]");
    TORCH_CHECK(staging_Wq.is_cuda() && staging_Wq.scalar_type() == torch::kUInt8 && staging_Wq.dim() == 2 &&
                    staging_Wq.is_contiguous() && staging_Wq.size(1) == expected_bytes,
                name, "(staging_Wq): must be a contiguous 2D uint8 CUDA tensor [M, ceil(row_dim/8)*4]");
    TORCH_CHECK(cache_scale.is_cuda() && cache_scale.scalar_type() == torch::kFloat32 && cache_scale.dim() == 2 &&
                    cache_scale.is_contiguous(),
                name, "(cache_scale): must be a contiguous 2D float32 CUDA tensor [C, num_groups]");
    TORCH_CHECK(staging_scale.is_cuda() && staging_scale.scalar_type() == torch::kFloat32 &&
                    staging_scale.dim() == 2 && staging_scale.is_contiguous(),
                name, "(staging_scale): must be a contiguous 2D float32 CUDA tensor [M, num_groups]");
    TORCH_CHECK(cache_scale.size(1) == staging_scale.size(1), name,
                ": cache_scale and staging_scale must have the same num_groups");
    TORCH_CHECK(descriptors.is_cuda() && descriptors.scalar_type() == torch::kInt32 && descriptors.dim() == 1 &&
                    descriptors.is_contiguous(),
                name, "(descriptors): must be a contiguous 1D int32 CUDA tensor");
    // Row counts of each source bound the descriptor offsets inside the kernel.
    TORCH_CHECK(cache_scale.size(0) >= cache_Wq.size(0) || cache_Wq.size(0) == 0, name,
                ": cache_scale must have a row per cache_Wq row");
    TORCH_CHECK(staging_scale.size(0) >= staging_Wq.size(0) || staging_Wq.size(0) == 0, name,
                ": staging_scale must have a row per staging_Wq row");
    check_same_device(descriptors, cache_Wq, name);
    check_same_device(descriptors, staging_Wq, name);
    check_same_device(descriptors, cache_scale, name);
    check_same_device(descriptors, staging_scale, name);
}

}  // namespace

torch::Tensor gemv_dip_fused_up(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor staging_Wq,
                                torch::Tensor staging_scale, torch::Tensor descriptors, torch::Tensor x, int64_t K,
                                int64_t group_size) {
    const char* name = "gemv_dip_fused_up";
    check_dip_fused_common(cache_Wq, cache_scale, staging_Wq, staging_scale, descriptors, K, name);
    check_f16_cuda_contiguous(x, "gemv_dip_fused_up(x)");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == K, name, ": x must be 1D [K]");
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    const int64_t k = descriptors.size(0);
    const int64_t num_groups = cache_scale.size(1);
    TORCH_CHECK(num_groups == expected_num_groups(K, group_size), name, ": cache_scale/staging_scale's num_groups "
                "must be ceil(K/group_size) for the given K and group_size, got ", num_groups, " but expected ",
                expected_num_groups(K, group_size));
    check_same_device(descriptors, x, name);
    const at::DeviceGuard guard(x.device());
    auto y = torch::empty({k}, x.options());
    const int64_t C = std::min(cache_Wq.size(0), cache_scale.size(0));
    const int64_t M = std::min(staging_Wq.size(0), staging_scale.size(0));
    check_status(soi_gemv_dip_fused_up(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(), C,
                                       staging_Wq.data_ptr<uint8_t>(), staging_scale.data_ptr<float>(), M,
                                       descriptors.data_ptr<int32_t>(), k, h16(x), h16m(y), K, group_size, num_groups,
                                       cur_stream(x)),
                 name);
    return y;
}

torch::Tensor gemv_dip_fused_down(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor staging_Wq,
                                  torch::Tensor staging_scale, torch::Tensor descriptors, torch::Tensor h_selected,
                                  int64_t H, int64_t group_size) {
    const char* name = "gemv_dip_fused_down";
    check_dip_fused_common(cache_Wq, cache_scale, staging_Wq, staging_scale, descriptors, H, name);
    check_f16_cuda_contiguous(h_selected, "gemv_dip_fused_down(h_selected)");
    const int64_t k = descriptors.size(0);
    TORCH_CHECK(h_selected.dim() == 1 && h_selected.size(0) == k, name, ": h_selected must be 1D [k]");
    TORCH_CHECK(H >= 1, name, ": H must be >= 1");
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    const int64_t num_groups = cache_scale.size(1);
    TORCH_CHECK(num_groups == expected_num_groups(H, group_size), name, ": cache_scale/staging_scale's num_groups "
                "must be ceil(H/group_size) for the given H and group_size, got ", num_groups, " but expected ",
                expected_num_groups(H, group_size));
    check_same_device(descriptors, h_selected, name);
    const at::DeviceGuard guard(h_selected.device());
    auto y = torch::empty({H}, h_selected.options());
    const size_t wsb = soi_sparse_accumulate_workspace_bytes(H, k);
    auto ws = zeroed_workspace(h_selected, wsb);
    const int64_t C = std::min(cache_Wq.size(0), cache_scale.size(0));
    const int64_t M = std::min(staging_Wq.size(0), staging_scale.size(0));
    check_status(soi_gemv_dip_fused_down(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(), C,
                                         staging_Wq.data_ptr<uint8_t>(), staging_scale.data_ptr<float>(), M,
                                         descriptors.data_ptr<int32_t>(), k, h16(h_selected), h16m(y), H, group_size,
                                         num_groups, ws.data_ptr<uint8_t>(), wsb, cur_stream(h_selected)),
                 name);
    return y;
}

// ---------------------------------------------------------------------------
// resident-weight (index-driven) sparse GEMVs and device gather
// ---------------------------------------------------------------------------

torch::Tensor gemv_w4a16_indexed(torch::Tensor Wq_packed, torch::Tensor scale, torch::Tensor idx, torch::Tensor x,
                                 int64_t K, int64_t group_size) {
    const char* name = "gemv_w4a16_indexed";
    TORCH_CHECK(Wq_packed.is_cuda() && Wq_packed.scalar_type() == torch::kUInt8 && Wq_packed.is_contiguous() &&
                    Wq_packed.dim() == 2,
                name, "(Wq_packed): must be a contiguous 2D CUDA uint8 tensor [N, ceil(K/8)*4]");
    TORCH_CHECK(Wq_packed.size(1) == ((K + 7) / 8) * 4, name, ": Wq_packed.size(1) must be ceil(K/8)*4");
    check_f32_cuda_contiguous(scale, "gemv_w4a16_indexed(scale)");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq_packed.size(0), name, ": scale must be 2D [N, num_groups]");
    TORCH_CHECK(idx.is_cuda() && idx.scalar_type() == torch::kInt32 && idx.dim() == 1 && idx.is_contiguous(), name,
                "(idx): must be a contiguous 1D int32 CUDA tensor");
    check_f16_cuda_contiguous(x, "gemv_w4a16_indexed(x)");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == K, name, ": x must be 1D [K]");
    TORCH_CHECK(group_size >= 1 && group_size % 8 == 0, name, ": group_size must be a positive multiple of 8");
    TORCH_CHECK(scale.size(1) == expected_num_groups(K, group_size), name,
                ": scale's num_groups must be ceil(K/group_size)");
    check_same_device(Wq_packed, x, name);
    check_same_device(Wq_packed, idx, name);
    check_same_device(Wq_packed, scale, name);
    const at::DeviceGuard guard(x.device());
    const int64_t k = idx.size(0);
    auto y = torch::empty({k}, x.options());
    check_status(soi_gemv_w4a16_indexed(Wq_packed.data_ptr<uint8_t>(), scale.data_ptr<float>(), Wq_packed.size(0),
                                        idx.data_ptr<int32_t>(), k, h16(x), h16m(y), K, group_size, scale.size(1),
                                        cur_stream(x)),
                 name);
    return y;
}

torch::Tensor gemv_w4a16_indexed_accumulate(torch::Tensor Wq_T, torch::Tensor scale_T, torch::Tensor idx,
                                            torch::Tensor h_selected, int64_t H, int64_t group_size) {
    const char* name = "gemv_w4a16_indexed_accumulate";
    TORCH_CHECK(Wq_T.is_cuda() && Wq_T.scalar_type() == torch::kUInt8 && Wq_T.is_contiguous() && Wq_T.dim() == 2,
                name, "(Wq_T): must be a contiguous 2D CUDA uint8 tensor [I, ceil(H/8)*4]");
    TORCH_CHECK(Wq_T.size(1) == ((H + 7) / 8) * 4, name, ": Wq_T.size(1) must be ceil(H/8)*4");
    check_f32_cuda_contiguous(scale_T, "gemv_w4a16_indexed_accumulate(scale_T)");
    TORCH_CHECK(scale_T.dim() == 2 && scale_T.size(0) == Wq_T.size(0), name, ": scale_T must be 2D [I, num_groups]");
    TORCH_CHECK(idx.is_cuda() && idx.scalar_type() == torch::kInt32 && idx.dim() == 1 && idx.is_contiguous(), name,
                "(idx): must be a contiguous 1D int32 CUDA tensor");
    check_f16_cuda_contiguous(h_selected, "gemv_w4a16_indexed_accumulate(h_selected)");
    TORCH_CHECK(h_selected.dim() == 1 && h_selected.size(0) == idx.size(0), name, ": h_selected must be 1D [k]");
    TORCH_CHECK(H >= 1 && group_size >= 1 && group_size % 8 == 0, name, ": bad H or group_size");
    TORCH_CHECK(scale_T.size(1) == expected_num_groups(H, group_size), name,
                ": scale_T's num_groups must be ceil(H/group_size)");
    check_same_device(Wq_T, h_selected, name);
    check_same_device(Wq_T, idx, name);
    check_same_device(Wq_T, scale_T, name);
    const at::DeviceGuard guard(h_selected.device());
    const int64_t k = idx.size(0);
    auto y = torch::empty({H}, h_selected.options());
    const size_t wsb = soi_sparse_accumulate_workspace_bytes(H, k);
    auto ws = zeroed_workspace(h_selected, wsb);
    check_status(soi_gemv_w4a16_indexed_accumulate(Wq_T.data_ptr<uint8_t>(), scale_T.data_ptr<float>(), Wq_T.size(0),
                                                   idx.data_ptr<int32_t>(), k, h16(h_selected), h16m(y), H, group_size,
                                                   scale_T.size(1), ws.data_ptr<uint8_t>(), wsb,
                                                   cur_stream(h_selected)),
                 name);
    return y;
}

void gather_rows_device(torch::Tensor src, torch::Tensor idx, torch::Tensor dst) {
    const char* name = "gather_rows_device";
    TORCH_CHECK(src.is_cuda() && src.scalar_type() == torch::kUInt8 && src.dim() == 2 && src.is_contiguous(), name,
                "(src): must be a contiguous 2D CUDA uint8 tensor");
    TORCH_CHECK(idx.is_cuda() && idx.scalar_type() == torch::kInt32 && idx.dim() == 1 && idx.is_contiguous(), name,
                "(idx): must be a contiguous 1D int32 CUDA tensor");
    TORCH_CHECK(dst.is_cuda() && dst.scalar_type() == torch::kUInt8 && dst.is_contiguous(), name,
                "(dst): must be a contiguous CUDA uint8 tensor");
    TORCH_CHECK(dst.numel() >= idx.size(0) * src.size(1), name, "(dst): too small for k * row_nbytes bytes");
    check_same_device(src, idx, name);
    check_same_device(src, dst, name);
    const at::DeviceGuard guard(src.device());
    check_status(soi_gather_rows_device(src.data_ptr<uint8_t>(), src.size(0), src.size(1), idx.data_ptr<int32_t>(),
                                        idx.size(0), dst.data_ptr<uint8_t>(), cur_stream(src)),
                 name);
}

// ---------------------------------------------------------------------------
// attention, top-k, host gathers
// ---------------------------------------------------------------------------

torch::Tensor decode_attention(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, int64_t cur_len) {
    check_f16_cuda_contiguous(q, "decode_attention(q)");
    check_f16_cuda_contiguous(k_cache, "decode_attention(k_cache)");
    check_f16_cuda_contiguous(v_cache, "decode_attention(v_cache)");
    TORCH_CHECK(q.dim() == 2, "decode_attention: q must be 2D [num_q_heads, head_dim]");
    TORCH_CHECK(k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes(),
                "decode_attention: k_cache/v_cache must be 3D [num_kv_heads, max_seq_len, head_dim] and same shape");
    TORCH_CHECK(q.size(1) == k_cache.size(2), "decode_attention: q's head_dim must match the cache's head_dim");
    const int64_t NQ = q.size(0), NKV = k_cache.size(0), S = k_cache.size(1), hd = k_cache.size(2);
    TORCH_CHECK(NKV >= 1 && NQ % NKV == 0, "decode_attention: num_q_heads must be a multiple of num_kv_heads");
    TORCH_CHECK(cur_len >= 1 && cur_len <= S, "decode_attention: cur_len out of range for max_seq_len");
    TORCH_CHECK(hd >= 1 && hd <= 1024, "decode_attention: head_dim must be in [1, 1024]");
    check_same_device(q, k_cache, "decode_attention");
    check_same_device(q, v_cache, "decode_attention");
    const at::DeviceGuard guard(q.device());
    auto out = torch::empty({NQ, hd}, q.options());
    const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
    const size_t wsb = soi_decode_attention_workspace_bytes(NQ, NKV, hd, cur_len);
    auto ws = zeroed_workspace(q, wsb);
    check_status(soi_decode_attention(h16(q), h16(k_cache), h16(v_cache), h16m(out), NQ, NKV, S, hd, cur_len, scale,
                                      ws.data_ptr<uint8_t>(), wsb, cur_stream(q)),
                 "decode_attention");
    return out;
}

std::tuple<torch::Tensor, torch::Tensor> topk_threshold_select(torch::Tensor abs_g, int64_t k) {
    check_f32_cuda_contiguous(abs_g, "topk_threshold_select(abs_g)");
    TORCH_CHECK(abs_g.dim() == 1, "topk_threshold_select: abs_g must be 1D [I]");
    TORCH_CHECK(k >= 1 && k <= abs_g.size(0), "topk_threshold_select: k must be in [1, I]");
    const at::DeviceGuard guard(abs_g.device());
    const int64_t n = abs_g.size(0);
    auto out_indices = torch::empty({k}, abs_g.options().dtype(torch::kInt32));
    auto out_count = torch::empty({1}, abs_g.options().dtype(torch::kInt32));
    check_status(soi_topk_threshold_select(abs_g.data_ptr<float>(), n, k, out_indices.data_ptr<int32_t>(),
                                           out_count.data_ptr<int32_t>(), cur_stream(abs_g)),
                 "topk_threshold_select");
    return {out_indices, out_count};
}

namespace {

void check_gather_rows_common(const torch::Tensor& matrix, const torch::Tensor& indices, const torch::Tensor& gpu_dst,
                              const char* name) {
    TORCH_CHECK(matrix.is_cpu() && matrix.is_pinned(), name, "(matrix): must be pinned host memory");
    TORCH_CHECK(matrix.scalar_type() == torch::kUInt8 && matrix.dim() == 2 && matrix.is_contiguous(), name,
                "(matrix): must be a contiguous 2D uint8 tensor [num_rows, row_nbytes]");
    TORCH_CHECK(indices.is_cpu() && indices.scalar_type() == torch::kInt64 && indices.dim() == 1, name,
                "(indices): must be a 1D int64 CPU tensor");
    TORCH_CHECK(gpu_dst.is_cuda() && gpu_dst.scalar_type() == torch::kUInt8 && gpu_dst.is_contiguous(), name,
                "(gpu_dst): must be a contiguous CUDA uint8 tensor");
    TORCH_CHECK(gpu_dst.numel() >= indices.size(0) * matrix.size(1), name,
                "(gpu_dst): too small for k * row_nbytes bytes");
}

}  // namespace

void gather_rows_staged(torch::Tensor matrix, torch::Tensor indices, torch::Tensor staging, torch::Tensor gpu_dst) {
    check_gather_rows_common(matrix, indices, gpu_dst, "gather_rows_staged");
    TORCH_CHECK(staging.is_cpu() && staging.is_pinned() && staging.scalar_type() == torch::kUInt8,
                "gather_rows_staged(staging): must be pinned host uint8 memory");
    TORCH_CHECK(staging.is_contiguous(), "gather_rows_staged(staging): must be contiguous");
    const int64_t k = indices.size(0), row_nbytes = matrix.size(1);
    TORCH_CHECK(staging.numel() >= k * row_nbytes, "gather_rows_staged(staging): too small for k * row_nbytes bytes");
    auto idx = indices.contiguous();
    const at::DeviceGuard guard(gpu_dst.device());
    check_status(soi_gather_rows_staged(matrix.data_ptr<uint8_t>(), matrix.size(0), row_nbytes,
                                        idx.data_ptr<int64_t>(), k, staging.data_ptr<uint8_t>(),
                                        gpu_dst.data_ptr<uint8_t>(), cur_stream(gpu_dst)),
                 "gather_rows_staged");
}

void gather_rows_naive(torch::Tensor matrix, torch::Tensor indices, torch::Tensor gpu_dst) {
    check_gather_rows_common(matrix, indices, gpu_dst, "gather_rows_naive");
    auto idx = indices.contiguous();
    const at::DeviceGuard guard(gpu_dst.device());
    check_status(soi_gather_rows_naive(matrix.data_ptr<uint8_t>(), matrix.size(0), matrix.size(1),
                                       idx.data_ptr<int64_t>(), idx.size(0), gpu_dst.data_ptr<uint8_t>(),
                                       cur_stream(gpu_dst)),
                 "gather_rows_naive");
}

// ---------------------------------------------------------------------------
// decoder-step glue (reference names: rmsnorm 141-150, gemv_fp16_v3 201-208,
// kv_cache_append 450-466, rope_apply 490-505)
// ---------------------------------------------------------------------------

torch::Tensor rmsnorm(torch::Tensor x, torch::Tensor weight, double eps) {
    check_f16_cuda_contiguous(x, "rmsnorm(x)");
    check_f16_cuda_contiguous(weight, "rmsnorm(weight)");
    TORCH_CHECK(x.dim() == 2, "rmsnorm: x must be 2D [rows, hidden]");
    TORCH_CHECK(weight.dim() == 1 && weight.size(0) == x.size(1), "rmsnorm: weight shape must match x's hidden dim");
    TORCH_CHECK(x.size(1) % 2 == 0, "rmsnorm: hidden dim must be even (half2 vectorization)");
    check_same_device(x, weight, "rmsnorm");
    const at::DeviceGuard guard(x.device());
    auto out = torch::empty_like(x);
    check_status(soi_rmsnorm(h16(x), h16(weight), h16m(out), x.size(0), x.size(1), static_cast<float>(eps),
                             cur_stream(x)),
                 "rmsnorm");
    return out;
}

torch::Tensor gemv_fp16_v3(torch::Tensor W, torch::Tensor x) {
    check_f16_cuda_contiguous(W, "gemv_fp16_v3(W)");
    check_f16_cuda_contiguous(x, "gemv_fp16_v3(x)");
    TORCH_CHECK(W.dim() == 2, "gemv_fp16_v3: W must be 2D [N, K]");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == W.size(1), "gemv_fp16_v3: x must be 1D [K] matching W's K");
    TORCH_CHECK(W.size(1) % 8 == 0, "gemv_fp16_v3: K must be a multiple of 8 (float4-vectorized loads)");
    check_same_device(W, x, "gemv_fp16_v3");
    const at::DeviceGuard guard(x.device());
    auto y = torch::empty({W.size(0)}, x.options());
    check_status(soi_gemv_f16(h16(W), h16(x), h16m(y), W.size(0), W.size(1), cur_stream(x)), "gemv_fp16_v3");
    return y;
}

// reference bindings.cpp:434-448 (same checks and messages)
torch::Tensor swiglu_gate_up(torch::Tensor gate_W, torch::Tensor up_W, torch::Tensor x) {
    check_f16_cuda_contiguous(gate_W, "swiglu_gate_up(gate_W)");
    check_f16_cuda_contiguous(up_W, "swiglu_gate_up(up_W)");
    check_f16_cuda_contiguous(x, "swiglu_gate_up(x)");
    TORCH_CHECK(gate_W.dim() == 2 && up_W.dim() == 2, "swiglu_gate_up: gate_W and up_W must be 2D [I, H]");
    TORCH_CHECK(gate_W.sizes() == up_W.sizes(), "swiglu_gate_up: gate_W and up_W must have the same shape");
    TORCH_CHECK(x.dim() == 1 && x.size(0) == gate_W.size(1),
                "swiglu_gate_up: x must be 1D [H] matching the weights' H");
    TORCH_CHECK(gate_W.size(1) % 8 == 0, "swiglu_gate_up: H must be a multiple of 8 (float4-vectorized loads)");
    check_same_device(gate_W, x, "swiglu_gate_up");
    check_same_device(up_W, x, "swiglu_gate_up");
    const at::DeviceGuard guard(x.device());
    auto h = torch::empty({gate_W.size(0)}, x.options());
    check_status(soi_swiglu_gate_up(h16(gate_W), h16(up_W), h16(x), h16m(h), gate_W.size(0), gate_W.size(1),
                                    cur_stream(x)),
                 "swiglu_gate_up");
    return h;
}

void kv_cache_append(torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor k_new, torch::Tensor v_new,
                     int64_t pos) {
    check_f16_cuda_contiguous(k_cache, "kv_cache_append(k_cache)");
    check_f16_cuda_contiguous(v_cache, "kv_cache_append(v_cache)");
    check_f16_cuda_contiguous(k_new, "kv_cache_append(k_new)");
    check_f16_cuda_contiguous(v_new, "kv_cache_append(v_new)");
    TORCH_CHECK(k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes(),
                "kv_cache_append: k_cache/v_cache must be 3D [num_kv_heads, max_seq_len, head_dim] and same shape");
    TORCH_CHECK(k_new.sizes() == v_new.sizes(), "kv_cache_append: k_new/v_new must have the same shape");
    TORCH_CHECK(k_new.dim() == 2 && k_new.size(0) == k_cache.size(0) && k_new.size(1) == k_cache.size(2),
                "kv_cache_append: k_new/v_new must be 2D [num_kv_heads, head_dim] matching the cache");
    TORCH_CHECK(pos >= 0 && pos < k_cache.size(1), "kv_cache_append: pos out of range for max_seq_len");
    for (const auto* t : {&v_cache, &k_new, &v_new}) check_same_device(k_cache, *t, "kv_cache_append");
    const at::DeviceGuard guard(k_cache.device());
    check_status(soi_kv_cache_append(h16(k_new), h16(v_new), h16m(k_cache), h16m(v_cache), k_cache.size(0),
                                     k_cache.size(1), k_cache.size(2), pos, cur_stream(k_cache)),
                 "kv_cache_append");
}

void rope_apply(torch::Tensor x, torch::Tensor cos_vals, torch::Tensor sin_vals) {
    check_f16_cuda_contiguous(x, "rope_apply(x)");
    TORCH_CHECK(x.dim() == 2, "rope_apply: x must be 2D [num_heads, head_dim]");
    TORCH_CHECK(x.size(1) % 2 == 0, "rope_apply: head_dim must be even");
    TORCH_CHECK(cos_vals.is_cuda() && cos_vals.scalar_type() == torch::kFloat32 && cos_vals.is_contiguous(),
                "rope_apply: cos_vals must be a contiguous float32 CUDA tensor");
    TORCH_CHECK(sin_vals.is_cuda() && sin_vals.scalar_type() == torch::kFloat32 && sin_vals.is_contiguous() &&
                    sin_vals.sizes() == cos_vals.sizes(),
                "rope_apply: sin_vals must match cos_vals (contiguous float32 CUDA, same shape)");
    TORCH_CHECK(cos_vals.dim() == 1 && cos_vals.size(0) == x.size(1) / 2,
                "rope_apply: cos_vals/sin_vals must be 1D [head_dim / 2]");
    check_same_device(x, cos_vals, "rope_apply");
    check_same_device(x, sin_vals, "rope_apply");
    const at::DeviceGuard guard(x.device());
    check_status(soi_rope_apply(h16m(x), cos_vals.data_ptr<float>(), sin_vals.data_ptr<float>(), x.size(0), x.size(1),
                                cur_stream(x)),
                 "rope_apply");
}

// ---------------------------------------------------------------------------
// decode-engine forms: write into caller buffers, allocate nothing (so a
// captured HIP graph replays them); position / token / counts are device int32
// ---------------------------------------------------------------------------

namespace {

void need(const torch::Tensor& t, torch::ScalarType dt, const torch::Tensor& dev, const char* name, const char* arg) {
    TORCH_CHECK(t.is_cuda() && t.scalar_type() == dt && t.is_contiguous(), name, "(", arg, "): must be a contiguous ",
                c10::toString(dt), " CUDA tensor");
    TORCH_CHECK(t.device() == dev.device(), name, "(", arg, "): all tensors must be on one device");
}

void need_numel(const torch::Tensor& t, int64_t n, const char* name, const char* arg) {
    TORCH_CHECK(t.numel() >= n, name, "(", arg, "): needs at least ", n, " elements, has ", t.numel());
}

}  // namespace

void rmsnorm_into(torch::Tensor x, torch::Tensor weight, torch::Tensor out, double eps) {
    const char* n = "rmsnorm_into";
    need(x, torch::kFloat16, x, n, "x");
    need(weight, torch::kFloat16, x, n, "weight");
    need(out, torch::kFloat16, x, n, "out");
    const int64_t hidden = weight.numel();
    TORCH_CHECK(hidden >= 1 && x.numel() % hidden == 0 && out.numel() == x.numel(), n, ": shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_rmsnorm(h16(x), h16(weight), h16m(out), x.numel() / hidden, hidden, static_cast<float>(eps),
                             cur_stream(x)),
                 n);
}

void residual_rmsnorm_(torch::Tensor x, torch::Tensor delta, torch::Tensor weight, torch::Tensor out, double eps) {
    const char* n = "residual_rmsnorm_";
    need(x, torch::kFloat16, x, n, "x");
    need(delta, torch::kFloat16, x, n, "delta");
    need(weight, torch::kFloat16, x, n, "weight");
    need(out, torch::kFloat16, x, n, "out");
    const int64_t hidden = weight.numel();
    TORCH_CHECK(hidden >= 1 && x.numel() % hidden == 0 && delta.numel() == x.numel() && out.numel() == x.numel(), n,
                ": shape mismatch");
    TORCH_CHECK(out.data_ptr() != x.data_ptr() && out.data_ptr() != delta.data_ptr(), n,
                ": out must not alias x or delta");
    const at::DeviceGuard guard(x.device());
    check_status(soi_residual_rmsnorm(h16m(x), h16(delta), h16(weight), h16m(out), x.numel() / hidden, hidden,
                                      static_cast<float>(eps), cur_stream(x)),
                 n);
}

void final_norm_advance(torch::Tensor x, torch::Tensor delta, torch::Tensor weight, torch::Tensor out, double eps,
                        torch::Tensor pos) {
    const char* n = "final_norm_advance";
    need(x, torch::kFloat16, x, n, "x");
    need(delta, torch::kFloat16, x, n, "delta");
    need(weight, torch::kFloat16, x, n, "weight");
    need(out, torch::kFloat16, x, n, "out");
    need(pos, torch::kInt32, x, n, "pos");
    need_numel(pos, 1, n, "pos");
    TORCH_CHECK(x.numel() == weight.numel() && delta.numel() == x.numel() && out.numel() == x.numel(), n,
                ": shape mismatch");
    TORCH_CHECK(out.data_ptr() != x.data_ptr() && out.data_ptr() != delta.data_ptr(), n,
                ": out must not alias x or delta");
    const at::DeviceGuard guard(x.device());
    check_status(soi_final_norm_advance(h16m(x), h16(delta), h16(weight), h16m(out), x.numel(), static_cast<float>(eps),
                                        pos.data_ptr<int32_t>(), cur_stream(x)),
                 n);
}

void qk_norm_rope_append(torch::Tensor qkv, torch::Tensor q_norm, torch::Tensor k_norm, torch::Tensor cos_table,
                         torch::Tensor sin_table, torch::Tensor pos, torch::Tensor q_out, torch::Tensor k_cache,
                         torch::Tensor v_cache, double eps) {
    const char* n = "qk_norm_rope_append";
    need(qkv, torch::kFloat16, qkv, n, "qkv");
    need(q_norm, torch::kFloat16, qkv, n, "q_norm");
    need(k_norm, torch::kFloat16, qkv, n, "k_norm");
    need(cos_table, torch::kFloat32, qkv, n, "cos_table");
    need(sin_table, torch::kFloat32, qkv, n, "sin_table");
    need(pos, torch::kInt32, qkv, n, "pos");
    need(q_out, torch::kFloat16, qkv, n, "q_out");
    need(k_cache, torch::kFloat16, qkv, n, "k_cache");
    need(v_cache, torch::kFloat16, qkv, n, "v_cache");
    TORCH_CHECK(k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes(), n,
                ": caches must be 3D [num_kv_heads, max_seq_len, head_dim] of one shape");
    TORCH_CHECK(q_out.dim() == 2 && q_out.size(1) == k_cache.size(2), n, ": q_out must be 2D [num_q_heads, head_dim]");
    const int64_t NQ = q_out.size(0), NKV = k_cache.size(0), S = k_cache.size(1), hd = k_cache.size(2);
    TORCH_CHECK(qkv.numel() == (NQ + 2 * NKV) * hd, n, ": qkv must hold (NQ + 2*NKV) * head_dim values");
    TORCH_CHECK(q_norm.numel() == hd && k_norm.numel() == hd, n, ": norm weights must be [head_dim]");
    TORCH_CHECK(cos_table.numel() == S * (hd / 2) && sin_table.numel() == S * (hd / 2), n,
                ": RoPE tables must be [max_seq_len, head_dim/2]");
    need_numel(pos, 1, n, "pos");
    const at::DeviceGuard guard(qkv.device());
    check_status(soi_qk_norm_rope_append(h16(qkv), h16(q_norm), h16(k_norm), cos_table.data_ptr<float>(),
                                         sin_table.data_ptr<float>(), pos.data_ptr<int32_t>(), h16m(q_out),
                                         h16m(k_cache), h16m(v_cache), NQ, NKV, S, hd, static_cast<float>(eps),
                                         cur_stream(qkv)),
                 n);
}

int64_t decode_attention_step_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t max_seq) {
    return static_cast<int64_t>(soi_decode_attention_step_workspace_bytes(NQ, NKV, head_dim, max_seq));
}

static void attention_step_impl(torch::Tensor qkv, torch::Tensor q_norm, torch::Tensor k_norm,
                                torch::Tensor cos_table, torch::Tensor sin_table, torch::Tensor pos,
                                torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor out, double eps,
                                torch::Tensor workspace_buf, bool deferred, const char* n) {
    need(qkv, torch::kFloat16, qkv, n, "qkv");
    need(q_norm, torch::kFloat16, qkv, n, "q_norm");
    need(k_norm, torch::kFloat16, qkv, n, "k_norm");
    need(cos_table, torch::kFloat32, qkv, n, "cos_table");
    need(sin_table, torch::kFloat32, qkv, n, "sin_table");
    need(pos, torch::kInt32, qkv, n, "pos");
    need(k_cache, torch::kFloat16, qkv, n, "k_cache");
    need(v_cache, torch::kFloat16, qkv, n, "v_cache");
    need(out, torch::kFloat16, qkv, n, "out");
    need(workspace_buf, torch::kUInt8, qkv, n, "workspace");
    TORCH_CHECK(k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes(), n,
                ": caches must be 3D [num_kv_heads, max_seq_len, head_dim] of one shape");
    TORCH_CHECK(out.dim() == 2 && out.size(1) == k_cache.size(2), n, ": out must be 2D [num_q_heads, head_dim]");
    const int64_t NQ = out.size(0), NKV = k_cache.size(0), S = k_cache.size(1), hd = k_cache.size(2);
    TORCH_CHECK(qkv.numel() == (NQ + 2 * NKV) * hd, n, ": qkv must hold (NQ + 2*NKV) * head_dim values");
    TORCH_CHECK(q_norm.numel() == hd && k_norm.numel() == hd, n, ": norm weights must be [head_dim]");
    TORCH_CHECK(cos_table.numel() == S * (hd / 2) && sin_table.numel() == S * (hd / 2), n,
                ": RoPE tables must be [max_seq_len, head_dim/2]");
    need_numel(pos, 1, n, "pos");
    const at::DeviceGuard guard(qkv.device());
    auto fn = deferred ? soi_decode_attention_step_deferred : soi_decode_attention_step;
    check_status(fn(h16(qkv), h16(q_norm), h16(k_norm), cos_table.data_ptr<float>(), sin_table.data_ptr<float>(),
                    pos.data_ptr<int32_t>(), h16m(k_cache), h16m(v_cache), h16m(out), NQ, NKV, S, hd,
                    static_cast<float>(eps), 1.0f / std::sqrt(static_cast<float>(hd)),
                    workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), cur_stream(qkv)),
                 n);
}

void decode_attention_step(torch::Tensor qkv, torch::Tensor q_norm, torch::Tensor k_norm, torch::Tensor cos_table,
                           torch::Tensor sin_table, torch::Tensor pos, torch::Tensor k_cache, torch::Tensor v_cache,
                           torch::Tensor out, double eps, torch::Tensor workspace_buf) {
    attention_step_impl(qkv, q_norm, k_norm, cos_table, sin_table, pos, k_cache, v_cache, out, eps, workspace_buf,
                        false, "decode_attention_step");
}

void decode_attention_step_deferred(torch::Tensor qkv, torch::Tensor q_norm, torch::Tensor k_norm,
                                    torch::Tensor cos_table, torch::Tensor sin_table, torch::Tensor pos,
                                    torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor out, double eps,
                                    torch::Tensor workspace_buf) {
    attention_step_impl(qkv, q_norm, k_norm, cos_table, sin_table, pos, k_cache, v_cache, out, eps, workspace_buf,
                        true, "decode_attention_step_deferred");
}

void gemv_w4a16_attn_combine_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor workspace_buf,
                                  torch::Tensor attn_out, torch::Tensor pos, int64_t num_kv_heads,
                                  int64_t max_seq_len, torch::Tensor y, int64_t group_size,
                                  c10::optional<torch::Tensor> res, c10::optional<torch::Tensor> res_out) {
    const char* n = "gemv_w4a16_attn_combine_into";
    need(Wq, torch::kUInt8, attn_out, n, "Wq");
    need(scale, torch::kFloat32, attn_out, n, "scale");
    need(workspace_buf, torch::kUInt8, attn_out, n, "workspace");
    need(attn_out, torch::kFloat16, attn_out, n, "attn_out");
    need(pos, torch::kInt32, attn_out, n, "pos");
    need(y, torch::kFloat16, attn_out, n, "y");
    need_numel(pos, 1, n, "pos");
    TORCH_CHECK(attn_out.dim() == 2, n, ": attn_out must be 2D [num_q_heads, head_dim]");
    const int64_t NQ = attn_out.size(0), hd = attn_out.size(1), K = NQ * hd;
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4, n, ": Wq must be [N, ceil(K/8)*4], K = NQ * head_dim");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0) && y.numel() == Wq.size(0), n,
                ": scale / y shape mismatch");
    TORCH_CHECK(res.has_value() == res_out.has_value(), n, ": res and res_out go together");
    const uint16_t* rp = nullptr;
    uint16_t* rop = nullptr;
    if (res.has_value()) {
        need(*res, torch::kFloat16, attn_out, n, "res");
        need(*res_out, torch::kFloat16, attn_out, n, "res_out");
        TORCH_CHECK(res->numel() == Wq.size(0) && res_out->numel() == Wq.size(0), n,
                    ": res and res_out must have N values");
        TORCH_CHECK(res_out->data_ptr() != y.data_ptr() && res->data_ptr() != y.data_ptr(), n,
                    ": res / res_out must not alias y");
        rp = h16(*res);
        rop = h16m(*res_out);
    }
    const at::DeviceGuard guard(attn_out.device());
    check_status(soi_gemv_w4a16_attn_combine(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(),
                                             workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), h16(attn_out),
                                             pos.data_ptr<int32_t>(), NQ, num_kv_heads, hd, max_seq_len, h16m(y), rp,
                                             rop, Wq.size(0), group_size, scale.size(1), cur_stream(attn_out)),
                 n);
}

int64_t decode_attention_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t cur_len) {
    return static_cast<int64_t>(soi_decode_attention_workspace_bytes(NQ, NKV, head_dim, cur_len));
}

void decode_attention_into(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, int64_t cur_len,
                           torch::Tensor out, torch::Tensor workspace_buf) {
    const char* n = "decode_attention_into";
    need(q, torch::kFloat16, q, n, "q");
    need(k_cache, torch::kFloat16, q, n, "k_cache");
    need(v_cache, torch::kFloat16, q, n, "v_cache");
    need(out, torch::kFloat16, q, n, "out");
    need(workspace_buf, torch::kUInt8, q, n, "workspace");
    TORCH_CHECK(q.dim() == 2 && k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes() &&
                    q.size(1) == k_cache.size(2) && out.sizes() == q.sizes(),
                n, ": q / out [num_q_heads, head_dim], caches [num_kv_heads, max_seq_len, head_dim]");
    const int64_t NQ = q.size(0), NKV = k_cache.size(0), S = k_cache.size(1), hd = k_cache.size(2);
    TORCH_CHECK(cur_len >= 1 && cur_len <= S, n, ": cur_len out of range for max_seq_len");
    const at::DeviceGuard guard(q.device());
    check_status(soi_decode_attention(h16(q), h16(k_cache), h16(v_cache), h16m(out), NQ, NKV, S, hd, cur_len,
                                      1.0f / std::sqrt(static_cast<float>(hd)), workspace_buf.data_ptr<uint8_t>(),
                                      workspace_buf.numel(), cur_stream(q)),
                 n);
}

void decode_attention_at(torch::Tensor q, torch::Tensor k_cache, torch::Tensor v_cache, torch::Tensor pos,
                         torch::Tensor out, torch::Tensor workspace_buf) {
    const char* n = "decode_attention_at";
    need(q, torch::kFloat16, q, n, "q");
    need(k_cache, torch::kFloat16, q, n, "k_cache");
    need(v_cache, torch::kFloat16, q, n, "v_cache");
    need(pos, torch::kInt32, q, n, "pos");
    need(out, torch::kFloat16, q, n, "out");
    need(workspace_buf, torch::kUInt8, q, n, "workspace");
    TORCH_CHECK(q.dim() == 2 && k_cache.dim() == 3 && v_cache.sizes() == k_cache.sizes() &&
                    q.size(1) == k_cache.size(2) && out.numel() == q.numel(),
                n, ": shape mismatch");
    need_numel(pos, 1, n, "pos");
    const int64_t NQ = q.size(0), NKV = k_cache.size(0), S = k_cache.size(1), hd = k_cache.size(2);
    const at::DeviceGuard guard(q.device());
    check_status(soi_decode_attention_at(h16(q), h16(k_cache), h16(v_cache), h16m(out), NQ, NKV, S, hd,
                                         pos.data_ptr<int32_t>(), 1.0f / std::sqrt(static_cast<float>(hd)),
                                         workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), cur_stream(q)),
                 n);
}

void gemv_w4a16_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x, torch::Tensor y, int64_t K,
                     int64_t group_size) {
    const char* n = "gemv_w4a16_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(x, torch::kFloat16, x, n, "x");
    need(y, torch::kFloat16, x, n, "y");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K, n, ": Wq / x shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0) && y.numel() == Wq.size(0), n,
                ": scale / y shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_group_lop3(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), h16m(y),
                                           Wq.size(0), K, group_size, scale.size(1), cur_stream(x)),
                 n);
}

void gemv_w4a16_residual_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x, torch::Tensor y,
                              torch::Tensor res, torch::Tensor res_out, int64_t K, int64_t group_size) {
    const char* n = "gemv_w4a16_residual_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(x, torch::kFloat16, x, n, "x");
    need(y, torch::kFloat16, x, n, "y");
    need(res, torch::kFloat16, x, n, "res");
    need(res_out, torch::kFloat16, x, n, "res_out");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K, n, ": Wq / x shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0) && y.numel() == Wq.size(0), n,
                ": scale / y shape mismatch");
    TORCH_CHECK(res.numel() == Wq.size(0) && res_out.numel() == Wq.size(0), n, ": res and res_out must have N values");
    TORCH_CHECK(res_out.data_ptr() != y.data_ptr() && res.data_ptr() != y.data_ptr(), n,
                ": res / res_out must not alias y");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_residual(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), h16m(y), h16(res),
                                         h16m(res_out), Wq.size(0), K, group_size, scale.size(1), cur_stream(x)),
                 n);
}

void gemv_w4a16_indexed_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor idx, torch::Tensor x,
                             torch::Tensor y, int64_t K, int64_t group_size) {
    const char* n = "gemv_w4a16_indexed_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(idx, torch::kInt32, x, n, "idx");
    need(x, torch::kFloat16, x, n, "x");
    need(y, torch::kFloat16, x, n, "y");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K, n, ": Wq / x shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0) && y.numel() == idx.numel(), n,
                ": scale / y shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_indexed(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), Wq.size(0),
                                        idx.data_ptr<int32_t>(), idx.numel(), h16(x), h16m(y), K, group_size,
                                        scale.size(1), cur_stream(x)),
                 n);
}

void gemv_w4a16_indexed_accumulate_into(torch::Tensor Wq_T, torch::Tensor scale_T, torch::Tensor idx,
                                        torch::Tensor h_sel, torch::Tensor y, int64_t H, int64_t group_size,
                                        torch::Tensor workspace_buf) {
    const char* n = "gemv_w4a16_indexed_accumulate_into";
    need(Wq_T, torch::kUInt8, h_sel, n, "Wq_T");
    need(scale_T, torch::kFloat32, h_sel, n, "scale_T");
    need(idx, torch::kInt32, h_sel, n, "idx");
    need(h_sel, torch::kFloat16, h_sel, n, "h_sel");
    need(y, torch::kFloat16, h_sel, n, "y");
    need(workspace_buf, torch::kUInt8, h_sel, n, "workspace");
    TORCH_CHECK(Wq_T.dim() == 2 && Wq_T.size(1) == ((H + 7) / 8) * 4 && y.numel() == H, n, ": Wq_T / y mismatch");
    TORCH_CHECK(scale_T.dim() == 2 && scale_T.size(0) == Wq_T.size(0) && h_sel.numel() == idx.numel(), n,
                ": scale_T / h_sel shape mismatch");
    const at::DeviceGuard guard(h_sel.device());
    check_status(soi_gemv_w4a16_indexed_accumulate(Wq_T.data_ptr<uint8_t>(), scale_T.data_ptr<float>(), Wq_T.size(0),
                                                   idx.data_ptr<int32_t>(), idx.numel(), h16(h_sel), h16m(y), H,
                                                   group_size, scale_T.size(1), workspace_buf.data_ptr<uint8_t>(),
                                                   workspace_buf.numel(), cur_stream(h_sel)),
                 n);
}

int64_t sparse_accumulate_workspace_bytes(int64_t H, int64_t k) {
    return static_cast<int64_t>(soi_sparse_accumulate_workspace_bytes(H, k));
}

void build_dip_descriptors_into(torch::Tensor sel, torch::Tensor slot_of, torch::Tensor desc,
                                torch::Tensor miss_channels, torch::Tensor miss_count) {
    const char* n = "build_dip_descriptors_into";
    for (auto* t : {&sel, &slot_of, &desc, &miss_channels, &miss_count}) need(*t, torch::kInt32, sel, n, "int32 arg");
    TORCH_CHECK(desc.numel() >= sel.numel() && miss_channels.numel() >= sel.numel() && miss_count.numel() >= 1, n,
                ": output buffers too small");
    const at::DeviceGuard guard(sel.device());
    check_status(soi_build_dip_descriptors(sel.data_ptr<int32_t>(), sel.numel(), slot_of.data_ptr<int32_t>(),
                                           slot_of.numel(), desc.data_ptr<int32_t>(),
                                           miss_channels.data_ptr<int32_t>(), miss_count.data_ptr<int32_t>(),
                                           cur_stream(sel)),
                 n);
}

void gemv_dip_fused_up_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor staging_Wq,
                            torch::Tensor staging_scale, torch::Tensor desc, torch::Tensor x, torch::Tensor y,
                            int64_t K, int64_t group_size) {
    const char* n = "gemv_dip_fused_up_into";
    check_dip_fused_common(cache_Wq, cache_scale, staging_Wq, staging_scale, desc, K, n);
    need(x, torch::kFloat16, desc, n, "x");
    need(y, torch::kFloat16, desc, n, "y");
    TORCH_CHECK(x.numel() == K && y.numel() == desc.numel(), n, ": x / y shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_dip_fused_up(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(),
                                       std::min(cache_Wq.size(0), cache_scale.size(0)), staging_Wq.data_ptr<uint8_t>(),
                                       staging_scale.data_ptr<float>(),
                                       std::min(staging_Wq.size(0), staging_scale.size(0)), desc.data_ptr<int32_t>(),
                                       desc.numel(), h16(x), h16m(y), K, group_size, cache_scale.size(1),
                                       cur_stream(x)),
                 n);
}

void gemv_dip_fused_down_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor staging_Wq,
                              torch::Tensor staging_scale, torch::Tensor desc, torch::Tensor h_sel, torch::Tensor y,
                              int64_t H, int64_t group_size, torch::Tensor workspace_buf) {
    const char* n = "gemv_dip_fused_down_into";
    check_dip_fused_common(cache_Wq, cache_scale, staging_Wq, staging_scale, desc, H, n);
    need(h_sel, torch::kFloat16, desc, n, "h_sel");
    need(y, torch::kFloat16, desc, n, "y");
    need(workspace_buf, torch::kUInt8, desc, n, "workspace");
    TORCH_CHECK(h_sel.numel() == desc.numel() && y.numel() == H, n, ": h_sel / y shape mismatch");
    const at::DeviceGuard guard(h_sel.device());
    check_status(soi_gemv_dip_fused_down(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(),
                                         std::min(cache_Wq.size(0), cache_scale.size(0)),
                                         staging_Wq.data_ptr<uint8_t>(), staging_scale.data_ptr<float>(),
                                         std::min(staging_Wq.size(0), staging_scale.size(0)),
                                         desc.data_ptr<int32_t>(), desc.numel(), h16(h_sel), h16m(y), H, group_size,
                                         cache_scale.size(1), workspace_buf.data_ptr<uint8_t>(),
                                         workspace_buf.numel(), cur_stream(h_sel)),
                 n);
}

void gemv_f16_into(torch::Tensor W, torch::Tensor x, torch::Tensor y) {
    const char* n = "gemv_f16_into";
    need(W, torch::kFloat16, x, n, "W");
    need(x, torch::kFloat16, x, n, "x");
    need(y, torch::kFloat16, x, n, "y");
    TORCH_CHECK(W.dim() == 2 && W.size(1) == x.numel() && y.numel() == W.size(0), n, ": shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_f16(h16(W), h16(x), h16m(y), W.size(0), W.size(1), cur_stream(x)), n);
}

int64_t argmax_workspace_bytes(int64_t n) { return static_cast<int64_t>(soi_argmax_workspace_bytes(n)); }

void argmax_f16_into(torch::Tensor x, torch::Tensor out_index, c10::optional<torch::Tensor> log,
                     c10::optional<torch::Tensor> log_len, torch::Tensor workspace_buf) {
    const char* n = "argmax_f16_into";
    need(x, torch::kFloat16, x, n, "x");
    need(out_index, torch::kInt32, x, n, "out_index");
    need(workspace_buf, torch::kUInt8, x, n, "workspace");
    need_numel(out_index, 1, n, "out_index");
    TORCH_CHECK(log.has_value() == log_len.has_value(), n, ": log and log_len go together");
    int32_t* lp = nullptr;
    int32_t* llp = nullptr;
    int64_t cap = 0;
    if (log.has_value()) {
        need(*log, torch::kInt32, x, n, "log");
        need(*log_len, torch::kInt32, x, n, "log_len");
        need_numel(*log_len, 1, n, "log_len");
        lp = log->data_ptr<int32_t>();
        llp = log_len->data_ptr<int32_t>();
        cap = log->numel();
    }
    const at::DeviceGuard guard(x.device());
    check_status(soi_argmax_f16(h16(x), x.numel(), out_index.data_ptr<int32_t>(), lp, llp, cap,
                                workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), cur_stream(x)),
                 n);
}

void silu_mul_into(torch::Tensor gate, torch::Tensor up, torch::Tensor out) {
    const char* n = "silu_mul_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(up, torch::kFloat16, gate, n, "up");
    need(out, torch::kFloat16, gate, n, "out");
    TORCH_CHECK(up.numel() == gate.numel() && out.numel() == gate.numel(), n, ": shape mismatch");
    const at::DeviceGuard guard(gate.device());
    check_status(soi_silu_mul(h16(gate), h16(up), h16m(out), gate.numel(), cur_stream(gate)), n);
}

void silu_mul_indexed_into(torch::Tensor gate, torch::Tensor idx, torch::Tensor u_sel, torch::Tensor out) {
    const char* n = "silu_mul_indexed_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(idx, torch::kInt32, gate, n, "idx");
    need(u_sel, torch::kFloat16, gate, n, "u_sel");
    need(out, torch::kFloat16, gate, n, "out");
    TORCH_CHECK(u_sel.numel() == idx.numel() && out.numel() == idx.numel(), n, ": shape mismatch");
    const at::DeviceGuard guard(gate.device());
    check_status(soi_silu_mul_indexed(h16(gate), gate.numel(), idx.data_ptr<int32_t>(), h16(u_sel), h16m(out),
                                      idx.numel(), cur_stream(gate)),
                 n);
}

void embed_lookup_into(torch::Tensor table, torch::Tensor token, torch::Tensor out) {
    const char* n = "embed_lookup_into";
    need(table, torch::kFloat16, table, n, "table");
    need(token, torch::kInt32, table, n, "token");
    need(out, torch::kFloat16, table, n, "out");
    TORCH_CHECK(table.dim() == 2 && out.numel() == table.size(1), n, ": out must be [hidden]");
    need_numel(token, 1, n, "token");
    const at::DeviceGuard guard(table.device());
    check_status(soi_embed_lookup(h16(table), table.size(0), table.size(1), token.data_ptr<int32_t>(), h16m(out),
                                  cur_stream(table)),
                 n);
}

void advance_position(torch::Tensor pos, int64_t delta) {
    const char* n = "advance_position";
    need(pos, torch::kInt32, pos, n, "pos");
    need_numel(pos, 1, n, "pos");
    const at::DeviceGuard guard(pos.device());
    check_status(soi_advance_position(pos.data_ptr<int32_t>(), static_cast<int32_t>(delta), cur_stream(pos)), n);
}

void topk_threshold_select_f16abs_into(torch::Tensor gate, int64_t k, torch::Tensor idx_out, torch::Tensor count_out) {
    const char* n = "topk_threshold_select_f16abs_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(idx_out, torch::kInt32, gate, n, "idx_out");
    need(count_out, torch::kInt32, gate, n, "count_out");
    TORCH_CHECK(k >= 1 && k <= gate.numel(), n, ": k must be in [1, n]");
    need_numel(idx_out, k, n, "idx_out");
    need_numel(count_out, 1, n, "count_out");
    const at::DeviceGuard guard(gate.device());
    check_status(soi_topk_threshold_select_f16abs(h16(gate), gate.numel(), k, idx_out.data_ptr<int32_t>(),
                                                  count_out.data_ptr<int32_t>(), cur_stream(gate)),
                 n);
}

// Device address of pinned host memory (hipHostGetDevicePointer), for the
// zero-copy miss gather. Raises if the memory is not device-mapped.
int64_t host_device_pointer(torch::Tensor t) {
    TORCH_CHECK(t.is_cpu() && t.is_pinned(), "host_device_pointer: tensor must be pinned host memory");
    void* dp = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dp, t.data_ptr(), 0);
    TORCH_CHECK(e == hipSuccess && dp != nullptr, "host_device_pointer: hipHostGetDevicePointer failed: ",
                hipGetErrorString(e));
    return reinterpret_cast<int64_t>(dp);
}

void gather_rows_device_counted(int64_t src_addr, int64_t num_rows, int64_t row_nbytes, torch::Tensor idx,
                                torch::Tensor count, torch::Tensor dst) {
    const char* n = "gather_rows_device_counted";
    need(idx, torch::kInt32, idx, n, "idx");
    need(count, torch::kInt32, idx, n, "count");
    need(dst, torch::kUInt8, idx, n, "dst");
    need_numel(count, 1, n, "count");
    TORCH_CHECK(src_addr != 0 && num_rows >= 0 && row_nbytes >= 0, n, ": bad source");
    TORCH_CHECK(dst.numel() >= idx.numel() * row_nbytes, n, "(dst): too small for max_k * row_nbytes bytes");
    const at::DeviceGuard guard(idx.device());
    check_status(soi_gather_rows_device_counted(reinterpret_cast<const uint8_t*>(src_addr), num_rows, row_nbytes,
                                                idx.data_ptr<int32_t>(), count.data_ptr<int32_t>(), idx.numel(),
                                                dst.data_ptr<uint8_t>(), cur_stream(idx)),
                 n);
}

void gemv_w4a16_rmsnorm_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x, c10::optional<torch::Tensor> delta,
                             torch::Tensor norm_weight, double eps, c10::optional<torch::Tensor> x_out,
                             c10::optional<torch::Tensor> h_out, torch::Tensor y, int64_t K, int64_t group_size,
                             bool swiglu) {
    const char* n = "gemv_w4a16_rmsnorm_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(x, torch::kFloat16, x, n, "x");
    need(norm_weight, torch::kFloat16, x, n, "norm_weight");
    need(y, torch::kFloat16, x, n, "y");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K && norm_weight.numel() == K, n,
                ": Wq / x / norm_weight shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0), n, ": scale must be [N, num_groups]");
    TORCH_CHECK(y.numel() == (swiglu ? Wq.size(0) / 2 : Wq.size(0)), n, ": y must have N (or N/2 with swiglu) values");
    const uint16_t* dp = nullptr;
    uint16_t* xo = nullptr;
    uint16_t* ho = nullptr;
    if (delta.has_value()) {
        need(*delta, torch::kFloat16, x, n, "delta");
        TORCH_CHECK(delta->numel() == K, n, ": delta must be [K]");
        dp = h16(*delta);
    }
    if (x_out.has_value()) {
        need(*x_out, torch::kFloat16, x, n, "x_out");
        TORCH_CHECK(x_out->numel() == K, n, ": x_out must be [K]");
        xo = h16m(*x_out);
    }
    if (h_out.has_value()) {
        need(*h_out, torch::kFloat16, x, n, "h_out");
        TORCH_CHECK(h_out->numel() == K, n, ": h_out must be [K]");
        ho = h16m(*h_out);
    }
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_rmsnorm(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), dp, h16(norm_weight),
                                        static_cast<float>(eps), xo, ho, h16m(y), Wq.size(0), K, group_size,
                                        scale.size(1), swiglu ? 1 : 0, cur_stream(x)),
                 n);
}

void gemv_w4a16_rmsnorm_gate_up_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x,
                                     c10::optional<torch::Tensor> delta, torch::Tensor norm_weight, double eps,
                                     c10::optional<torch::Tensor> x_out, torch::Tensor gate_out, torch::Tensor up_out,
                                     int64_t K, int64_t group_size) {
    const char* n = "gemv_w4a16_rmsnorm_gate_up_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(x, torch::kFloat16, x, n, "x");
    need(norm_weight, torch::kFloat16, x, n, "norm_weight");
    need(gate_out, torch::kFloat16, x, n, "gate_out");
    need(up_out, torch::kFloat16, x, n, "up_out");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K && norm_weight.numel() == K, n,
                ": Wq / x / norm_weight shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0), n, ": scale must be [N, num_groups]");
    TORCH_CHECK(gate_out.numel() == Wq.size(0) / 2 && up_out.numel() == Wq.size(0) / 2, n,
                ": gate_out and up_out must have N/2 values");
    const uint16_t* dp = nullptr;
    uint16_t* xo = nullptr;
    if (delta.has_value()) {
        need(*delta, torch::kFloat16, x, n, "delta");
        TORCH_CHECK(delta->numel() == K, n, ": delta must be [K]");
        dp = h16(*delta);
    }
    if (x_out.has_value()) {
        need(*x_out, torch::kFloat16, x, n, "x_out");
        TORCH_CHECK(x_out->numel() == K, n, ": x_out must be [K]");
        xo = h16m(*x_out);
    }
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_rmsnorm_gate_up(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), dp,
                                                h16(norm_weight), static_cast<float>(eps), xo, nullptr,
                                                h16m(gate_out), h16m(up_out), Wq.size(0), K, group_size,
                                                scale.size(1), cur_stream(x)),
                 n);
}

void gemv_w4a16_rmsnorm_swiglu_gate_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor x,
                                         c10::optional<torch::Tensor> delta, torch::Tensor norm_weight, double eps,
                                         c10::optional<torch::Tensor> x_out, torch::Tensor gate_out, torch::Tensor y,
                                         int64_t K, int64_t group_size) {
    const char* n = "gemv_w4a16_rmsnorm_swiglu_gate_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(x, torch::kFloat16, x, n, "x");
    need(norm_weight, torch::kFloat16, x, n, "norm_weight");
    need(gate_out, torch::kFloat16, x, n, "gate_out");
    need(y, torch::kFloat16, x, n, "y");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K && norm_weight.numel() == K, n,
                ": Wq / x / norm_weight shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0), n, ": scale must be [N, num_groups]");
    TORCH_CHECK(gate_out.numel() == Wq.size(0) / 2 && y.numel() == Wq.size(0) / 2, n,
                ": gate_out and y must have N/2 values");
    const uint16_t* dp = nullptr;
    uint16_t* xo = nullptr;
    if (delta.has_value()) {
        need(*delta, torch::kFloat16, x, n, "delta");
        TORCH_CHECK(delta->numel() == K, n, ": delta must be [K]");
        dp = h16(*delta);
    }
    if (x_out.has_value()) {
        need(*x_out, torch::kFloat16, x, n, "x_out");
        TORCH_CHECK(x_out->numel() == K, n, ": x_out must be [K]");
        xo = h16m(*x_out);
    }
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_rmsnorm_swiglu_gate(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), h16(x), dp,
                                                    h16(norm_weight), static_cast<float>(eps), xo, nullptr,
                                                    h16m(gate_out), h16m(y), Wq.size(0), K, group_size,
                                                    scale.size(1), cur_stream(x)),
                 n);
}

void dip_select_down_ordered_into(torch::Tensor gate, torch::Tensor h, int64_t k, torch::Tensor Wt,
                                           torch::Tensor St, c10::optional<torch::Tensor> idx_out,
                                           c10::optional<torch::Tensor> count_out, torch::Tensor y, int64_t group_size,
                                           c10::optional<torch::Tensor> res, c10::optional<torch::Tensor> res_out) {
    const char* n = "dip_select_down_ordered_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(h, torch::kFloat16, gate, n, "h");
    need(Wt, torch::kUInt8, gate, n, "Wt");
    need(St, torch::kFloat32, gate, n, "St");
    need(y, torch::kFloat16, gate, n, "y");
    const int64_t I = gate.numel(), H = y.numel();
    TORCH_CHECK(h.numel() == I, n, ": gate and h must have the same length");
    TORCH_CHECK(k >= 1 && k <= I, n, ": k must be in [1, n]");
    TORCH_CHECK(Wt.dim() == 2 && Wt.size(0) == H && Wt.size(1) == I / 2, n, ": Wt must be [H, n/2]");
    TORCH_CHECK(St.dim() == 2 && St.size(1) == I, n, ": St must be [num_groups, n]");
    int32_t* ip = nullptr;
    int32_t* cp = nullptr;
    if (idx_out.has_value()) {
        need(*idx_out, torch::kInt32, gate, n, "idx_out");
        need_numel(*idx_out, k, n, "idx_out");
        ip = idx_out->data_ptr<int32_t>();
    }
    if (count_out.has_value()) {
        need(*count_out, torch::kInt32, gate, n, "count_out");
        need_numel(*count_out, 1, n, "count_out");
        cp = count_out->data_ptr<int32_t>();
    }
    TORCH_CHECK(res.has_value() == res_out.has_value(), n, ": res and res_out go together");
    const uint16_t* rp = nullptr;
    uint16_t* rop = nullptr;
    if (res.has_value()) {
        need(*res, torch::kFloat16, gate, n, "res");
        need(*res_out, torch::kFloat16, gate, n, "res_out");
        TORCH_CHECK(res->numel() == H && res_out->numel() == H, n, ": res and res_out must have H values");
        TORCH_CHECK(res_out->data_ptr() != y.data_ptr() && res->data_ptr() != y.data_ptr(), n,
                    ": res / res_out must not alias y");
        rp = h16(*res);
        rop = h16m(*res_out);
    }
    const at::DeviceGuard guard(gate.device());
    check_status(soi_dip_select_down_ordered(h16(gate), h16(h), I, k, Wt.data_ptr<uint8_t>(), St.data_ptr<float>(),
                                             ip, cp, h16m(y), rp, rop, H, group_size, St.size(0), cur_stream(gate)),
                 n);
}

int64_t dip_select_down_ordered_lds_bytes(int64_t H, int64_t num_channels, int64_t k) {
    return static_cast<int64_t>(soi_dip_select_down_ordered_lds_bytes(H, num_channels, k));
}

void dip_select_dense_down_into(torch::Tensor gate, torch::Tensor h, int64_t k, torch::Tensor Wt, torch::Tensor St,
                                c10::optional<torch::Tensor> idx_out, c10::optional<torch::Tensor> count_out,
                                torch::Tensor y, int64_t group_size, c10::optional<torch::Tensor> res,
                                c10::optional<torch::Tensor> res_out) {
    const char* n = "dip_select_dense_down_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(h, torch::kFloat16, gate, n, "h");
    need(Wt, torch::kUInt8, gate, n, "Wt");
    need(St, torch::kFloat32, gate, n, "St");
    need(y, torch::kFloat16, gate, n, "y");
    const int64_t I = gate.numel(), H = y.numel();
    TORCH_CHECK(h.numel() == I, n, ": gate and h must have the same length");
    TORCH_CHECK(k >= 1 && k <= I, n, ": k must be in [1, n]");
    TORCH_CHECK(Wt.dim() == 2 && Wt.size(0) == H && Wt.size(1) == I / 2, n, ": Wt must be [H, n/2]");
    TORCH_CHECK(St.dim() == 2 && St.size(1) == I, n, ": St must be [num_groups, n]");
    int32_t* ip = nullptr;
    int32_t* cp = nullptr;
    if (idx_out.has_value()) {
        need(*idx_out, torch::kInt32, gate, n, "idx_out");
        need_numel(*idx_out, k, n, "idx_out");
        ip = idx_out->data_ptr<int32_t>();
    }
    if (count_out.has_value()) {
        need(*count_out, torch::kInt32, gate, n, "count_out");
        need_numel(*count_out, 1, n, "count_out");
        cp = count_out->data_ptr<int32_t>();
    }
    TORCH_CHECK(res.has_value() == res_out.has_value(), n, ": res and res_out go together");
    const at::DeviceGuard guard(gate.device());
    if (res.has_value()) {
        need(*res, torch::kFloat16, gate, n, "res");
        need(*res_out, torch::kFloat16, gate, n, "res_out");
        TORCH_CHECK(res->numel() == H && res_out->numel() == H, n, ": res and res_out must have H values");
        TORCH_CHECK(res_out->data_ptr() != y.data_ptr() && res->data_ptr() != y.data_ptr(), n,
                    ": res / res_out must not alias y");
        check_status(soi_dip_select_dense_down_residual(h16(gate), h16(h), I, k, Wt.data_ptr<uint8_t>(),
                                                        St.data_ptr<float>(), ip, cp, h16m(y), h16(*res),
                                                        h16m(*res_out), H, group_size, St.size(0), cur_stream(gate)),
                     n);
        return;
    }
    check_status(soi_dip_select_dense_down(h16(gate), h16(h), I, k, Wt.data_ptr<uint8_t>(), St.data_ptr<float>(), ip,
                                           cp, h16m(y), H, group_size, St.size(0), cur_stream(gate)),
                 n);
}

void gemv_w4a16_indexed_accumulate_gated_into(torch::Tensor Wq_T, torch::Tensor scale_T, torch::Tensor idx,
                                              torch::Tensor gate, torch::Tensor up, torch::Tensor y, int64_t H,
                                              int64_t group_size, torch::Tensor workspace_buf) {
    const char* n = "gemv_w4a16_indexed_accumulate_gated_into";
    need(Wq_T, torch::kUInt8, gate, n, "Wq_T");
    need(scale_T, torch::kFloat32, gate, n, "scale_T");
    need(idx, torch::kInt32, gate, n, "idx");
    need(gate, torch::kFloat16, gate, n, "gate");
    need(up, torch::kFloat16, gate, n, "up");
    need(y, torch::kFloat16, gate, n, "y");
    need(workspace_buf, torch::kUInt8, gate, n, "workspace");
    TORCH_CHECK(Wq_T.dim() == 2 && Wq_T.size(1) == ((H + 7) / 8) * 4 && y.numel() == H, n, ": Wq_T / y mismatch");
    TORCH_CHECK(scale_T.dim() == 2 && scale_T.size(0) == Wq_T.size(0), n, ": scale_T shape mismatch");
    TORCH_CHECK(up.numel() == gate.numel(), n, ": gate and up must have the same length");
    const at::DeviceGuard guard(gate.device());
    check_status(soi_gemv_w4a16_indexed_accumulate_gated(
                     Wq_T.data_ptr<uint8_t>(), scale_T.data_ptr<float>(), Wq_T.size(0), idx.data_ptr<int32_t>(),
                     idx.numel(), h16(gate), h16(up), gate.numel(), h16m(y), H, group_size, scale_T.size(1),
                     workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), cur_stream(gate)),
                 n);
}

// DIP selection + gated sparse down in one launch: idx_out / count_out as
// topk_threshold_select_f16abs_into(gate, k), y as
// gemv_w4a16_indexed_accumulate_gated_into over those indices.
void dip_select_gated_down_into(torch::Tensor gate, torch::Tensor up, int64_t k, torch::Tensor Wq_T,
                                torch::Tensor scale_T, torch::Tensor idx_out, torch::Tensor count_out, torch::Tensor y,
                                int64_t H, int64_t group_size, torch::Tensor workspace_buf) {
    const char* n = "dip_select_gated_down_into";
    need(gate, torch::kFloat16, gate, n, "gate");
    need(up, torch::kFloat16, gate, n, "up");
    need(Wq_T, torch::kUInt8, gate, n, "Wq_T");
    need(scale_T, torch::kFloat32, gate, n, "scale_T");
    need(idx_out, torch::kInt32, gate, n, "idx_out");
    need(count_out, torch::kInt32, gate, n, "count_out");
    need(y, torch::kFloat16, gate, n, "y");
    need(workspace_buf, torch::kUInt8, gate, n, "workspace");
    TORCH_CHECK(k >= 1 && k <= gate.numel(), n, ": k must be in [1, n]");
    need_numel(idx_out, k, n, "idx_out");
    need_numel(count_out, 1, n, "count_out");
    TORCH_CHECK(up.numel() == gate.numel(), n, ": gate and up must have the same length");
    TORCH_CHECK(Wq_T.dim() == 2 && Wq_T.size(1) == ((H + 7) / 8) * 4 && y.numel() == H, n, ": Wq_T / y mismatch");
    TORCH_CHECK(scale_T.dim() == 2 && scale_T.size(0) == Wq_T.size(0), n, ": scale_T shape mismatch");
    const at::DeviceGuard guard(gate.device());
    check_status(soi_dip_select_gated_down(h16(gate), h16(up), gate.numel(), k, Wq_T.data_ptr<uint8_t>(),
                                           scale_T.data_ptr<float>(), Wq_T.size(0), idx_out.data_ptr<int32_t>(),
                                           count_out.data_ptr<int32_t>(), h16m(y), H, group_size, scale_T.size(1),
                                           workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(),
                                           cur_stream(gate)),
                 n);
}

void gemv_w4a16_indexed_silu_into(torch::Tensor Wq, torch::Tensor scale, torch::Tensor idx, torch::Tensor x,
                                  torch::Tensor gate, torch::Tensor h_sel, int64_t K, int64_t group_size) {
    const char* n = "gemv_w4a16_indexed_silu_into";
    need(Wq, torch::kUInt8, x, n, "Wq");
    need(scale, torch::kFloat32, x, n, "scale");
    need(idx, torch::kInt32, x, n, "idx");
    need(x, torch::kFloat16, x, n, "x");
    need(gate, torch::kFloat16, x, n, "gate");
    need(h_sel, torch::kFloat16, x, n, "h_sel");
    TORCH_CHECK(Wq.dim() == 2 && Wq.size(1) == ((K + 7) / 8) * 4 && x.numel() == K, n, ": Wq / x shape mismatch");
    TORCH_CHECK(scale.dim() == 2 && scale.size(0) == Wq.size(0) && h_sel.numel() == idx.numel(), n,
                ": scale / h_sel shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_w4a16_indexed_silu(Wq.data_ptr<uint8_t>(), scale.data_ptr<float>(), Wq.size(0),
                                             idx.data_ptr<int32_t>(), idx.numel(), h16(x), h16(gate), gate.numel(),
                                             h16m(h_sel), K, group_size, scale.size(1), cur_stream(x)),
                 n);
}

void gemv_dip_fused_up_silu_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor staging_Wq,
                                 torch::Tensor staging_scale, torch::Tensor desc, torch::Tensor sel, torch::Tensor x,
                                 torch::Tensor gate, torch::Tensor h_sel, int64_t K, int64_t group_size) {
    const char* n = "gemv_dip_fused_up_silu_into";
    check_dip_fused_common(cache_Wq, cache_scale, staging_Wq, staging_scale, desc, K, n);
    need(sel, torch::kInt32, desc, n, "sel");
    need(x, torch::kFloat16, desc, n, "x");
    need(gate, torch::kFloat16, desc, n, "gate");
    need(h_sel, torch::kFloat16, desc, n, "h_sel");
    TORCH_CHECK(x.numel() == K && h_sel.numel() == desc.numel() && sel.numel() >= desc.numel(), n, ": shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_dip_fused_up_silu(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(),
                                            std::min(cache_Wq.size(0), cache_scale.size(0)),
                                            staging_Wq.data_ptr<uint8_t>(), staging_scale.data_ptr<float>(),
                                            std::min(staging_Wq.size(0), staging_scale.size(0)),
                                            desc.data_ptr<int32_t>(), sel.data_ptr<int32_t>(), desc.numel(), h16(x),
                                            h16(gate), gate.numel(), h16m(h_sel), K, group_size, cache_scale.size(1),
                                            cur_stream(x)),
                 n);
}

namespace {

// Device-visible address of a weight matrix read in place: a CUDA tensor, or pinned host memory through its
// device mapping (the mapping of the allocation's base plus the view's offset, so views into one pinned arena
// work).
const uint8_t* readable_rows(const torch::Tensor& W, int64_t row_bytes, const torch::Tensor& dev, const char* name) {
    TORCH_CHECK(W.scalar_type() == torch::kUInt8 && W.dim() == 2 && W.is_contiguous() && W.size(1) == row_bytes,
                name, "(full_Wq): must be a contiguous 2D uint8 tensor [num_channels, ceil(row_dim/8)*4]");
    if (W.is_cuda()) {
        check_same_device(dev, W, name);
        return W.data_ptr<uint8_t>();
    }
    TORCH_CHECK(W.is_cpu() && W.is_pinned(), name, "(full_Wq): must be a CUDA tensor or pinned host memory");
    const auto* base = static_cast<const uint8_t*>(W.storage().data());
    const auto* at = static_cast<const uint8_t*>(W.data_ptr());
    void* dp = nullptr;
    const hipError_t e = hipHostGetDevicePointer(&dp, const_cast<uint8_t*>(base), 0);
    TORCH_CHECK(e == hipSuccess && dp != nullptr, name, ": hipHostGetDevicePointer failed: ", hipGetErrorString(e));
    return static_cast<const uint8_t*>(dp) + (at - base);
}

struct CachedArgs {
    const uint8_t* full;
    int64_t cache_rows;
    int64_t num_channels;
};

CachedArgs check_cached_common(const torch::Tensor& cache_Wq, const torch::Tensor& cache_scale,
                               const torch::Tensor& full_Wq, const torch::Tensor& full_scale,
                               const torch::Tensor& slot_of, const torch::Tensor& sel, int64_t row_dim,
                               const char* name) {
    const int64_t row_bytes = ((row_dim + 7) / 8) * 4;
    TORCH_CHECK(cache_Wq.is_cuda() && cache_Wq.scalar_type() == torch::kUInt8 && cache_Wq.dim() == 2 &&
                    cache_Wq.is_contiguous() && cache_Wq.size(1) == row_bytes,
                name, "(cache_Wq): must be a contiguous 2D uint8 CUDA tensor [C, ceil(row_dim/8)*4]");
    need(cache_scale, torch::kFloat32, sel, name, "cache_scale");
    need(full_scale, torch::kFloat32, sel, name, "full_scale");
    need(slot_of, torch::kInt32, sel, name, "slot_of");
    need(sel, torch::kInt32, sel, name, "sel");
    check_same_device(sel, cache_Wq, name);
    TORCH_CHECK(cache_scale.dim() == 2 && full_scale.dim() == 2 && cache_scale.size(1) == full_scale.size(1), name,
                ": cache_scale and full_scale must be 2D with the same num_groups");
    TORCH_CHECK(cache_scale.size(0) >= cache_Wq.size(0), name, ": cache_scale must have a row per cache_Wq row");
    TORCH_CHECK(full_scale.size(0) == full_Wq.size(0) && slot_of.numel() == full_Wq.size(0), name,
                ": full_Wq, full_scale and slot_of must have one entry per channel");
    return {readable_rows(full_Wq, row_bytes, sel, name), cache_Wq.size(0), full_Wq.size(0)};
}

}  // namespace

void gemv_dip_cached_up_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor full_Wq,
                             torch::Tensor full_scale, torch::Tensor slot_of, torch::Tensor sel, torch::Tensor x,
                             torch::Tensor y, int64_t K, int64_t group_size) {
    const char* n = "gemv_dip_cached_up_into";
    const CachedArgs a = check_cached_common(cache_Wq, cache_scale, full_Wq, full_scale, slot_of, sel, K, n);
    need(x, torch::kFloat16, sel, n, "x");
    need(y, torch::kFloat16, sel, n, "y");
    TORCH_CHECK(x.numel() == K && y.numel() == sel.numel(), n, ": shape mismatch");
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_dip_cached_up(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(), a.cache_rows,
                                        a.full, full_scale.data_ptr<float>(), a.num_channels,
                                        slot_of.data_ptr<int32_t>(), sel.data_ptr<int32_t>(), sel.numel(), h16(x),
                                        h16m(y), K, group_size, cache_scale.size(1), cur_stream(x)),
                 n);
}

void gemv_dip_cached_up_silu_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor full_Wq,
                                  torch::Tensor full_scale, torch::Tensor slot_of, torch::Tensor sel, torch::Tensor x,
                                  torch::Tensor gate, torch::Tensor h_sel, int64_t K, int64_t group_size,
                                  c10::optional<torch::Tensor> copy_src, c10::optional<torch::Tensor> copy_dst) {
    const char* n = "gemv_dip_cached_up_silu_into";
    const CachedArgs a = check_cached_common(cache_Wq, cache_scale, full_Wq, full_scale, slot_of, sel, K, n);
    need(x, torch::kFloat16, sel, n, "x");
    need(gate, torch::kFloat16, sel, n, "gate");
    need(h_sel, torch::kFloat16, sel, n, "h_sel");
    TORCH_CHECK(x.numel() == K && h_sel.numel() == sel.numel() && gate.numel() == a.num_channels, n,
                ": shape mismatch");
    TORCH_CHECK(copy_src.has_value() == copy_dst.has_value(), n, ": copy_src and copy_dst go together");
    const uint8_t* csrc = nullptr;
    uint8_t* cdst = nullptr;
    int64_t crow = 0;
    if (copy_src.has_value()) {
        const torch::Tensor& cd = *copy_dst;
        crow = copy_src->dim() == 2 ? copy_src->size(1) : -1;
        TORCH_CHECK(crow > 0 && copy_src->size(0) == a.num_channels, n,
                    "(copy_src): must be 2D with one row per channel");
        csrc = readable_rows(*copy_src, crow, sel, n);
        need(cd, torch::kUInt8, sel, n, "copy_dst");
        TORCH_CHECK(cd.dim() == 2 && cd.size(0) >= sel.numel() && cd.size(1) == crow, n,
                    "(copy_dst): must be [>= k, copy row bytes]");
        cdst = cd.data_ptr<uint8_t>();
    }
    const at::DeviceGuard guard(x.device());
    check_status(soi_gemv_dip_cached_up_silu(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(),
                                             a.cache_rows, a.full, full_scale.data_ptr<float>(), a.num_channels,
                                             slot_of.data_ptr<int32_t>(), sel.data_ptr<int32_t>(), sel.numel(),
                                             h16(x), h16(gate), h16m(h_sel), K, group_size, cache_scale.size(1), csrc,
                                             crow, cdst, cur_stream(x)),
                 n);
}

void gemv_dip_cached_down_into(torch::Tensor cache_Wq, torch::Tensor cache_scale, torch::Tensor full_Wq,
                               torch::Tensor full_scale, torch::Tensor slot_of, torch::Tensor sel, torch::Tensor h_sel,
                               torch::Tensor y, int64_t H, int64_t group_size, torch::Tensor workspace_buf,
                               c10::optional<torch::Tensor> staging_Wq) {
    const char* n = "gemv_dip_cached_down_into";
    const CachedArgs a = check_cached_common(cache_Wq, cache_scale, full_Wq, full_scale, slot_of, sel, H, n);
    need(h_sel, torch::kFloat16, sel, n, "h_sel");
    need(y, torch::kFloat16, sel, n, "y");
    need(workspace_buf, torch::kUInt8, sel, n, "workspace");
    TORCH_CHECK(h_sel.numel() == sel.numel() && y.numel() == H, n, ": h_sel / y shape mismatch");
    const uint8_t* stg_p = nullptr;
    if (staging_Wq.has_value()) {
        const torch::Tensor& st = *staging_Wq;
        need(st, torch::kUInt8, sel, n, "staging_Wq");
        TORCH_CHECK(st.dim() == 2 && st.size(0) >= sel.numel() && st.size(1) == full_Wq.size(1), n,
                    "(staging_Wq): must be [>= k, row bytes]");
        stg_p = st.data_ptr<uint8_t>();
    }
    const at::DeviceGuard guard(h_sel.device());
    check_status(soi_gemv_dip_cached_down(cache_Wq.data_ptr<uint8_t>(), cache_scale.data_ptr<float>(), a.cache_rows,
                                          a.full, full_scale.data_ptr<float>(), a.num_channels,
                                          slot_of.data_ptr<int32_t>(), sel.data_ptr<int32_t>(), sel.numel(),
                                          h16(h_sel), h16m(y), H, group_size, cache_scale.size(1), stg_p,
                                          workspace_buf.data_ptr<uint8_t>(), workspace_buf.numel(), cur_stream(h_sel)),
                 n);
}

// ---- grid barrier cost (measurement) ----
int64_t grid_barrier_bench_workspace_bytes(int64_t P) {
    return static_cast<int64_t>(soi_grid_barrier_bench_workspace_bytes(P));
}

int64_t grid_barrier_max_workgroups() {
    int64_t p = 0;
    check_status(soi_grid_barrier_max_workgroups(&p), "grid_barrier_max_workgroups");
    return p;
}

void grid_barrier_bench(bool fenced, int64_t P, int64_t rounds, torch::Tensor workspace) {
    const char* n = "grid_barrier_bench";
    TORCH_CHECK(workspace.is_cuda() && workspace.scalar_type() == torch::kUInt8 && workspace.is_contiguous(), n,
                ": workspace must be a contiguous uint8 CUDA tensor");
    const at::DeviceGuard guard(workspace.device());
    check_status(soi_grid_barrier_bench(fenced ? 1 : 0, P, rounds, workspace.data_ptr(),
                                        static_cast<size_t>(workspace.numel()), cur_stream(workspace)),
                 n);
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "soinfer MI355X (gfx950) quantized decode hot path";
    m.def("gemv_w8a16", &gemv_w8a16, "INT8 GEMV");
    m.def("gemv_w4a16_group", &gemv_w4a16_group, "INT4 group GEMV (scalar nibble dequant)");
    m.def("gemv_w4a16_group_lop3", &gemv_w4a16_group_lop3, "INT4 group GEMV (bitfield dequant)");
    m.def("gemv_w4a16_batched", &gemv_w4a16_batched, "P same-shape INT4 GEMVs in one launch");
    m.def("gemv_w4a16_grouped", &gemv_w4a16_grouped, "INT4 GEMVs of up to 8 shapes in one launch");
    m.def("gemv_w4a16_sparse_accumulate", &gemv_w4a16_sparse_accumulate, "sparse down-proj accumulate");
    m.def("build_dip_descriptors", &build_dip_descriptors, "hot-cache descriptors");
    m.def("gemv_dip_fused_up", &gemv_dip_fused_up, "descriptor-driven up GEMV");
    m.def("gemv_dip_fused_down", &gemv_dip_fused_down, "descriptor-driven down accumulate");
    m.def("gemv_w4a16_indexed", &gemv_w4a16_indexed, "index-driven up GEMV over resident weights");
    m.def("gemv_w4a16_indexed_accumulate", &gemv_w4a16_indexed_accumulate,
          "index-driven down accumulate over resident weights");
    m.def("gather_rows_device", &gather_rows_device, "device-resident row gather");
    m.def("decode_attention", &decode_attention, "batch-1 GQA decode attention");
    m.def("decode_attention_into", &decode_attention_into,
          "decode attention over a host length into a caller buffer, with a caller workspace");
    m.def("topk_threshold_select", &topk_threshold_select, "deterministic threshold top-k");
    m.def("gather_rows_staged", &gather_rows_staged, "pinned-host row gather, staged");
    m.def("gather_rows_naive", &gather_rows_naive, "pinned-host row gather, per row");
    m.def("rmsnorm", &rmsnorm, "RMSNorm over the last dim (reference rmsnorm)");
    m.def("gemv_fp16_v3", &gemv_fp16_v3, "fp16 GEMV (LM head)");
    m.def("swiglu_gate_up", &swiglu_gate_up, "h = silu(gate_W @ x) * (up_W @ x), one fused pass (fp16)");
    m.def("kv_cache_append", &kv_cache_append, "KV cache append at pos");
    m.def("rope_apply", &rope_apply, "RoPE in place (rotate-half)");
    m.def("rmsnorm_into", &rmsnorm_into, "RMSNorm into a caller buffer");
    m.def("residual_rmsnorm_", &residual_rmsnorm_, "x += delta (fp16), out = rmsnorm(x)");
    m.def("final_norm_advance", &final_norm_advance, "x += delta, out = rmsnorm(x), pos[0] += 1");
    m.def("qk_norm_rope_append", &qk_norm_rope_append, "q/k norm + RoPE + KV append at a device position");
    m.def("decode_attention_workspace_bytes", &decode_attention_workspace_bytes, "attention workspace size");
    m.def("decode_attention_at", &decode_attention_at, "decode attention over pos[0]+1 timesteps");
    m.def("decode_attention_step_workspace_bytes", &decode_attention_step_workspace_bytes,
          "workspace of decode_attention_step");
    m.def("decode_attention_step", &decode_attention_step,
          "q/k norm + RoPE + KV append + attention in one launch (device position)");
    m.def("decode_attention_step_deferred", &decode_attention_step_deferred,
          "decode_attention_step that leaves a split context's states for gemv_w4a16_attn_combine_into");
    m.def("gemv_w4a16_attn_combine_into", &gemv_w4a16_attn_combine_into,
          "INT4 GEMV of the attention output that combines a deferred step's split states on load",
          py::arg("Wq"), py::arg("scale"), py::arg("workspace"), py::arg("attn_out"), py::arg("pos"),
          py::arg("num_kv_heads"), py::arg("max_seq_len"), py::arg("y"), py::arg("group_size"),
          py::arg("res") = py::none(), py::arg("res_out") = py::none());
    m.def("gemv_w4a16_into", &gemv_w4a16_into, "INT4 GEMV into a caller buffer");
    m.def("gemv_w4a16_residual_into", &gemv_w4a16_residual_into,
          "INT4 GEMV into a caller buffer that also writes res_out = res + y (binary16)");
    m.def("gemv_w4a16_indexed_into", &gemv_w4a16_indexed_into, "index-driven INT4 GEMV into a caller buffer");
    m.def("gemv_w4a16_indexed_accumulate_into", &gemv_w4a16_indexed_accumulate_into,
          "index-driven sparse down accumulate into a caller buffer");
    m.def("sparse_accumulate_workspace_bytes", &sparse_accumulate_workspace_bytes, "sparse down workspace size");
    m.def("build_dip_descriptors_into", &build_dip_descriptors_into, "hot-cache descriptors into caller buffers");
    m.def("gemv_dip_fused_up_into", &gemv_dip_fused_up_into, "descriptor-driven up GEMV into a caller buffer");
    m.def("gemv_dip_fused_down_into", &gemv_dip_fused_down_into, "descriptor-driven down into a caller buffer");
    m.def("gemv_f16_into", &gemv_f16_into, "fp16 GEMV into a caller buffer");
    m.def("argmax_workspace_bytes", &argmax_workspace_bytes, "argmax workspace size");
    m.def("argmax_f16_into", &argmax_f16_into, "argmax of fp16 values (torch.argmax order)");
    m.def("silu_mul_into", &silu_mul_into, "fp16(silu(gate) * up)");
    m.def("silu_mul_indexed_into", &silu_mul_indexed_into, "fp16(silu(gate[idx]) * u_sel)");
    m.def("embed_lookup_into", &embed_lookup_into, "embedding row of a device token");
    m.def("advance_position", &advance_position, "pos[0] += delta on the device");
    m.def("gemv_w8a16_batched", &gemv_w8a16_batched, "P same-shape INT8 GEMVs in one launch (device pointer tables)");
    m.def("grid_barrier_bench_workspace_bytes", &grid_barrier_bench_workspace_bytes,
          "workspace bytes of grid_barrier_bench for P workgroups");
    m.def("grid_barrier_max_workgroups", &grid_barrier_max_workgroups,
          "most workgroups of the barrier measurement kernel resident at once");
    m.def("grid_barrier_bench", &grid_barrier_bench,
          "rounds of a grid-wide barrier among P co-resident workgroups, stamped (measurement)");
    m.def("topk_threshold_select_f16abs_into", &topk_threshold_select_f16abs_into,
          "threshold top-k over |fp16 gate| into caller buffers");
    m.def("host_device_pointer", &host_device_pointer, "device address of pinned host memory");
    m.def("gather_rows_device_counted", &gather_rows_device_counted, "device gather of count[0] rows");
    m.def("gemv_w4a16_rmsnorm_into", &gemv_w4a16_rmsnorm_into,
          "INT4 GEMV of rmsnorm(x + delta) (optionally with the interleaved SwiGLU epilogue)");
    m.def("gemv_w4a16_indexed_silu_into", &gemv_w4a16_indexed_silu_into, "DIP up GEMV with SiLU gating");
    m.def("gemv_w4a16_rmsnorm_gate_up_into", &gemv_w4a16_rmsnorm_gate_up_into,
          "INT4 GEMV of rmsnorm(x + delta) over interleaved gate|up rows, both halves written");
    m.def("gemv_w4a16_rmsnorm_swiglu_gate_into", &gemv_w4a16_rmsnorm_swiglu_gate_into,
          "INT4 GEMV of rmsnorm(x + delta) over interleaved gate|up rows: SwiGLU output and the gate half");
    m.def("dip_select_down_ordered_into", &dip_select_down_ordered_into,
          "DIP selection + sparse down over the transposed down^T values in one launch, in the sparse accumulate's "
          "order (equal to top-k + the sparse down of h[idx] bit for bit); optional residual add",
          py::arg("gate"), py::arg("h"), py::arg("k"), py::arg("Wt"), py::arg("St"), py::arg("idx_out"),
          py::arg("count_out"), py::arg("y"), py::arg("group_size"), py::arg("res") = py::none(),
          py::arg("res_out") = py::none());
    m.def("dip_select_down_ordered_lds_bytes", &dip_select_down_ordered_lds_bytes,
          "LDS bytes the ordered down needs for (H, n, k); 0 outside its limits");
    m.def("dip_select_dense_down_into", &dip_select_dense_down_into,
          "DIP selection + down projection over resident transposed down^T values in one launch (index outputs "
          "optional)",
          py::arg("gate"), py::arg("h"), py::arg("k"), py::arg("Wt"), py::arg("St"), py::arg("idx_out"),
          py::arg("count_out"), py::arg("y"), py::arg("group_size"), py::arg("res") = py::none(),
          py::arg("res_out") = py::none());
    m.def("gemv_w4a16_indexed_accumulate_gated_into", &gemv_w4a16_indexed_accumulate_gated_into,
          "sparse down over selected rows with the SiLU gating computed on the fly");
    m.def("dip_select_gated_down_into", &dip_select_gated_down_into,
          "DIP selection over |gate| and the gated sparse down in one launch");
    m.def("gemv_dip_fused_up_silu_into", &gemv_dip_fused_up_silu_into, "descriptor up GEMV with SiLU gating");
    m.def("gemv_dip_cached_up_into", &gemv_dip_cached_up_into, "hot-cache up GEMV, misses read in place");
    m.def("gemv_dip_cached_up_silu_into", &gemv_dip_cached_up_silu_into,
          "hot-cache up GEMV with SiLU gating, misses read in place (optionally copying the down^T miss rows)",
          py::arg("cache_Wq"), py::arg("cache_scale"), py::arg("full_Wq"), py::arg("full_scale"), py::arg("slot_of"),
          py::arg("sel"), py::arg("x"), py::arg("gate"), py::arg("h_sel"), py::arg("K"), py::arg("group_size"),
          py::arg("copy_src") = py::none(), py::arg("copy_dst") = py::none());
    m.def("gemv_dip_cached_down_into", &gemv_dip_cached_down_into,
          "hot-cache down accumulate, misses read in place or from staging", py::arg("cache_Wq"),
          py::arg("cache_scale"), py::arg("full_Wq"), py::arg("full_scale"), py::arg("slot_of"), py::arg("sel"),
          py::arg("h_sel"), py::arg("y"), py::arg("H"), py::arg("group_size"), py::arg("workspace"),
          py::arg("staging_Wq") = py::none());
    m.def("version", []() { return std::string(soi_version()); });
}
