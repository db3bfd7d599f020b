/*
 * soinfer_amd.h -- C ABI of the MI355X (gfx950) quantized decode hot path.
 *
 * Library: sparse-offload-infer_amd/soinfer/libsoinfer_hip.so
 *
 * Every entry point takes plain pointers and sizes, launches asynchronously
 * on `stream` (a hipStream_t passed as void*; NULL = the legacy default
 * stream) and returns a soi_status (0 = success). Device pointers must be HIP
 * device allocations on the current device. binary16 data crosses this
 * interface as uint16_t bit patterns. No entry point allocates device memory
 * except where it says so; scratch space is passed in by the caller as a
 * `workspace` argument sized by the matching *_workspace_bytes() query.
 *
 * Each declaration cites the reference interface it replaces (file:line in
 * the sparse-offload-infer repository). The soinfer._C extension
 * (csrc/bindings.cpp in this package) is a thin torch wrapper over exactly
 * these functions.
 */
#ifndef SOINFER_AMD_H_
#define SOINFER_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum soi_status {
    SOI_OK = 0,
    SOI_ERR_INVALID_ARGUMENT = 1, /* a size, shape or pointer precondition failed; nothing launched */
    SOI_ERR_WORKSPACE = 2,        /* workspace missing or smaller than *_workspace_bytes() */
    SOI_ERR_HIP = 3,              /* a HIP runtime call or kernel launch failed */
    SOI_ERR_UNSUPPORTED = 4       /* arguments valid but outside what this build implements */
} soi_status;

/* Human-readable text for a status code, and the detail of the last error
 * raised on the calling thread (which check failed, or the HIP error). */
const char* soi_status_string(int status);
const char* soi_last_error(void);

/* Library version string and the GPU architecture it was compiled for. */
const char* soi_version(void);

/* --------------------------------------------------------------------------
 * INT4 group-quantized GEMV, y[N] = dequant(Wq, scale) @ x.
 * Wq: uint8 [N, ceil(K/8)*4], AWQ nibble order (layout.h:19-45);
 * scale: fp32 [N, num_groups], num_groups == ceil(K/group_size);
 * group_size: positive multiple of 8; x: fp16 [K]; y: fp16 [N].
 *   soi_gemv_w4a16_group       replaces launch_gemv_w4a16_group
 *                              (csrc/kernels/gemv_w4a16_group.cu:64-70;
 *                               binding csrc/bindings.cpp:300-303)
 *   soi_gemv_w4a16_group_lop3  replaces launch_gemv_w4a16_group_lop3
 *                              (gemv_w4a16_group.cu:129-134; bindings.cpp:305-309)
 * The two differ only in how nibbles become binary16 (per-nibble extract vs.
 * three-input bitwise construction); both are exact, share one accumulation
 * order and return bit-identical results.
 * ------------------------------------------------------------------------ */
int soi_gemv_w4a16_group(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N,
                         int64_t K, int64_t group_size, int64_t num_groups, void* stream);
int soi_gemv_w4a16_group_lop3(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N,
                              int64_t K, int64_t group_size, int64_t num_groups, void* stream);

/* Batched form: P independent problems of one shape in ONE launch.
 * Wq_ptrs, scale_ptrs, x_ptrs, y_ptrs are DEVICE arrays of P device pointers
 * (problem p: Wq [N, ceil(K/8)*4], scale [N, num_groups], x [K], y [N]).
 * The pointer table is trusted (the caller validated the buffers); a problem
 * whose pointers are null is skipped, and one whose Wq or x is not 16-byte
 * aligned when K % 32 == 0 gets NaN in every row of y (the vector loads
 * need the alignment; soinfer.ops.GemvBatch / GemvGroup reject such problems
 * before launch). Each y is bit-identical to soi_gemv_w4a16_group_lop3 on that
 * problem. No reference counterpart: amortises the ~2.6 us per-launch latency
 * floor of MI355X over many GEMVs (the reference launches one per matrix). */
int soi_gemv_w4a16_batched(const uint8_t* const* Wq_ptrs, const float* const* scale_ptrs,
                           const uint16_t* const* x_ptrs, uint16_t* const* y_ptrs, int64_t P, int64_t N, int64_t K,
                           int64_t group_size, int64_t num_groups, void* stream);

/* Grouped form: independent problems of up to 8 shape classes in ONE launch.
 * The pointer tables (device arrays, as for the batched form) list the
 * problems class by class: class c has class_count[c] problems of shape
 * [class_N[c], class_K[c]] with ceil(class_K[c]/group_size) scale columns.
 * class_count, class_N, class_K are HOST arrays of num_classes (<= 8)
 * entries. Workgroups are laid out class by class in the given order (put
 * the longest rows first to keep the tail short). Null and misaligned
 * problems are treated as in the batched form. Each y is bit-identical to
 * soi_gemv_w4a16_group_lop3 on that problem. No reference counterpart: one
 * launch for a whole decoder's independent GEMVs. */
int soi_gemv_w4a16_grouped(const uint8_t* const* Wq_ptrs, const float* const* scale_ptrs,
                           const uint16_t* const* x_ptrs, uint16_t* const* y_ptrs, int64_t num_classes,
                           const int64_t* class_count, const int64_t* class_N, const int64_t* class_K,
                           int64_t group_size, void* stream);

/* --------------------------------------------------------------------------
 * INT8 GEMV, y[N] = sum_k scale[n*scale_row_stride + k/group_size] * Wq[n,k] * x[k].
 * Wq: int8 [N, K]; scale: fp32 [N or 1, num_groups]; scale_row_stride is 0
 * for a per-tensor [1, G] scale, else num_groups. group_size % 4 == 0 when
 * num_groups > 1. Replaces launch_gemv_w8a16 (csrc/kernels/gemv_w8a16.cu:64-70;
 * binding csrc/bindings.cpp:239-262).
 * ------------------------------------------------------------------------ */
int soi_gemv_w8a16(const int8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y, int64_t N, int64_t K,
                   int64_t group_size, int64_t num_groups, int64_t scale_row_stride, void* stream);
/* Batched INT8 form: P independent problems of one shape in ONE launch; Wq_ptrs, scale_ptrs, x_ptrs, y_ptrs
 * are DEVICE arrays of P device pointers (problem p: Wq [N, K], scale with the row stride above, x [K], y [N]).
 * Each y is bit-identical to soi_gemv_w8a16 on that problem (same tile for the shape). A problem with a null
 * pointer is skipped; with K % 16 == 0, one whose Wq or x is not 16-byte aligned gets NaN rows (soinfer.ops.
 * Int8Batch rejects such problems before launch). No reference counterpart: the per-launch latency floor
 * amortised over many GEMVs, as soi_gemv_w4a16_batched does for INT4. */
int soi_gemv_w8a16_batched(const int8_t* const* Wq_ptrs, const float* const* scale_ptrs, const uint16_t* const* x_ptrs,
                           uint16_t* const* y_ptrs, int64_t P, int64_t N, int64_t K, int64_t group_size,
                           int64_t num_groups, int64_t scale_row_stride, void* stream);

/* --------------------------------------------------------------------------
 * Deterministic threshold top-k over non-negative values (Dynamic Input
 * Pruning channel selection). Replaces launch_topk_threshold_select
 * (csrc/kernels/topk_select.cu:98-102; binding csrc/bindings.cpp:507-518).
 * Semantics are the reference's: tau = the 24-step fp32 bisection of
 * topk_select.cu:19-61 (lo=0, hi=max+1e-3f, mid=0.5f*(lo+hi),
 * lo=mid iff count(v>=mid)>=k), then out_indices = the first k indices in
 * ascending order with v >= tau, *out_count = the number written.
 * 1 <= k <= n. One workgroup; bit-identical output on every call.
 * ------------------------------------------------------------------------ */
int soi_topk_threshold_select(const float* abs_g, int64_t n, int64_t k, int32_t* out_indices, int32_t* out_count,
                              void* stream);

/* Same selection over |gate| of binary16 gate values: identical output to
 * soi_topk_threshold_select on gate.float().abs() (the conversion and the
 * absolute value are exact). Fuses the glue of generate.py:276-277 into the
 * load; no separate reference entry point. */
int soi_topk_threshold_select_f16abs(const uint16_t* gate, int64_t n, int64_t k, int32_t* out_indices,
                                     int32_t* out_count, void* stream);

/* --------------------------------------------------------------------------
 * Row gather from pinned host memory into device memory.
 * matrix: pinned host bytes [num_rows, row_nbytes]; indices: host int64 [k],
 * each in [0, num_rows) (checked; the reference leaves this unchecked).
 *   soi_gather_rows_staged: host memcpy of the k rows into pinned `staging`
 *     (>= k*row_nbytes), then ONE hipMemcpyAsync H2D into gpu_dst.
 *     Replaces launch_gather_rows_staged (csrc/kernels/gather_rows.cu:6-13;
 *     binding csrc/bindings.cpp:538-549).
 *   soi_gather_rows_naive: one hipMemcpyAsync per row.
 *     Replaces launch_gather_rows_naive (gather_rows.cu:15-21; bindings.cpp:551-559).
 * Both return once the copies are queued; gpu_dst is valid after `stream`
 * reaches them.
 * ------------------------------------------------------------------------ */
int soi_gather_rows_staged(const uint8_t* matrix, int64_t num_rows, int64_t row_nbytes, const int64_t* indices,
                           int64_t k, uint8_t* staging, uint8_t* gpu_dst, void* stream);
int soi_gather_rows_naive(const uint8_t* matrix, int64_t num_rows, int64_t row_nbytes, const int64_t* indices,
                          int64_t k, uint8_t* gpu_dst, void* stream);

/* Device-resident row gather (rows already in HBM): dst[j,:] = src[indices[j],:].
 * indices: device int32 [k]; an index outside [0, num_rows) writes a zero row.
 * No reference counterpart: on MI355X the weights stay resident in HBM. */
int soi_gather_rows_device(const uint8_t* src, int64_t num_rows, int64_t row_nbytes, const int32_t* indices,
                           int64_t k, uint8_t* dst, void* stream);

/* Same with the row count read from device memory: rows j < count[0] (<= max_k)
 * are copied. src may be a device mapping of pinned host memory
 * (hipHostGetDevicePointer), so the hot-cache miss rows can be fetched inside
 * a captured graph with no host round trip. No reference counterpart: the
 * reference copies misses with host-side gathers after a device-to-host sync
 * (generate.py:367-404). */
int soi_gather_rows_device_counted(const uint8_t* src, int64_t num_rows, int64_t row_nbytes, const int32_t* indices,
                                   const int32_t* count, int64_t max_k, uint8_t* dst, void* stream);

/* --------------------------------------------------------------------------
 * Sparse down projection over k gathered rows of down_proj^T:
 * y[H] = sum_{j<k} h_sel[j] * dequant(Wq_sel[j,:], scale_sel[j,:]).
 * Wq_sel: uint8 [k, ceil(H/8)*4]; scale_sel: fp32 [k, ceil(H/group_size)];
 * h_sel: fp16 [k]; y: fp16 [H]. One launch: (256-column slice) x (row chunk)
 * workgroups write fp32 partial rows; the last workgroup of each slice sums
 * them in a fixed order (deterministic, no float atomics). The workspace
 * (soi_sparse_accumulate_workspace_bytes) starts with per-slice arrival
 * counters that must be zero before the first call (e.g. zero-filled once);
 * every call leaves them zero, so one workspace serves repeated calls with
 * the same H and any k it was sized for, including graph replays (calls that
 * overlap on one workspace race). The same holds for the workspace of
 * soi_gemv_dip_fused_down and soi_gemv_w4a16_indexed_accumulate.
 * Replaces launch_gemv_w4a16_sparse_accumulate
 * (csrc/kernels/gemv_sparse_accumulate.cu:40-47; binding csrc/bindings.cpp:311-339).
 * ------------------------------------------------------------------------ */
size_t soi_sparse_accumulate_workspace_bytes(int64_t H, int64_t k);
int soi_gemv_w4a16_sparse_accumulate(const uint8_t* Wq_sel, const float* scale_sel, const uint16_t* h_sel,
                                     uint16_t* y, int64_t H, int64_t k, int64_t group_size, int64_t num_groups,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free form of soi_gemv_w4a16_sparse_accumulate: same arguments
 * without the workspace, same kernel, bit-identical y. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). It
 * calls no hipMalloc / hipFree: its workspace is a fixed device array of
 * soi_sparse_accumulate_noalloc_max_scratch_bytes() (2 MiB) that each GPU the
 * library runs on holds until the process ends, set up on the first call on a
 * device (address lookup, arrival counters cleared by a fill kernel on
 * `stream`). The array holds 16 KB of arrival counters and then the fp32
 * partial rows; a call that needs more than that (R x H x 4 bytes, R the
 * row-chunk count of the partition, about k / 192: H = 2048 takes k up to
 * about 48000, H = 5120 up to about 19000) returns SOI_ERR_INVALID_ARGUMENT without
 * launching. All calls on
 * one GPU share the array: calls that overlap on one GPU (different streams,
 * or graphs replayed concurrently) race; calls ordered on one stream do not. */
size_t soi_sparse_accumulate_noalloc_max_scratch_bytes(void);
int soi_gemv_w4a16_sparse_accumulate_noalloc(const uint8_t* Wq_sel, const float* scale_sel, const uint16_t* h_sel,
                                             uint16_t* y, int64_t H, int64_t k, int64_t group_size,
                                             int64_t num_groups, void* stream);

/* --------------------------------------------------------------------------
 * Hot-channel cache descriptors. desc[j] = slot_of[sel[j]] when >= 0 (cache
 * row), else (m | 0x80000000) where m numbers the misses in ascending j;
 * miss_channels[m] = sel[j]; *miss_count = number of misses. A channel
 * outside [0, num_channels) is treated as a miss. Replaces
 * launch_build_dip_descriptors (csrc/kernels/gemv_dip_fused.cu:35-42; binding
 * csrc/bindings.cpp:341-359), whose miss numbering is atomic-order dependent;
 * here it is deterministic.
 * ------------------------------------------------------------------------ */
int soi_build_dip_descriptors(const int32_t* sel, int64_t k, const int32_t* slot_of, int64_t num_channels,
                              int32_t* desc, int32_t* miss_channels, int32_t* miss_count, void* stream);

/* --------------------------------------------------------------------------
 * Descriptor-driven fused GEMVs: row j of the logical selected matrix comes
 * from cache row desc[j] (top bit clear) or staging row desc[j]&0x7fffffff
 * (top bit set). cache_rows / staging_rows bound the offsets; an offset out
 * of range yields NaN for that row instead of a read.
 *   soi_gemv_dip_fused_up: y[k] = rows @ x; bit-identical to
 *     soi_gemv_w4a16_group_lop3 on the same logical rows. Replaces
 *     launch_gemv_dip_fused_up (gemv_dip_fused.cu:104-111; bindings.cpp:388-408).
 *   soi_gemv_dip_fused_down: y[H] = sum_j h_sel[j] * row_j; bit-identical to
 *     soi_gemv_w4a16_sparse_accumulate on the same logical rows. Replaces
 *     launch_gemv_dip_fused_down (gemv_dip_fused.cu:156-164; bindings.cpp:410-432).
 * ------------------------------------------------------------------------ */
int soi_gemv_dip_fused_up(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                          const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                          const int32_t* desc, int64_t k, const uint16_t* x, uint16_t* y, int64_t K,
                          int64_t group_size, int64_t num_groups, void* stream);
int soi_gemv_dip_fused_down(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                            const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                            const int32_t* desc, int64_t k, const uint16_t* h_sel, uint16_t* y, int64_t H,
                            int64_t group_size, int64_t num_groups, void* workspace, size_t workspace_bytes,
                            void* stream);

/* --------------------------------------------------------------------------
 * Index-driven sparse GEMVs over weights resident in HBM (no gather): row j
 * is row idx[j] of the full matrix. Bit-identical to gathering the rows
 * first and calling soi_gemv_w4a16_group_lop3 / soi_gemv_w4a16_sparse_accumulate.
 * An index outside [0, num_rows) yields NaN for that row. No reference
 * counterpart (the reference must offload); used by the resident DIP layer.
 * ------------------------------------------------------------------------ */
int soi_gemv_w4a16_indexed(const uint8_t* Wq, const float* scale, int64_t num_rows, const int32_t* idx, int64_t k,
                           const uint16_t* x, uint16_t* y, int64_t K, int64_t group_size, int64_t num_groups,
                           void* stream);
int soi_gemv_w4a16_indexed_accumulate(const uint8_t* Wq_T, const float* scale_T, int64_t num_rows,
                                      const int32_t* idx, int64_t k, const uint16_t* h_sel, uint16_t* y, int64_t H,
                                      int64_t group_size, int64_t num_groups, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* --------------------------------------------------------------------------
 * Batch-1 GQA decode attention:
 * out[h,:] = softmax_t(q[h,:].k[kvh,t,:] / sqrt(head_dim)) @ v[kvh,t,:],
 * kvh = h / (NQ/NKV), t < cur_len. q: fp16 [NQ, hd]; k_cache, v_cache:
 * fp16 [NKV, max_seq, hd]; out: fp16 [NQ, hd]; 1 <= cur_len <= max_seq,
 * NQ % NKV == 0. `scale` is the score multiplier (the binding passes
 * 1/sqrt(hd)). One launch: a short context is one workgroup per KV head; a
 * long one is split over the KV sequence and the last split of each KV head
 * combines the split states in a fixed order. The workspace
 * (soi_decode_attention_workspace_bytes, 16-byte aligned) holds the split
 * states and ends in arrival counters that must be zero before the first
 * call (e.g. zero-filled once); every call leaves them zero, so a workspace
 * is reused across calls and graph replays (calls that overlap on one
 * workspace race). Replaces launch_decode_attention
 * (csrc/kernels/decode_attention.cu:57-63; binding csrc/bindings.cpp:468-488).
 * ------------------------------------------------------------------------ */
size_t soi_decode_attention_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t cur_len);
int soi_decode_attention(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                         int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim, int64_t cur_len, float scale,
                         void* workspace, size_t workspace_bytes, void* stream);

/* Device-position form of soi_decode_attention: cur_len = pos[0] + 1 read on
 * the device (clamped to [1, max_seq]), so one captured graph serves every
 * position. The grid covers cur_len = max_seq and the split plan of the
 * current length is made on the device (the host form's formula: identical
 * outputs); workgroups past it exit at once. Workspace (same rules):
 * soi_decode_attention_workspace_bytes(NQ, NKV, head_dim, max_seq). Used by
 * the decode engine. */
int soi_decode_attention_at(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                            int64_t NQ, int64_t NKV, int64_t max_seq, int64_t head_dim, const int32_t* pos,
                            float scale, void* workspace, size_t workspace_bytes, void* stream);

/* One launch per decoder layer for the attention block of the decode engine
 * (no reference entry point; fuses generate.py:160-169): for the fused
 * projection qkv [q (NQ*hd) | k (NKV*hd) | v (NKV*hd)] at position p = pos[0],
 * q/k RMSNorm (q_norm / k_norm) + RoPE (tables cos/sin [max_seq, hd/2]), the
 * KV append of k, v at p, and attention of the NQ query heads over p + 1
 * timesteps into out [NQ, hd]. Same binary16 rounding points as
 * soi_qk_norm_rope_append followed by soi_decode_attention_at, and the same
 * attention kernel and split plan, so the outputs are identical. Workspace:
 * soi_decode_attention_step_workspace_bytes, under the rules above. Returns
 * SOI_ERR_UNSUPPORTED for head sizes outside the fast path (head_dim a
 * power of two in [8, 256], at most 8 query heads per KV head). */
size_t soi_decode_attention_step_workspace_bytes(int64_t NQ, int64_t NKV, int64_t head_dim, int64_t max_seq);
int soi_decode_attention_step(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                              const float* cos_table, const float* sin_table, const int32_t* pos, uint16_t* k_cache,
                              uint16_t* v_cache, uint16_t* out, int64_t NQ, int64_t NKV, int64_t max_seq,
                              int64_t head_dim, float eps, float scale, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Deferred combine. soi_decode_attention_step_deferred: soi_decode_attention_step
 * (same arguments, same KV append) except that a context long enough to split
 * across workgroups (more than 8 passes of the kernel: 256 timesteps at
 * head_dim 128) leaves `out` unwritten and its per-split softmax states in the
 * workspace; a shorter one writes `out` itself as before.
 * soi_gemv_w4a16_attn_combine: y[N] = the INT4 GEMV (soi_gemv_w4a16_group_lop3
 * arithmetic) of that step's attention output x [NQ * head_dim], with x
 * finished on load: `out` when the context did not split, else the split
 * states combined with the step's own combine arithmetic. y is bit-identical
 * to soi_decode_attention_step followed by soi_gemv_w4a16_group_lop3 on its
 * out. The workspace, pos, NQ, NKV, head_dim and max_seq are the step's;
 * attn_out is its `out`. With res and res_out (both or neither) it also writes
 * res_out = res + y (one binary16 add, as soi_gemv_w4a16_residual). Limits:
 * the step's fast form (head_dim a power of two in [8, 256], at most 8 query
 * heads per KV head), NQ * head_dim a multiple of 32 and at most 2048,
 * group_size a multiple of 8, Wq / attn_out / workspace 16-byte aligned.
 * No reference counterpart as single entry points: the pair replaces
 * decode_attention (csrc/kernels/decode_attention.cu:17-63) followed by the
 * o_proj GEMV (python/soinfer/runtime/generate.py:169-171), moving the split
 * combine out of the attention launch into the GEMV's load phase, where it
 * overlaps the weight loads instead of adding a cross-workgroup step. */
int soi_decode_attention_step_deferred(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                                       const float* cos_table, const float* sin_table, const int32_t* pos,
                                       uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, int64_t NQ, int64_t NKV,
                                       int64_t max_seq, int64_t head_dim, float eps, float scale, void* workspace,
                                       size_t workspace_bytes, void* stream);
int soi_gemv_w4a16_attn_combine(const uint8_t* Wq, const float* scale, const void* workspace,
                                size_t workspace_bytes, const uint16_t* attn_out, const int32_t* pos, int64_t NQ,
                                int64_t NKV, int64_t head_dim, int64_t max_seq, uint16_t* y, const uint16_t* res,
                                uint16_t* res_out, int64_t N, int64_t group_size, int64_t num_groups, void* stream);

/* --------------------------------------------------------------------------
 * Decoder-step glue (binary16 in/out, fp32 math).
 *
 * soi_rmsnorm: out[r,:] = x[r,:] * rsqrt(mean(x[r,:]^2) + eps) * weight, one
 *   row of `hidden` per r. Replaces launch_rmsnorm (csrc/kernels/rmsnorm.cu:
 *   46-50; binding csrc/bindings.cpp:141-150); qk_norm is the same op with
 *   rows = heads, hidden = head_dim (python/soinfer/ops.py qk_norm).
 * soi_residual_rmsnorm: x[r,:] <- x[r,:] + delta[r,:] (binary16 add, in place),
 *   then out = rmsnorm(x). Fuses `h2 = residual + o` and the next rmsnorm of
 *   generate.py:171-175; identical to the two separate ops.
 * soi_rope_apply: RoPE in place on x [num_heads, head_dim], rotate-half
 *   convention, cos/sin fp32 [head_dim/2]. Replaces launch_rope_apply
 *   (rope.cu:21-25; bindings.cpp:490-505).
 * soi_kv_cache_append: k/v_new [NKV, hd] into k/v_cache [NKV, max_seq, hd] at
 *   pos. Replaces launch_kv_cache_append (kv_cache.cu:22-27; bindings.cpp:450-466).
 * soi_gemv_f16: y[N] = W[N,K] x[K] with fp16 W (the LM head). Replaces
 *   launch_gemv_fp16_v3 (gemv_fp16.cu:89-93; bindings.cpp:201-208).
 * soi_swiglu_gate_up: h[I] = fp16(silu(g) * u), g = gate_W[I,H] x and
 *   u = up_W[I,H] x summed in fp32 over fp16 products, silu(t) = t/(1+exp(-t)),
 *   one pass over x for both matrices. Replaces launch_swiglu_gate_up
 *   (swiglu_fused.cu:15-56; bindings.cpp:434-448).
 * soi_argmax_f16: index of the largest of n binary16 values (NaN above every
 *   number, ties to the lowest index: torch.argmax, generate.py:446). Writes
 *   out_index[0]; if log/log_len are given, also log[log_len[0]] = index and
 *   log_len[0] += 1 while log_len[0] < log_cap. Workspace:
 *   soi_argmax_workspace_bytes(n).
 * soi_silu_mul: out = fp16(silu(fp32 gate) * fp32 up), silu(t) = t/(1+exp(-t))
 *   (generate.py:178). soi_silu_mul_indexed: out[j] = fp16(silu(gate[idx[j]]) *
 *   u_sel[j]) (generate.py:304-305); an index outside [0, n_gate) gives NaN.
 * soi_embed_lookup: out = table[token[0], :] with the token read on the device
 *   (a token outside [0, rows) gives zeros) (generate.py:440).
 * soi_qk_norm_rope_append: the engine form of q/k norm + RoPE + KV append of
 *   one layer (generate.py:160-168) for the fused projection qkv
 *   [q (NQ*hd) | k (NKV*hd) | v (NKV*hd)], at position pos[0] read on the
 *   device, with RoPE tables cos/sin fp32 [max_seq, hd/2]. Writes q_out
 *   [NQ, hd] and the caches; a position outside [0, max_seq) writes nothing.
 * soi_advance_position: pos[0] += delta on the device.
 * ------------------------------------------------------------------------ */
int soi_rmsnorm(const uint16_t* x, const uint16_t* weight, uint16_t* out, int64_t rows, int64_t hidden, float eps,
                void* stream);
int soi_residual_rmsnorm(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* out, int64_t rows,
                         int64_t hidden, float eps, void* stream);
/* Engine form of the last op of a decode step: soi_residual_rmsnorm of one row
 * (x += delta, out = rmsnorm(x), the final norm of generate.py:444) that also
 * advances the device position: pos[0] += 1. */
int soi_final_norm_advance(uint16_t* x, const uint16_t* delta, const uint16_t* weight, uint16_t* out, int64_t hidden,
                           float eps, int32_t* pos, void* stream);
int soi_rope_apply(uint16_t* x, const float* cos_vals, const float* sin_vals, int64_t num_heads, int64_t head_dim,
                   void* stream);
int soi_kv_cache_append(const uint16_t* k_new, const uint16_t* v_new, uint16_t* k_cache, uint16_t* v_cache,
                        int64_t num_kv_heads, int64_t max_seq, int64_t head_dim, int64_t pos, void* stream);
int soi_gemv_f16(const uint16_t* W, const uint16_t* x, uint16_t* y, int64_t N, int64_t K, void* stream);
int soi_swiglu_gate_up(const uint16_t* gate_W, const uint16_t* up_W, const uint16_t* x, uint16_t* h, int64_t I,
                       int64_t H, void* stream);
size_t soi_argmax_workspace_bytes(int64_t n);
int soi_argmax_f16(const uint16_t* x, int64_t n, int32_t* out_index, int32_t* log, int32_t* log_len, int64_t log_cap,
                   void* workspace, size_t workspace_bytes, void* stream);
int soi_silu_mul(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t n, void* stream);
int soi_silu_mul_indexed(const uint16_t* gate, int64_t n_gate, const int32_t* idx, const uint16_t* u_sel,
                         uint16_t* out, int64_t k, void* stream);
int soi_embed_lookup(const uint16_t* table, int64_t rows, int64_t hidden, const int32_t* token, uint16_t* out,
                     void* stream);
int soi_qk_norm_rope_append(const uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                            const float* cos_table, const float* sin_table, const int32_t* pos, uint16_t* q_out,
                            uint16_t* k_cache, uint16_t* v_cache, int64_t num_q_heads, int64_t num_kv_heads,
                            int64_t max_seq, int64_t head_dim, float eps, void* stream);
int soi_advance_position(int32_t* pos, int32_t delta, void* stream);

/* --------------------------------------------------------------------------
 * Fused decode-step GEMVs (no reference entry points: each fuses glue of
 * generate.py into the INT4 GEMV so a decoder layer needs fewer launches;
 * every rounding point of the separate ops is kept).
 *
 * soi_gemv_w4a16_rmsnorm: y = W . rmsnorm(x + delta, norm_weight) with the
 *   residual add (binary16) and RMSNorm done while loading x. delta may be
 *   NULL (no add). When given, x_out receives x + delta and h_out the
 *   normalised vector (both fp16 [K], must not alias x or delta). K % 32 == 0;
 *   Wq, x, delta, norm_weight, x_out, h_out 16-byte aligned. With swiglu != 0
 *   the rows of W are interleaved by 8-row tiles (gate rows 4t..4t+3, then up
 *   rows 4t..4t+3) and y[i] = fp16(silu(fp16(gate_i)) * fp16(up_i)) for
 *   i < N/2 (N % 8 == 0): the dense SwiGLU of generate.py:176-178 in one pass.
 * soi_gemv_w4a16_indexed_silu: h_sel[j] = fp16(silu(gate[idx[j]]) *
 *   fp16(sum_k W[idx[j],k] x[k])): the DIP up projection with the SiLU gating
 *   of generate.py:301-305 in its epilogue (NaN for an index outside
 *   [0, min(num_rows, n_gate))).
 * soi_gemv_dip_fused_up_silu: the same epilogue on soi_gemv_dip_fused_up
 *   (descriptor rows; sel = the selected channel indices).
 * soi_gemv_w4a16_rmsnorm_gate_up: soi_gemv_w4a16_rmsnorm over the interleaved
 *   gate|up rows (8-row tiles as above, N % 8 == 0) writing both halves
 *   unfused: gate_out[i] = fp16(gate_i), up_out[i] = fp16(up_i), i < N/2,
 *   each equal to the plain GEMV of that row.
 * soi_gemv_w4a16_indexed_accumulate_gated: soi_gemv_w4a16_indexed_accumulate
 *   with h_sel computed on the fly: h_sel[j] = fp16(silu(gate[c]) * up[c]),
 *   c = idx[j] (NaN for c outside [0, num_channels)), the rounding of
 *   soi_gemv_w4a16_indexed_silu, so the two-step and the fused forms give
 *   identical y. Workspace rules of soi_gemv_w4a16_sparse_accumulate.
 *   Together they are a DIP MLP schedule for resident weights: gate and up of
 *   every channel in one launch, top-k on gate, then the gated sparse down
 *   (one launch fewer than the indexed up GEMV; up is read for all channels).
 * ------------------------------------------------------------------------ */
int soi_gemv_w4a16_rmsnorm(const uint8_t* Wq, const float* scale, const uint16_t* x, const uint16_t* delta,
                           const uint16_t* norm_weight, float eps, uint16_t* x_out, uint16_t* h_out, uint16_t* y,
                           int64_t N, int64_t K, int64_t group_size, int64_t num_groups, int swiglu, void* stream);
int soi_gemv_w4a16_indexed_silu(const uint8_t* Wq, const float* scale, int64_t num_rows, const int32_t* idx,
                                int64_t k, const uint16_t* x, const uint16_t* gate, int64_t n_gate, uint16_t* h_sel,
                                int64_t K, int64_t group_size, int64_t num_groups, void* stream);
int soi_gemv_dip_fused_up_silu(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                               const uint8_t* staging_Wq, const float* staging_scale, int64_t staging_rows,
                               const int32_t* desc, const int32_t* sel, int64_t k, const uint16_t* x,
                               const uint16_t* gate, int64_t n_gate, uint16_t* h_sel, int64_t K, int64_t group_size,
                               int64_t num_groups, void* stream);
int soi_gemv_w4a16_rmsnorm_gate_up(const uint8_t* Wq, const float* scale, const uint16_t* x, const uint16_t* delta,
                                   const uint16_t* norm_weight, float eps, uint16_t* x_out, uint16_t* h_out,
                                   uint16_t* gate_out, uint16_t* up_out, int64_t N, int64_t K, int64_t group_size,
                                   int64_t num_groups, void* stream);
/* soi_gemv_w4a16_rmsnorm_swiglu_gate: soi_gemv_w4a16_rmsnorm with swiglu = 1
 *   (y[N/2] = fp16(silu(gate) * up) over the 8-row interleaved gate|up rows)
 *   that also writes gate_out[N/2] = fp16(gate), the value
 *   soi_gemv_w4a16_rmsnorm_gate_up writes: the input of
 *   soi_dip_select_dense_down. */
int soi_gemv_w4a16_rmsnorm_swiglu_gate(const uint8_t* Wq, const float* scale, const uint16_t* x,
                                       const uint16_t* delta, const uint16_t* norm_weight, float eps, uint16_t* x_out,
                                       uint16_t* h_out, uint16_t* gate_out, uint16_t* y, int64_t N, int64_t K,
                                       int64_t group_size, int64_t num_groups, void* stream);
int soi_gemv_w4a16_indexed_accumulate_gated(const uint8_t* Wq_T, const float* scale_T, int64_t num_rows,
                                            const int32_t* idx, int64_t k, const uint16_t* gate, const uint16_t* up,
                                            int64_t num_channels, uint16_t* y, int64_t H, int64_t group_size,
                                            int64_t num_groups, void* workspace, size_t workspace_bytes,
                                            void* stream);
/* soi_dip_select_gated_down: the DIP selection and the gated sparse down of
 *   one MLP in ONE launch. Equals soi_topk_threshold_select_f16abs(gate, n =
 *   num_channels, k) -> (out_indices, out_count) followed by
 *   soi_gemv_w4a16_indexed_accumulate_gated over those indices, bit for bit
 *   (indices, count and y); a selection of fewer than k channels (NaN gates)
 *   sums over the selected ones only. Fuses the reference's
 *   topk_threshold_select (csrc/bindings.cpp:507-518), the SiLU gating of
 *   python/soinfer/runtime/generate.py:304-305 and gemv_w4a16_sparse_accumulate
 *   (csrc/bindings.cpp:311-339). Every workgroup of the down grid computes the
 *   selection itself and keeps its own rows' channels in LDS. Requires
 *   num_rows >= num_channels and 1 <= k <= num_channels; workspace rules of
 *   soi_gemv_w4a16_sparse_accumulate. Sizes past the fused kernel's limits
 *   (num_channels > 8192, a row chunk over 1024 rows, or rows / scales that
 *   the vector path cannot read) run the two kernels instead, same results. */
int soi_dip_select_gated_down(const uint16_t* gate, const uint16_t* up, int64_t num_channels, int64_t k,
                              const uint8_t* Wq_T, const float* scale_T, int64_t num_rows, int32_t* out_indices,
                              int32_t* out_count, uint16_t* y, int64_t H, int64_t group_size, int64_t num_groups,
                              void* workspace, size_t workspace_bytes, void* stream);
/* soi_dip_select_down_ordered: the DIP selection and the sparse down of one
 *   MLP in ONE launch from the binary16 gates and h = fp16(silu(gate) * up) of
 *   every channel (as soi_gemv_w4a16_rmsnorm_swiglu_gate writes them), over
 *   the transposed copy of down_proj^T that soi_dip_select_dense_down reads
 *   (Wt [H, n/2], St [H/gs, n]). Indices, count and y equal
 *   soi_topk_threshold_select_f16abs followed by
 *   soi_gemv_w4a16_indexed_accumulate over h_sel = h[indices] (so also
 *   soi_dip_select_gated_down on the same gate and up) bit for bit, with no
 *   workspace and no cross-workgroup step: every output column replays the
 *   sparse accumulate's partition and summation order (its row chunks of the
 *   plan for (H, k), the 32 fma chains of each chunk, their sums in order).
 *   Replaces the reference's topk_threshold_select (csrc/bindings.cpp:507-518)
 *   and gemv_w4a16_sparse_accumulate (csrc/bindings.cpp:311-339) of one MLP.
 *   Optional res / res_out (res_out null, or both given): res_out[H] = res +
 *   y, one binary16 add. out_indices / out_count may be null. Requires
 *   num_channels a multiple of 32 up to 24576, group_size a multiple of 8,
 *   gate / h 8-byte and Wt / St 16-byte aligned, and a shape inside the
 *   kernel's limits: soi_dip_select_down_ordered_lds_bytes(H, num_channels,
 *   k) > 0 (the plan has at most 64 row chunks and the tables fit in 144 KB
 *   of LDS; H = 2048 with n = 6144 fits for every k). */
size_t soi_dip_select_down_ordered_lds_bytes(int64_t H, int64_t num_channels, int64_t k);
int soi_dip_select_down_ordered(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                                const uint8_t* Wt, const float* St, int32_t* out_indices, int32_t* out_count,
                                uint16_t* y, const uint16_t* res, uint16_t* res_out, int64_t H, int64_t group_size,
                                int64_t num_groups, void* stream);

/* --------------------------------------------------------------------------
 * Hot-cache GEMVs that read the misses in place (cache-aware DIP without a
 * staging copy). Row j of the logical selected matrix is channel ch = sel[j]:
 * cache row slot_of[ch] when slot_of[ch] >= 0 (cache_Wq / cache_scale, as
 * built by HotCache), else row ch of the full matrix full_Wq [num_channels,
 * row_bytes] with scales full_scale [num_channels, G]. full_Wq is normally
 * the device address of pinned host memory (hipHostGetDevicePointer), so a
 * miss row crosses PCIe once, inside the GEMV that consumes it, while the
 * hits stream from HBM in the same launch; no descriptors, gathers or
 * staging buffers. slot_of: int32 [num_channels]. A channel outside
 * [0, num_channels) or a slot outside [0, cache_rows) yields NaN for that row.
 * The row bytes and arithmetic are those of the descriptor forms, so results
 * equal soi_build_dip_descriptors + gathers + soi_gemv_dip_fused_up /
 * _up_silu / _down bit for bit, and equal plain DIP over resident weights.
 * No reference counterpart: replaces the staged miss path of
 * run_decoder_layer_cached_dip (generate.py:367-404: descriptors, a host sync,
 * gather_rows_staged of the misses, then gemv_dip_fused_up / _down).
 *   soi_gemv_dip_cached_up: y[k] = rows @ x.
 *   soi_gemv_dip_cached_up_silu: h_sel[j] = fp16(silu(gate[sel[j]]) * fp16(row_j . x)).
 *     With copy_src / copy_dst (both or neither): the same waves also copy,
 *     for every miss j, row sel[j] of copy_src ([num_channels,
 *     copy_row_bytes], e.g. the pinned down^T matrix) to row j of copy_dst
 *     (device staging [k, copy_row_bytes]); copy_row_bytes a multiple of 16,
 *     at most 4096, both 16-byte aligned. The copy's loads are issued before
 *     the GEMV's, so the down^T misses cross PCIe as whole-row reads while
 *     the up rows stream; rows of hits are not written.
 *   soi_gemv_dip_cached_down: y[H] = sum_j h_sel[j] * row_j (rows of down^T);
 *     a miss reads row j of staging_Wq when it is given (as filled by the
 *     copy above), else row sel[j] of full_Wq in place; scales always from
 *     full_scale. Workspace rules of soi_gemv_w4a16_sparse_accumulate.
 * ------------------------------------------------------------------------ */
int soi_gemv_dip_cached_up(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                           const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                           const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* x, uint16_t* y,
                           int64_t K, int64_t group_size, int64_t num_groups, void* stream);
int soi_gemv_dip_cached_up_silu(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                                const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                                const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* x,
                                const uint16_t* gate, uint16_t* h_sel, int64_t K, int64_t group_size,
                                int64_t num_groups, const uint8_t* copy_src, int64_t copy_row_bytes,
                                uint8_t* copy_dst, void* stream);
int soi_gemv_dip_cached_down(const uint8_t* cache_Wq, const float* cache_scale, int64_t cache_rows,
                             const uint8_t* full_Wq, const float* full_scale, int64_t num_channels,
                             const int32_t* slot_of, const int32_t* sel, int64_t k, const uint16_t* h_sel,
                             uint16_t* y, int64_t H, int64_t group_size, int64_t num_groups,
                             const uint8_t* staging_Wq, void* workspace, size_t workspace_bytes, void* stream);

/* --------------------------------------------------------------------------
 * soi_dip_select_dense_down: the DIP selection and down projection of one
 * MLP over RESIDENT weights in one launch with no cross-workgroup step. It
 * computes the reference's sparse accumulate (python/soinfer/runtime/
 * generate.py:304-308 over gemv_w4a16_sparse_accumulate, csrc/bindings.cpp:
 * 311-339) after its topk_threshold_select (csrc/bindings.cpp:507-518):
 * y[col] = sum over the selected channels c of h[c] * s_T[c, col/gs] *
 * q_T[c, col], the selection being that of soi_topk_threshold_select_f16abs
 * (gate, num_channels, k). Inputs: gate[n] and h[n] = fp16(silu(gate) * up)
 * of every channel (as soi_gemv_w4a16_rmsnorm_swiglu_gate writes them), and
 * down_proj^T's quantized values stored TRANSPOSED: Wt [H, n/2] (row col holds
 * q_T[0..n-1, col] packed like any INT4 row) and St [num_groups, n] (St[g, c]
 * = s_T[c, g]). Every workgroup computes the selection itself while its rows
 * load, then a GEMV of its 8 output columns with the coefficients h * s
 * (fp32, carried as exact binary16 hi + lo pairs under a power-of-two scale).
 * Reads all n channels' rows (the bytes of a dense down projection), needs
 * no workspace; sums the reference's terms in another order (tolerance of
 * the sparse accumulate). out_indices[k] / out_count, when not null, receive
 * the selection exactly as the top-k function writes it (computed after y;
 * leave them null when not needed). n a multiple of 32 in [32, 24576],
 * 1 <= k <= n, group_size a multiple of 8, num_groups = ceil(H / group_size),
 * Wt and St 16-byte aligned, gate and h 8-byte aligned. No reference
 * counterpart as a single entry point: it replaces the pair cited above.
 * ------------------------------------------------------------------------ */
int soi_dip_select_dense_down(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                              const uint8_t* Wt, const float* St, int32_t* out_indices, int32_t* out_count,
                              uint16_t* y, int64_t H, int64_t group_size, int64_t num_groups, void* stream);

/* ------------------------------------------------------------------------
 * Residual update in the producer's epilogue: the projection whose output is
 * added to the residual stream (o_proj: python/soinfer/runtime/generate.py:172
 * `h2 = residual + o`; down: generate.py:182 / 310 `residual2 + down`) also
 * writes res_out[i] = res[i] + y[i], one binary16 addition (the fp32 sum
 * rounded once), the value soi_gemv_w4a16_rmsnorm / soi_residual_rmsnorm
 * compute from (res, delta = y). The next RMSNorm-fused GEMV then reads
 * res_out alone (delta null, x_out null) with bit-identical results.
 *   soi_gemv_w4a16_residual: soi_gemv_w4a16_group_lop3 (same y) plus
 *     res_out[N] = res + y; res and res_out are [N] and must not overlap y.
 *   soi_dip_select_dense_down_residual: soi_dip_select_dense_down (same y,
 *     index list and count) plus res_out[H] = res + y.
 * res_out may be res itself (each element is read, then written, by the one
 * lane that owns its row). No reference counterpart as single entry points:
 * each replaces a projection plus the add cited above.
 * ------------------------------------------------------------------------ */
int soi_gemv_w4a16_residual(const uint8_t* Wq, const float* scale, const uint16_t* x, uint16_t* y,
                            const uint16_t* res, uint16_t* res_out, int64_t N, int64_t K, int64_t group_size,
                            int64_t num_groups, void* stream);
int soi_dip_select_dense_down_residual(const uint16_t* gate, const uint16_t* h, int64_t num_channels, int64_t k,
                                       const uint8_t* Wt, const float* St, int32_t* out_indices,
                                       int32_t* out_count, uint16_t* y, const uint16_t* res, uint16_t* res_out,
                                       int64_t H, int64_t group_size, int64_t num_groups, void* stream);

/* ------------------------------------------------------------------------
 * Grid-wide barrier cost (measurement; no counterpart in the reference, whose
 * decode runs one kernel per op). A persistent decode launch would replace
 * each dependent launch boundary by a barrier among co-resident workgroups;
 * this measures the cheapest such barrier on the device: P workgroups of 256
 * threads run `rounds` rounds of (write 64 words device-coherent, barrier,
 * read another workgroup's words and count mismatches). Arrival is O(P) over
 * 8 counters (one per XCD) and a global counter, one lane per workgroup polls
 * one of 8 generation copies; fenced = 1 adds an agent-scope release before
 * the arrival and an acquire after the wait (plain data stores and loads).
 * Workspace (soi_grid_barrier_bench_workspace_bytes(P), 16-byte aligned,
 * zero-filled before the first call; later calls with the same P and fenced
 * flag may reuse it, since its counters continue from the last call's, but a
 * different P needs a fresh zero-filled workspace):
 * bytes [0, 4608) the sync block (uint32 word 1088: 1 if a bounded wait gave
 * up; word 1089: mismatched words), then 2 x P uint64 s_memrealtime stamps
 * (100 MHz; begin and end of workgroup b at 2b, 2b + 1), then the data.
 * P must not exceed soi_grid_barrier_max_workgroups() (every workgroup
 * resident at once); larger P is rejected before any launch.
 * ------------------------------------------------------------------------ */
size_t soi_grid_barrier_bench_workspace_bytes(int64_t P);
int soi_grid_barrier_max_workgroups(int64_t* max_workgroups);
int soi_grid_barrier_bench(int fenced, int64_t P, int64_t rounds, void* workspace, size_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOINFER_AMD_H_ */
