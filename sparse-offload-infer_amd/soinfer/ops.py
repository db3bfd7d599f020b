"""Typed wrappers over soinfer._C, the MI355X hot-path operators.

Names, arguments and return values follow the reference's python/soinfer/ops.py
(gemv_w8a16 :92-96, gemv_w4a16_group{,_lop3} :99-109, topk_threshold_select
:151-158, gather_rows_{staged,naive} :161-176, gemv_w4a16_sparse_accumulate
:179-188, build_dip_descriptors :191-199, gemv_dip_fused_{up,down} :202-219,
decode_attention :253-260) and, for the decode step around the hot path,
rmsnorm :57-59, gemv_fp16_v3 :82-84, precompute_rope_cos_sin / apply_rope /
qk_norm / kv_cache_append :222-250. Validation errors surface as
RuntimeError, as in the reference. Operators with no reference counterpart:
the batched / grouped GEMVs, the index-driven sparse GEMVs over HBM-resident
weights and the device row gather (the resident DIP path uses them instead of
host gathers); the decode engine's no-allocation forms live in soinfer._C.
"""
from __future__ import annotations

import torch

from . import _C


def gemv_w8a16(Wq: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, group_size: int) -> torch.Tensor:
    """y = dequant(Wq, scale) @ x. Wq: [N, K] int8; scale: [N, num_groups] or [1, num_groups] fp32 (per-tensor
    broadcast); x: [K] fp16. group_size: K for per-tensor/per-channel, else the quant group size."""
    return _C.gemv_w8a16(Wq, scale, x, group_size)


def gemv_w4a16_group(Wq_packed: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, K: int,
                     group_size: int) -> torch.Tensor:
    """y = dequant(Wq_packed, scale) @ x. Wq_packed: [N, ceil(K/8)*4] uint8 AWQ-order INT4 (soinfer.quant.pack);
    scale: [N, ceil(K/group_size)] fp32; group_size a positive multiple of 8. Per-nibble scalar dequant."""
    return _C.gemv_w4a16_group(Wq_packed, scale, x, K, group_size)


def gemv_w4a16_group_lop3(Wq_packed: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, K: int,
                          group_size: int) -> torch.Tensor:
    """Same contract and bit-identical result as gemv_w4a16_group; dequantizes with three-input bitwise
    binary16 construction (v_bitop3) instead of per-nibble conversion."""
    return _C.gemv_w4a16_group_lop3(Wq_packed, scale, x, K, group_size)


def gemv_w4a16_residual(Wq_packed: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, res: torch.Tensor, K: int,
                        group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The projection that feeds a residual add (reference generate.py:172 `h2 = residual + o`, :182 `residual2 +
    down`) with the add in its epilogue: returns (y, res_out), y as gemv_w4a16_group_lop3 gives it and
    res_out = res + y rounded once to binary16 (res: [N] fp16)."""
    N = Wq_packed.shape[0]
    y = torch.empty(N, dtype=torch.float16, device=x.device)
    res_out = torch.empty(N, dtype=torch.float16, device=x.device)
    _C.gemv_w4a16_residual_into(Wq_packed, scale, x, y, res, res_out, K, group_size)
    return y, res_out


def _check_aligned16(what: str, K: int, W: torch.Tensor, x: torch.Tensor) -> None:
    """The batched and grouped kernels read Wq and x with 16-byte loads when K % 32 == 0; a misaligned
    problem there would only come back as NaN rows, so it is rejected before launch."""
    if K % 32 == 0 and (W.data_ptr() % 16 or x.data_ptr() % 16):
        raise RuntimeError(f"{what}: Wq and x must be 16-byte aligned when K % 32 == 0 (got Wq at "
                           f"{W.data_ptr():#x}, x at {x.data_ptr():#x}); pass a .clone() of an offset view")


class GemvBatch:
    """P independent INT4 GEMVs of one shape [N, K] executed in ONE kernel launch.

    Validates every tensor once and keeps device pointer tables, so run() is a
    single launch (and can be captured in a HIP graph). y[p] is bit-identical to
    gemv_w4a16_group_lop3(Wqs[p], scales[p], xs[p], K, group_size)."""

    def __init__(self, Wqs, scales, xs, K: int, group_size: int, ys=None):
        P = len(Wqs)
        if not (len(scales) == len(xs) == P and P > 0):
            raise ValueError("GemvBatch: Wqs, scales and xs must be non-empty lists of equal length")
        N = Wqs[0].shape[0]
        G = -(-K // group_size)
        dev = Wqs[0].device
        if ys is None:
            ys = [torch.empty(N, dtype=torch.float16, device=dev) for _ in range(P)]
        for W, s, x, y in zip(Wqs, scales, xs, ys):
            if not (W.dtype == torch.uint8 and W.is_contiguous() and tuple(W.shape) == (N, -(-K // 8) * 4)):
                raise RuntimeError("GemvBatch: every Wq must be a contiguous uint8 [N, ceil(K/8)*4] tensor")
            if not (s.dtype == torch.float32 and s.is_contiguous() and tuple(s.shape) == (N, G)):
                raise RuntimeError("GemvBatch: every scale must be a contiguous float32 [N, ceil(K/gs)] tensor")
            if not (x.dtype == torch.float16 and x.is_contiguous() and tuple(x.shape) == (K,)):
                raise RuntimeError("GemvBatch: every x must be a contiguous float16 [K] tensor")
            if not (y.dtype == torch.float16 and y.is_contiguous() and tuple(y.shape) == (N,)):
                raise RuntimeError("GemvBatch: every y must be a contiguous float16 [N] tensor")
            if not all(t.device == dev for t in (W, s, x, y)):
                raise RuntimeError("GemvBatch: all tensors must be on one device")
            _check_aligned16("GemvBatch", K, W, x)
        self._keep = (list(Wqs), list(scales), list(xs), list(ys))
        self.ys = self._keep[3]
        self.N, self.K, self.group_size = N, K, group_size

        def table(ts):
            return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)

        self._tables = tuple(table(ts) for ts in self._keep)

    def run(self):
        _C.gemv_w4a16_batched(*self._tables, self.N, self.K, self.group_size)
        return self.ys


class Int8Batch:
    """P independent INT8 GEMVs of one shape [N, K] in ONE kernel launch (the INT8 counterpart of GemvBatch).

    scales: [N, G] group / per-channel scales, or [1, G] per-tensor (every problem the same kind). y[p] is
    bit-identical to gemv_w8a16(Wqs[p], scales[p], xs[p], group_size)."""

    def __init__(self, Wqs, scales, xs, group_size: int, ys=None):
        P = len(Wqs)
        if not (len(scales) == len(xs) == P and P > 0):
            raise ValueError("Int8Batch: Wqs, scales and xs must be non-empty lists of equal length")
        N, K = Wqs[0].shape
        G = scales[0].shape[1]
        per_tensor = scales[0].shape[0] == 1 and N != 1
        dev = Wqs[0].device
        if ys is None:
            ys = [torch.empty(N, dtype=torch.float16, device=dev) for _ in range(P)]
        for W, s, x, y in zip(Wqs, scales, xs, ys):
            if not (W.dtype == torch.int8 and W.is_contiguous() and tuple(W.shape) == (N, K)):
                raise RuntimeError("Int8Batch: every Wq must be a contiguous int8 [N, K] tensor")
            if not (s.dtype == torch.float32 and s.is_contiguous() and tuple(s.shape) == ((1 if per_tensor else N), G)):
                raise RuntimeError("Int8Batch: every scale must be a contiguous float32 [N or 1, G] tensor, all alike")
            if not (x.dtype == torch.float16 and x.is_contiguous() and tuple(x.shape) == (K,)):
                raise RuntimeError("Int8Batch: every x must be a contiguous float16 [K] tensor")
            if not (y.dtype == torch.float16 and y.is_contiguous() and tuple(y.shape) == (N,)):
                raise RuntimeError("Int8Batch: every y must be a contiguous float16 [N] tensor")
            if not all(t.device == dev for t in (W, s, x, y)):
                raise RuntimeError("Int8Batch: all tensors must be on one device")
            if K % 16 == 0 and (W.data_ptr() % 16 or x.data_ptr() % 16):
                raise RuntimeError("Int8Batch: Wq and x must be 16-byte aligned when K % 16 == 0")
        if G != 1 and (G != -(-K // group_size) or group_size % 4):
            raise RuntimeError("Int8Batch: G must be 1 or ceil(K / group_size), group_size a multiple of 4")
        self._keep = (list(Wqs), list(scales), list(xs), list(ys))
        self.ys = self._keep[3]
        self.N, self.K, self.group_size, self.G = N, K, group_size, G
        self.stride = 0 if per_tensor else G

        def table(ts):
            return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)

        self._tables = tuple(table(ts) for ts in self._keep)

    def run(self):
        _C.gemv_w8a16_batched(*self._tables, self.N, self.K, self.group_size, self.G, self.stride)
        return self.ys


class GemvGroup:
    """Independent INT4 GEMVs of up to 8 different shapes executed in ONE kernel launch.

    problems: list of (Wq, scale, x, K). Problems are grouped by shape; classes are
    laid out longest-row first. run() is a single launch; ys[i] (same order as
    problems) is bit-identical to gemv_w4a16_group_lop3 on problem i."""

    def __init__(self, problems, group_size: int, ys=None):
        if not problems:
            raise ValueError("GemvGroup: no problems")
        dev = problems[0][0].device
        shapes = []
        for W, s, x, K in problems:
            N = W.shape[0]
            G = -(-K // group_size)
            if not (W.dtype == torch.uint8 and W.is_contiguous() and tuple(W.shape) == (N, -(-K // 8) * 4)):
                raise RuntimeError("GemvGroup: every Wq must be a contiguous uint8 [N, ceil(K/8)*4] tensor")
            if not (s.dtype == torch.float32 and s.is_contiguous() and tuple(s.shape) == (N, G)):
                raise RuntimeError("GemvGroup: every scale must be a contiguous float32 [N, ceil(K/gs)] tensor")
            if not (x.dtype == torch.float16 and x.is_contiguous() and tuple(x.shape) == (K,)):
                raise RuntimeError("GemvGroup: every x must be a contiguous float16 [K] tensor")
            if not all(t.device == dev for t in (W, s, x)):
                raise RuntimeError("GemvGroup: all tensors must be on one device")
            _check_aligned16("GemvGroup", K, W, x)
            shapes.append((N, K))
        classes = sorted(set(shapes), key=lambda nk: (-nk[1], -nk[0]))
        if len(classes) > 8:
            raise RuntimeError("GemvGroup: at most 8 distinct shapes per launch")
        if ys is None:
            ys = [torch.empty(N, dtype=torch.float16, device=dev) for N, _ in shapes]
        for y, (N, _) in zip(ys, shapes):
            if not (y.dtype == torch.float16 and y.is_contiguous() and tuple(y.shape) == (N,) and y.device == dev):
                raise RuntimeError("GemvGroup: every y must be a contiguous float16 [N] tensor on the device")
        order = [i for c in classes for i, sh in enumerate(shapes) if sh == c]
        self._keep = ([problems[i][0] for i in order], [problems[i][1] for i in order],
                      [problems[i][2] for i in order], [ys[i] for i in order])
        self.ys = list(ys)
        self.class_count = [shapes.count(c) for c in classes]
        self.class_N = [c[0] for c in classes]
        self.class_K = [c[1] for c in classes]
        self.group_size = group_size

        def table(ts):
            return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device=dev)

        self._tables = tuple(table(ts) for ts in self._keep)

    def run(self):
        _C.gemv_w4a16_grouped(*self._tables, self.class_count, self.class_N, self.class_K, self.group_size)
        return self.ys


def gemv_w4a16_batched(Wqs, scales, xs, K: int, group_size: int):
    """Convenience one-shot form of GemvBatch: returns the list of outputs."""
    return GemvBatch(Wqs, scales, xs, K, group_size).run()


def topk_threshold_select(abs_g: torch.Tensor, k: int) -> torch.Tensor:
    """Indices (int32 [k], ascending) selected by the reference's threshold rule over abs_g (1-D fp32,
    non-negative): tau from 24 fp32 bisection steps, then the first k indices with abs_g >= tau.
    Deterministic: repeated calls return identical tensors."""
    indices, _count = _C.topk_threshold_select(abs_g, k)
    return indices


def gather_rows_staged(matrix: torch.Tensor, indices: torch.Tensor, staging: torch.Tensor,
                       gpu_dst: torch.Tensor) -> None:
    """Copy the selected rows of `matrix` (pinned CPU uint8 [num_rows, row_nbytes]) into pinned `staging`
    (>= k*row_nbytes) with host memcpy, then one async H2D copy into `gpu_dst` on the current stream.
    indices: 1-D int64 CPU tensor (range-checked). Synchronize before reading gpu_dst."""
    _C.gather_rows_staged(matrix, indices, staging, gpu_dst)


def gather_rows_naive(matrix: torch.Tensor, indices: torch.Tensor, gpu_dst: torch.Tensor) -> None:
    """One async H2D copy per selected row; same arguments and semantics as gather_rows_staged."""
    _C.gather_rows_naive(matrix, indices, gpu_dst)


def gemv_w4a16_sparse_accumulate(Wq_selected: torch.Tensor, scale_selected: torch.Tensor,
                                 h_selected: torch.Tensor, H: int, group_size: int) -> torch.Tensor:
    """y[H] = sum_i h_selected[i] * dequant(Wq_selected[i, :]) over k already-gathered rows of down_proj stored
    transposed ([intermediate, hidden]). Deterministic split over rows with a fixed-order combine."""
    return _C.gemv_w4a16_sparse_accumulate(Wq_selected, scale_selected, h_selected, H, group_size)


def build_dip_descriptors(selected_indices: torch.Tensor, slot_of: torch.Tensor):
    """(descriptors, miss_channels, miss_count) for the hot-channel cache: descriptor = cache slot, or miss
    position | 1<<31. Misses are numbered in ascending selection order; only miss_channels[:miss_count] is
    valid."""
    return _C.build_dip_descriptors(selected_indices, slot_of)


def gemv_dip_fused_up(cache_Wq: torch.Tensor, cache_scale: torch.Tensor, staging_Wq: torch.Tensor,
                      staging_scale: torch.Tensor, descriptors: torch.Tensor, x: torch.Tensor, K: int,
                      group_size: int) -> torch.Tensor:
    """y[k] = selected rows @ x, each row read from the resident cache or the staging buffer per its
    descriptor. Bit-identical to gemv_w4a16_group_lop3 on the same logical rows."""
    return _C.gemv_dip_fused_up(cache_Wq, cache_scale, staging_Wq, staging_scale, descriptors, x, K, group_size)


def gemv_dip_fused_down(cache_Wq: torch.Tensor, cache_scale: torch.Tensor, staging_Wq: torch.Tensor,
                        staging_scale: torch.Tensor, descriptors: torch.Tensor, h_selected: torch.Tensor, H: int,
                        group_size: int) -> torch.Tensor:
    """Descriptor-driven form of gemv_w4a16_sparse_accumulate; bit-identical to it on the same logical rows."""
    return _C.gemv_dip_fused_down(cache_Wq, cache_scale, staging_Wq, staging_scale, descriptors, h_selected, H,
                                  group_size)


def gemv_w4a16_indexed(Wq_packed: torch.Tensor, scale: torch.Tensor, idx: torch.Tensor, x: torch.Tensor, K: int,
                       group_size: int) -> torch.Tensor:
    """y[j] = row idx[j] of the HBM-resident INT4 matrix @ x (no gather). Bit-identical to
    gemv_w4a16_group_lop3(Wq_packed[idx], scale[idx], x, K, group_size)."""
    return _C.gemv_w4a16_indexed(Wq_packed, scale, idx, x, K, group_size)


def gemv_w4a16_indexed_accumulate(Wq_T: torch.Tensor, scale_T: torch.Tensor, idx: torch.Tensor,
                                  h_selected: torch.Tensor, H: int, group_size: int) -> torch.Tensor:
    """y[H] = sum_j h_selected[j] * row idx[j] of the HBM-resident down_proj^T (no gather). Bit-identical to
    gemv_w4a16_sparse_accumulate(Wq_T[idx], scale_T[idx], h_selected, H, group_size)."""
    return _C.gemv_w4a16_indexed_accumulate(Wq_T, scale_T, idx, h_selected, H, group_size)


def transposed_down_T(Wq_T: torch.Tensor, scale_T: torch.Tensor, H: int) -> tuple[torch.Tensor, torch.Tensor]:
    """The same quantized down_proj^T values laid out for dip_select_dense_down: Wq_T [n, ceil(H/8)*4] packed
    rows (channel c's H nibbles) -> Wt [H, n/2] (output column col's n nibbles, packed like every INT4 row,
    n % 8 == 0), scale_T [n, G] -> St [G, n]. No rounding: Wt unpacks to the transpose of Wq_T's values."""
    from soinfer.quant import pack

    n = Wq_T.shape[0]
    if n % 8:
        raise ValueError("transposed_down_T: the channel count must be a multiple of 8")
    q = pack.unpack_int4(Wq_T, H)  # int8 [n, H]
    Wt, _ = pack.pack_int4(q.t().contiguous())
    return Wt.contiguous(), scale_T.t().contiguous()


def dip_select_dense_down(gate: torch.Tensor, h: torch.Tensor, k: int, Wt: torch.Tensor, St: torch.Tensor,
                          group_size: int, with_indices: bool = True):
    """One-launch DIP selection + down projection over resident weights (Wt, St from transposed_down_T):
    y[H] = sum over the rule-A selection of top-k |gate| of h[c] * down_proj^T row c. Returns (y, indices,
    count), the indices and count as topk_threshold_select gives them (None without with_indices)."""
    H = Wt.shape[0]
    y = torch.empty(H, dtype=torch.float16, device=gate.device)
    idx = torch.empty(k, dtype=torch.int32, device=gate.device) if with_indices else None
    cnt = torch.empty(1, dtype=torch.int32, device=gate.device) if with_indices else None
    _C.dip_select_dense_down_into(gate, h, k, Wt, St, idx, cnt, y, group_size)
    return y, idx, cnt


def dip_select_dense_down_residual(gate: torch.Tensor, h: torch.Tensor, k: int, Wt: torch.Tensor, St: torch.Tensor,
                                   group_size: int, res: torch.Tensor, with_indices: bool = True):
    """dip_select_dense_down with the residual add (reference generate.py:310 `residual2 + down_out`) in the
    same launch: returns (y, res_out, indices, count), res_out = res + y rounded once to binary16."""
    H = Wt.shape[0]
    y = torch.empty(H, dtype=torch.float16, device=gate.device)
    res_out = torch.empty(H, dtype=torch.float16, device=gate.device)
    idx = torch.empty(k, dtype=torch.int32, device=gate.device) if with_indices else None
    cnt = torch.empty(1, dtype=torch.int32, device=gate.device) if with_indices else None
    _C.dip_select_dense_down_into(gate, h, k, Wt, St, idx, cnt, y, group_size, res, res_out)
    return y, res_out, idx, cnt


def gather_rows_device(src: torch.Tensor, idx: torch.Tensor, dst: torch.Tensor) -> None:
    """dst[j, :] = src[idx[j], :] for device-resident rows (int32 indices; out-of-range -> zero row)."""
    _C.gather_rows_device(src, idx, dst)


def decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cur_len: int) -> torch.Tensor:
    """out = attention(q, k_cache[:, :cur_len], v_cache[:, :cur_len]) for one query token. q: [NQ, hd] fp16
    (already RoPE'd / QK-normed); caches: [NKV, max_seq_len, hd] fp16; NQ % NKV == 0 (query head h reads KV
    head h // (NQ // NKV)); scale 1/sqrt(hd)."""
    return _C.decode_attention(q, k_cache, v_cache, cur_len)


# ---------------------------------------------------------------------------
# decode-step glue (reference python/soinfer/ops.py:57-59, 82-84, 222-250)
# ---------------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """RMSNorm over the last dim: x * rsqrt(mean(x^2) + eps) * weight. x: [rows, hidden] fp16, weight: [hidden]
    fp16, hidden even; fp32 math, fp16 out."""
    return _C.rmsnorm(x, weight, eps)


def gemv_fp16_v3(W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """y = W @ x for fp16 W [N, K] and x [K] (K % 8 == 0), fp32 accumulation, fp16 out (the LM head)."""
    return _C.gemv_fp16_v3(W, x)


def swiglu_gate_up(gate_W: torch.Tensor, up_W: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """h = silu(gate_W @ x) * (up_W @ x) (reference ops.py:112-116). gate_W, up_W: [I, H] fp16 of the same
    shape, x: [H] fp16, H % 8 == 0. One kernel: each wave streams rows of both matrices against one read of x,
    sums in fp32 and applies silu(g) * u = g / (1 + exp(-g)) * u to the sums; only h is written."""
    return _C.swiglu_gate_up(gate_W, up_W, x)


def fused_swiglu_mlp(gate_W: torch.Tensor, up_W: torch.Tensor, down_W: torch.Tensor,
                     x: torch.Tensor) -> torch.Tensor:
    """y = down_W @ (silu(gate_W @ x) * (up_W @ x)), the fp16 SwiGLU MLP (reference ops.py:119-125): gate_W, up_W
    [I, H], down_W [H, I], x [H]. swiglu_gate_up, then gemv_fp16_v3 for the down projection, which needs all of
    h before any output row can finish."""
    return gemv_fp16_v3(down_W, swiglu_gate_up(gate_W, up_W, x))


def concat_qkv_weights(Wq: torch.Tensor, Wk: torch.Tensor, Wv: torch.Tensor) -> torch.Tensor:
    """[q_dim + 2 kv_dim, H] = rows of Wq, then Wk, then Wv (reference ops.py:128-132), built once at load time
    for fused_qkv_projection."""
    return torch.cat([Wq, Wk, Wv], dim=0).contiguous()


def fused_qkv_projection(qkv_W: torch.Tensor, x: torch.Tensor, q_dim: int,
                         kv_dim: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v = split(qkv_W @ x, [q_dim, kv_dim, kv_dim]) (reference ops.py:135-149): one fp16 GEMV over the
    concatenated weight from concat_qkv_weights, one pass over x; q, k, v are views of its output (a row count
    other than q_dim + 2 kv_dim makes the split raise, as in the reference)."""
    q, k, v = gemv_fp16_v3(qkv_W, x).split([q_dim, kv_dim, kv_dim])
    return q, k, v


def precompute_rope_cos_sin(head_dim: int, theta: float, pos: int, device, dtype=torch.float32):
    """cos/sin [head_dim/2] at absolute position pos: inv_freq[i] = 1 / theta^(2i/head_dim),
    angle_i = pos * inv_freq[i], computed in fp32 (the Qwen3 / HF rotary convention)."""
    cos_t, sin_t = rope_tables(head_dim, theta, pos + 1, device)
    return cos_t[pos].to(dtype).contiguous(), sin_t[pos].to(dtype).contiguous()


def rope_tables(head_dim: int, theta: float, max_seq: int, device):
    """cos/sin tables [max_seq, head_dim/2] fp32, row p = the angles at position p (same fp32 operations as
    precompute_rope_cos_sin, one row per position)."""
    exponent = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim
    inv_freq = 1.0 / (theta ** exponent)
    angles = torch.arange(max_seq, dtype=torch.float32, device=device)[:, None] * inv_freq[None, :]
    return angles.cos().contiguous(), angles.sin().contiguous()


def apply_rope(x: torch.Tensor, cos_vals: torch.Tensor, sin_vals: torch.Tensor) -> torch.Tensor:
    """RoPE in place on x [num_heads, head_dim] fp16 (rotate-half convention); cos/sin fp32 [head_dim/2].
    Returns x."""
    _C.rope_apply(x, cos_vals, sin_vals)
    return x


def qk_norm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Qwen3 per-head QK-norm: RMSNorm over head_dim for each head of x [num_heads, head_dim]."""
    return rmsnorm(x, weight, eps)


def kv_cache_append(k_cache: torch.Tensor, v_cache: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                    pos: int) -> None:
    """Write k_new / v_new [NKV, hd] into the caches [NKV, max_seq, hd] at position pos, in place."""
    _C.kv_cache_append(k_cache, v_cache, k_new, v_new, pos)
