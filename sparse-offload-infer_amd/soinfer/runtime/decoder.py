"""Batch-1 greedy decoding of a Qwen3-shaped INT4 decoder on one MI355X.

Follows the reference's decode step (python/soinfer/runtime/generate.py):
per layer (run_decoder_layer_streaming :141-182, run_decoder_layer_dip
:215-310, run_decoder_layer_cached_dip :313-404)

    h    = rmsnorm(x, input_layernorm)
    q,k,v= INT4 GEMV(h)                            (one fused [q|k|v] GEMV here)
    q,k  = rope(qk_norm(q)), rope(qk_norm(k));  append k, v at pos
    a    = decode_attention(q, caches, pos + 1)
    x    = x + INT4 GEMV(W_o, a)
    h3   = rmsnorm(x, post_attention_layernorm)
    MLP  dense: down(fp16(silu(gate) * up))     DIP: top-k of |gate|, sparse up/down
    x    = x + MLP(h3)

and the loop of generate_streaming / generate_dip / generate_cached_dip
(:429-520): prompt tokens one at a time, then rmsnorm(final_norm) -> fp16
LM head GEMV -> argmax per new token.

MI355X design: every weight is resident in HBM (the whole 1.7B INT4 model,
its fp16 embedding and LM head take ~2.2 GB of 288 GB); the token, the
position and the generated-token log live in device memory, every op writes
into preallocated buffers, and one decode step (LM head + argmax + 28 layers)
is captured once as a HIP graph and replayed, so generation needs no host
round trip until the end. The residual add is fused into the following
RMSNorm and q/k-norm + RoPE + KV append into one launch; both give the same
binary16 values as the separate ops. The cache-aware DIP mode keeps every
layer's up / down^T matrices in one pinned host arena (PinnedWeightStore) and
the hot rows in HBM; the up GEMV and the down accumulate read each selected
channel from the cache or, for a miss, straight from the arena's device
mapping (miss_path "direct"), or the misses are first gathered into device
staging buffers and read through descriptors (miss_path "staged", the
reference's shape). Either way the output is bit-identical to DIP with
everything resident.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import torch

from .. import _C
from .. import ops
from ..offload.hot_cache import HotCache
from ..offload.stream_manager import StreamManager
from ..offload.weight_store import PinnedWeightStore, plan_bytes
from ..quant import formats, pack

# Generation steps per replay of the chunk graph (decode replays it for each full chunk of the requested steps)
GRAPH_CHUNK = 4


@dataclass(frozen=True)
class DecoderConfig:
    hidden: int = 2048
    layers: int = 28
    q_heads: int = 16
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 6144
    vocab: int = 151936
    group_size: int = 128
    rms_eps: float = 1e-6
    rope_theta: float = 1_000_000.0
    max_seq: int = 2048

    @property
    def qkv_rows(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


QWEN3_1P7B = DecoderConfig()


@dataclass
class LayerWeights:
    in_norm: torch.Tensor  # [H] fp16
    post_norm: torch.Tensor  # [H]
    q_norm: torch.Tensor  # [hd]
    k_norm: torch.Tensor  # [hd]
    qkv_Wq: torch.Tensor  # [(NQ+2NKV)*hd, H/2] uint8, rows q | k | v
    qkv_scale: torch.Tensor  # [(NQ+2NKV)*hd, H/gs] fp32
    o_Wq: torch.Tensor  # [H, NQ*hd/2]
    o_scale: torch.Tensor
    gu_Wq: torch.Tensor  # [2I, H/2], rows gate | up
    gu_scale: torch.Tensor
    down_Wq: torch.Tensor  # [H, I/2] (dense path)
    down_scale: torch.Tensor
    down_T_Wq: torch.Tensor  # [I, H/2] (DIP path: a channel is a row)
    down_T_scale: torch.Tensor

    def gate(self, I: int):
        return self.gu_Wq[:I], self.gu_scale[:I]

    def up(self, I: int):
        return self.gu_Wq[I:], self.gu_scale[I:]


@dataclass
class DecoderWeights:
    config: DecoderConfig
    embed: torch.Tensor  # [V, H] fp16
    lm_head: torch.Tensor  # [V, H] fp16
    final_norm: torch.Tensor  # [H] fp16
    layers: list = field(default_factory=list)
    # the LM head quantized like every linear (INT4, group config.group_size, fp32 scales): (packed [V, H/2],
    # scales [V, H/gs]); made on first use by quantize_lm_head
    lm_head_int4: Optional[tuple] = None


def _quant_int4(w: torch.Tensor, gs: int):
    qt = formats.quantize(w, formats.QuantConfig(bits=4, granularity="group", group_size=gs))
    Wq, _ = pack.pack_int4(qt.qweight)
    return Wq.contiguous(), qt.scale.contiguous()


def quantize_lm_head(w: "DecoderWeights") -> tuple:
    """The fp16 LM head quantized with the linears' quantizer (symmetric INT4, group config.group_size, fp32
    scales; formats.quantize + pack_int4), kept on the weights for later engines. The reference keeps its head
    in fp16 (loader.py:55, generate.py:489-491); this is the head of a decoder whose weights are all INT4 g128."""
    if w.lm_head_int4 is None:
        V, H = w.lm_head.shape
        rows = 16384  # quantize in row blocks: the fp32 copy of a whole 151936 x 2048 head would be 1.2 GB
        parts = [_quant_int4(w.lm_head[r:r + rows].float(), w.config.group_size) for r in range(0, V, rows)]
        w.lm_head_int4 = (torch.cat([p[0] for p in parts]).contiguous(), torch.cat([p[1] for p in parts]).contiguous())
    return w.lm_head_int4


def random_decoder(config: DecoderConfig = QWEN3_1P7B, seed: int = 0, device="cuda", linear_std: float = 0.02,
                   norm_jitter: float = 0.0) -> DecoderWeights:
    """Random-init weights of the given shape: linears N(0, linear_std) quantized to INT4 (group
    config.group_size, fp32 scales), embedding N(0, 1) and LM head N(0, linear_std) in fp16, norms 1
    (+ N(0, norm_jitter) when given). down_proj is quantized twice, as [H, I] for the dense path and as
    its transpose [I, H] for DIP (the reference registers both, load_hf_checkpoint.py:90-111)."""
    c = config
    g = torch.Generator(device=device).manual_seed(seed)

    def randn(*shape, std=1.0):
        return torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std

    def norm(n):
        v = torch.ones(n, device=device)
        if norm_jitter:
            v = v + randn(n, std=norm_jitter)
        return v.half().contiguous()

    H, I, hd, gs = c.hidden, c.intermediate, c.head_dim, c.group_size
    layers = []
    for _ in range(c.layers):
        wq = randn(c.qkv_rows, H, std=linear_std)
        wo = randn(H, c.q_heads * hd, std=linear_std)
        wgu = randn(2 * I, H, std=linear_std)
        wd = randn(H, I, std=linear_std)
        qkv_Wq, qkv_s = _quant_int4(wq, gs)
        o_Wq, o_s = _quant_int4(wo, gs)
        gu_Wq, gu_s = _quant_int4(wgu, gs)
        d_Wq, d_s = _quant_int4(wd, gs)
        dT_Wq, dT_s = _quant_int4(wd.t().contiguous(), gs)
        del wq, wo, wgu, wd
        layers.append(LayerWeights(norm(H), norm(H), norm(hd), norm(hd), qkv_Wq, qkv_s, o_Wq, o_s, gu_Wq, gu_s,
                                   d_Wq, d_s, dT_Wq, dT_s))
    embed = randn(c.vocab, H).half().contiguous()
    lm_head = randn(c.vocab, H, std=linear_std).half().contiguous()
    return DecoderWeights(c, embed, lm_head, norm(H), layers)


def decoder_weights_from_arena(store, matrices, config: DecoderConfig, embed: torch.Tensor, lm_head: torch.Tensor,
                               final_norm: torch.Tensor, layer_norms: list, device=None) -> DecoderWeights:
    """DecoderWeights over a checkpoint loaded by offload.load_hf_checkpoint.stream_load_layers (with
    include_down_proj_t=True): q|k|v and gate|up are views of consecutive arena rows (the loader registers them
    in that order), scales are concatenated on the GPU. device=None keeps every packed matrix in the pinned
    arena (for DecodeEngine(offload=True)); a device copies them there (resident modes). embed / lm_head /
    final_norm: fp16 on the GPU; layer_norms[l]: dict with input_layernorm, post_attention_layernorm, q_norm,
    k_norm (fp16 on the GPU), as the reference keeps them (generate.py:60-80)."""
    from ..offload.load_hf_checkpoint import DOWN_PROJ_T_SUFFIX

    def span(names):
        hs = [matrices[n].handle for n in names]
        rb = hs[0].row_nbytes
        for a, b in zip(hs, hs[1:]):
            if b.offset != a.offset + a.nbytes or b.row_nbytes != rb:
                raise ValueError(f"{names}: not consecutive rows of one width in the arena")
        rows = sum(h.num_rows for h in hs)
        v = store.arena[hs[0].offset:hs[0].offset + rows * rb].view(rows, rb)
        return v if device is None else v.to(device)

    def scales(names):
        return torch.cat([matrices[n].scale for n in names]).contiguous()

    def one(name):
        v = store.matrix_view(matrices[name].handle)
        return v if device is None else v.to(device)

    layers = []
    for l in range(config.layers):
        p = f"model.layers.{l}."
        qkv = [p + f"self_attn.{x}_proj.weight" for x in ("q", "k", "v")]
        gu = [p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight"]
        o, down, down_T = p + "self_attn.o_proj.weight", p + "mlp.down_proj.weight", p + DOWN_PROJ_T_SUFFIX
        nm = layer_norms[l]
        layers.append(LayerWeights(nm["input_layernorm"], nm["post_attention_layernorm"], nm["q_norm"], nm["k_norm"],
                                   span(qkv), scales(qkv), one(o), matrices[o].scale, span(gu), scales(gu),
                                   one(down), matrices[down].scale, one(down_T), matrices[down_T].scale))
    return DecoderWeights(config, embed, lm_head, final_norm, layers)


class DecodeEngine:
    """Greedy decoder over DecoderWeights. mode: "dense", "dip" (top dip_k channels per layer, weights
    resident) or "cached_dip" (hot channels resident, the rest in pinned host memory; miss_path "direct" reads
    the misses in place inside the up / down kernels, "staged" gathers them into device staging first).
    dip_schedule (mode "dip"): "indexed" (default; 4 MLP launches, the schedule cached_dip equals bit for bit),
    "gated" (2 MLP launches, the same tokens and hidden states as "indexed" bit for bit) or "dense_up" (2 MLP
    launches, y summed in another order; dip_dense_up=True is the same).
    offload=True keeps the dense weights of every layer (q|k|v, o, and gate|up + down for dense or gate for
    cached DIP) in a pinned host arena and copies each layer's block into one of two device slots: the
    reference's streamed configuration (WeightPipeline, generate.py:85-138). With overlap_copy=True (default)
    the copies run on a StreamManager's copy streams, two layers ahead of the kernels: layer l + 2's block goes
    into slot l % 2 as soon as layer l's kernels are done with it (read-done fence), layer l's kernels wait for
    its block to land, and a generation step starts the copies of layers 0 and 1 before the LM head, so they
    overlap it. overlap_copy=False copies each block stream-ordered right before its layer. Scales, norms,
    embedding and LM head stay in HBM. With fused layers and residual_epilogue=True (default) the projections
    that feed a residual add (o in every mode, down in the dense and dense-up schedules) write the updated
    residual stream themselves, one binary16 add as the next RMSNorm-fused GEMV would do on load (results bit
    for bit those of residual_epilogue=False, which leaves the add to the consumer). With
    defer_attention_combine=True (default, fused layers) a context long enough to split the attention across
    workgroups leaves its split states to the o projection, which combines them while its weight rows load
    (bit-identical to False, where the attention launch's last workgroup per KV head combines them).
    int4_head=True runs the LM head as the INT4 g128 GEMV of the head quantized like the linears
    (quantize_lm_head: 166 MB read per token instead of the fp16 head's 622 MB); the default is the reference's
    fp16 head.

    All buffers are allocated here; decode steps launch only this package's kernels on the current stream
    and are captured into HIP graphs by capture()."""

    def __init__(self, w: DecoderWeights, mode: str = "dense", dip_k: Optional[int] = None,
                 hot_channels: Optional[list] = None, max_new_tokens: int = 256, fused: bool = True,
                 dip_dense_up: bool = False, miss_path: str = "direct", offload: bool = False,
                 down_copy: bool = True, overlap_copy: bool = True, residual_epilogue: bool = True,
                 defer_attention_combine: bool = True, int4_head: bool = False, dip_schedule: Optional[str] = None):
        if mode not in ("dense", "dip", "cached_dip"):
            raise ValueError(f"unknown mode {mode!r}")
        if dip_schedule is None:
            dip_schedule = "dense_up" if dip_dense_up else "indexed"
        if dip_schedule not in ("indexed", "dense_up", "gated"):
            raise ValueError(f"unknown dip_schedule {dip_schedule!r}")
        if dip_dense_up and dip_schedule != "dense_up":
            raise ValueError("dip_dense_up=True is dip_schedule='dense_up'")
        if dip_schedule != "indexed" and mode != "dip":
            raise ValueError(f"dip_schedule {dip_schedule!r} applies to mode 'dip' (weights resident)")
        dip_dense_up = dip_schedule == "dense_up"
        if offload and mode == "dip":
            raise ValueError("offload streams the dense weights; for DIP with every selected row read from host "
                             "memory use mode 'cached_dip' with empty hot-channel lists")
        if miss_path not in ("direct", "staged"):
            raise ValueError(f"unknown miss_path {miss_path!r}")
        self.miss_path = miss_path
        # direct path, fused layers: the up GEMV also copies the down^T miss rows to staging (False: the down
        # accumulate reads them in place)
        self.down_copy = down_copy
        # DIP schedules for resident weights (mode 'dip'):
        #  * "indexed" (default): RMSNorm-fused gate GEMV, top-k, up GEMV over the selected rows with the SiLU
        #    epilogue, sparse down over the selected down^T rows (4 MLP launches); the cache-aware modes equal it
        #    bit for bit;
        #  * "gated" (2 MLP launches, the same y as "indexed" bit for bit): where the shape fits
        #    (dip_select_down_ordered_lds_bytes > 0), one launch computes gate and h = fp16(silu(gate) * up) of
        #    every channel (RMSNorm on load; the rounding of the indexed up GEMV's SiLU epilogue), and a second
        #    runs the rule-A selection in each of its workgroups and the down over a transposed copy of
        #    down_proj^T, each output column replaying the sparse accumulate's partition and order, with no
        #    cross-workgroup step and the residual add in its epilogue; otherwise the first launch stores gate
        #    and up, and the second runs the selection and the sparse down over the selected down^T rows with h
        #    formed on load;
        #  * "dense_up": one launch computes gate and h = fp16(silu(gate) * up) of every channel, a second runs
        #    the rule-A selection in each of its workgroups and the down projection as a GEMV over a transposed
        #    copy of down_proj^T's quantized values with the masked coefficients (no cross-workgroup step). The
        #    selection equals the other schedules'; y sums the same terms in another order (within the sparse
        #    accumulate's tolerance, not bit for bit).
        self.dip_schedule = dip_schedule
        self.dip_dense_up = dip_dense_up
        self.dip_gated = dip_schedule == "gated"
        self.dip_gated_tr = self.dip_gated and dip_k is not None and 1 <= dip_k <= w.config.intermediate and \
            _C.dip_select_down_ordered_lds_bytes(w.config.hidden, w.config.intermediate, dip_k) > 0
        c = w.config
        self.w, self.c, self.mode, self.fused = w, c, mode, fused
        self.residual_epilogue = bool(residual_epilogue)
        dev = w.embed.device
        self.device = dev
        H, I, hd = c.hidden, c.intermediate, c.head_dim
        f16, i32 = torch.float16, torch.int32

        def buf(n, dtype=f16):
            return torch.zeros(n, dtype=dtype, device=dev)

        self.token = buf(1, i32)
        self.pos = buf(1, i32)
        self.log = buf(max_new_tokens, i32)
        self.log_len = buf(1, i32)
        self.x, self.h, self.hn = buf(H), buf(H), buf(H)
        self.x2 = buf(H)  # second residual buffer (the fused GEMVs write x + delta to the other buffer)
        self.qkv = buf(c.qkv_rows)
        self.q = torch.zeros(c.q_heads, hd, dtype=f16, device=dev)
        self.attn = buf(c.q_heads * hd)
        self.o, self.down = buf(H), buf(H)
        self.gu = buf(2 * I)
        self.mlp_h = buf(I)
        self.logits = buf(c.vocab)
        self.k_cache = [torch.zeros(c.kv_heads, c.max_seq, hd, dtype=f16, device=dev) for _ in range(c.layers)]
        self.v_cache = [torch.zeros(c.kv_heads, c.max_seq, hd, dtype=f16, device=dev) for _ in range(c.layers)]
        self.cos_t, self.sin_t = ops.rope_tables(hd, c.rope_theta, c.max_seq, dev)
        self.attn_ws = buf(max(1, _C.decode_attention_workspace_bytes(c.q_heads, c.kv_heads, hd, c.max_seq)),
                           torch.uint8)
        self.argmax_ws = buf(_C.argmax_workspace_bytes(c.vocab), torch.uint8)
        # one-launch attention (its workspace ends in counters that must start at zero: buf() zero-fills)
        step_ws = _C.decode_attention_step_workspace_bytes(c.q_heads, c.kv_heads, hd, c.max_seq)
        self.step_ws = buf(step_ws, torch.uint8) if (fused and step_ws > 0) else None
        # a context that splits across attention workgroups: the o projection combines the split states on load
        # (soi_gemv_w4a16_attn_combine) instead of the attention launch's last workgroup per KV head
        K_o = c.q_heads * hd
        self.defer_combine = bool(defer_attention_combine) and self.step_ws is not None and K_o % 32 == 0 and \
            K_o <= 2048
        self.counts = None  # optional per-layer channel selection counts (eager calibration only)
        # LM head: fp16 GEMV (the reference's head), or the INT4 g128 GEMV of the quantized head
        self.head_q = quantize_lm_head(w) if int4_head else None

        if mode != "dense":
            if dip_k is None or not 1 <= dip_k <= I:
                raise ValueError("dip_k must be in [1, intermediate]")
            self.k = dip_k
            self.idx, self.cnt = buf(dip_k, i32), buf(1, i32)
            self.u_sel, self.h_sel = buf(dip_k), buf(dip_k)
            self.sd_ws = buf(max(1, _C.sparse_accumulate_workspace_bytes(H, dip_k)), torch.uint8)
        if mode == "cached_dip":
            if hot_channels is None or len(hot_channels) != c.layers:
                raise ValueError("cached_dip needs one hot-channel list per layer")
            self._setup_cache(hot_channels)
        if dip_dense_up or self.dip_gated_tr:
            # down_proj^T's values transposed for the one-launch down (the same quantized values, no rounding)
            self.down_tt = [ops.transposed_down_T(L.down_T_Wq, L.down_T_scale, H) for L in w.layers]
        if fused and (mode == "dense" or dip_schedule != "indexed"):
            # gate|up rows interleaved by 8-row tiles (gate 4t..4t+3, up 4t..4t+3) for the SwiGLU epilogue
            t = torch.arange(I // 4, device=dev)
            perm = torch.stack([4 * t + i for i in range(4)] + [I + 4 * t + i for i in range(4)], 1).reshape(-1)
            self.gu_il = [(L.gu_Wq.index_select(0, perm.to(L.gu_Wq.device)).contiguous(),
                           L.gu_scale.index_select(0, perm).contiguous()) for L in w.layers]
        self.offload = offload
        self.overlap_copy = bool(overlap_copy) and offload
        if not offload:
            packed = [t for L in w.layers for t in (L.qkv_Wq, L.o_Wq, L.gu_Wq, L.down_Wq)]
            if any(t.device != dev for t in packed):
                raise ValueError("resident modes need every packed weight on the engine's device (use offload=True "
                                 "for weights in host memory)")
        if offload:
            self._setup_offload()
        self._x_final = self.x
        self._graph_layers = None
        self._graph_gen = None
        self._graph_gen_chunk = None  # GRAPH_CHUNK generation steps in one graph
        # eager runs only: called as layer_hook(l) after layer l's MLP has been issued (the MLP output is in
        # self.down; in DIP modes gate is in self.gu[:I] and the selection in self.idx / self.cnt, and the MLP
        # input in self.h except for the fused dense and dense-up schedules); never set while capture() runs
        self.layer_hook = None

    # ---- cache-aware DIP: hot rows in HBM, the rest in pinned host memory ----
    def _setup_cache(self, hot_channels):
        c, dev, k = self.c, self.device, self.k
        I = c.intermediate
        # one pinned arena for all layers' up and down^T rows, registered in the order the layers use them
        shapes = []
        for L in self.w.layers:
            shapes += [tuple(L.up(I)[0].shape), tuple(L.down_T_Wq.shape)]
        self.store = PinnedWeightStore(plan_bytes(shapes))
        self.caches, self.host_up, self.host_down, self.host_up_ptr, self.host_down_ptr = [], [], [], [], []
        for l, (L, hot) in enumerate(zip(self.w.layers, hot_channels)):
            up_Wq, up_s = L.up(I)
            hu = self.store.register(f"model.layers.{l}.mlp.up_proj.weight", up_Wq)
            hd_ = self.store.register(f"model.layers.{l}.mlp.down_proj_T.weight", L.down_T_Wq)
            self.host_up.append(self.store.matrix_view(hu))
            self.host_down.append(self.store.matrix_view(hd_))
            if up_Wq.is_cuda and L.down_T_Wq.is_cuda:
                self.caches.append(HotCache.build(up_Wq, up_s, L.down_T_Wq, L.down_T_scale, hot))
            else:  # weights in host memory: fill the cache from the pinned arena
                self.caches.append(HotCache.from_host(self.host_up[l], up_s, self.host_down[l], L.down_T_scale, hot,
                                                      device=dev))
            self.host_up_ptr.append(self.store.device_address(hu))
            self.host_down_ptr.append(self.store.device_address(hd_))
        row_up = self.w.layers[0].gu_Wq.shape[1]
        row_dn = self.w.layers[0].down_T_Wq.shape[1]
        G = self.w.layers[0].gu_scale.shape[1]
        u8, f32, i32 = torch.uint8, torch.float32, torch.int32
        self.desc = torch.zeros(k, dtype=i32, device=dev)
        self.miss_ch = torch.zeros(k, dtype=i32, device=dev)
        self.miss_cnt = torch.zeros(1, dtype=i32, device=dev)
        self.st_up = torch.zeros(k, row_up, dtype=u8, device=dev)
        self.st_dn = torch.zeros(k, row_dn, dtype=u8, device=dev)
        self.st_up_s = torch.zeros(k, G, dtype=f32, device=dev)
        self.st_dn_s = torch.zeros(k, G, dtype=f32, device=dev)

    # ---- offloaded dense weights: pinned arena, two device slots, one copy per layer ----
    def _streamed(self, l: int, L: LayerWeights) -> list:
        """(field, tensor) of the packed matrices layer l streams, in the order the layer uses them."""
        I = self.c.intermediate
        out = [("qkv_Wq", L.qkv_Wq), ("o_Wq", L.o_Wq)]
        if self.mode == "dense":
            out.append(("gu_il", self.gu_il[l][0]) if self.fused else ("gu_Wq", L.gu_Wq))
            out.append(("down_Wq", L.down_Wq))
        else:
            out.append(("gu_Wq", L.gu_Wq[:I]))  # gate rows; up / down^T rows come from the cache or host arena
        return out

    def _setup_offload(self):
        blocks = [self._streamed(l, L) for l, L in enumerate(self.w.layers)]
        shapes0 = [(name, tuple(t.shape)) for name, t in blocks[0]]
        if any([(name, tuple(t.shape)) for name, t in b] != shapes0 for b in blocks):
            raise ValueError("offload needs the same streamed matrix shapes in every layer (one slot layout)")
        self.wstore = PinnedWeightStore(plan_bytes(tuple(t.shape) for b in blocks for _, t in b))
        self._blocks = []  # per layer: (arena offset, bytes)
        for l, b in enumerate(blocks):
            first = None
            for name, t in b:
                h = self.wstore.register(f"model.layers.{l}.{name}", t.contiguous())
                first = h.offset if first is None else first
            self._blocks.append((first, self.wstore.bytes_used - first))
        nbytes = max(n for _, n in self._blocks)
        self.slots = [torch.empty(nbytes, dtype=torch.uint8, device=self.device) for _ in range(2)]
        # the views of a slot for each layer (same shapes every layer)
        self._slot_views = []
        for slot in self.slots:
            views, off = {}, 0
            for name, t in blocks[0]:
                n = t.numel()
                views[name] = slot[off:off + n].view(t.shape)
                off += n
            self._slot_views.append(views)
        if self.overlap_copy:
            self.copies = StreamManager(2, shared_stream=True)
            self._fork = torch.cuda.Event()
            self._step_open = False

    def _prefetch(self, l: int):
        off, n = self._blocks[l]
        self.copies.prefetch(l % 2, self.slots[l % 2][:n], self.wstore.arena[off:off + n])

    def _begin_step(self):
        """Overlapped offload: start a step's copies of layers 0 and 1. The copy streams first wait for an event
        of the current stream (everything before this point, the previous step included), so a captured step
        holds its copies as graph branches; the slots' read-done fences start over."""
        if not self.overlap_copy or self._step_open:
            return
        self._fork.record()
        for slot in self.copies.slots:
            slot.stream.wait_event(self._fork)  # (the slots share one stream: a repeated wait is harmless)
            slot.has_reader = False
        for l in range(min(2, self.c.layers)):
            self._prefetch(l)
        self._step_open = True

    def _layer_done(self, l: int):
        """Overlapped offload: layer l's kernels are issued; its slot takes layer l + 2's block once they finish."""
        if not self.overlap_copy:
            return
        self.copies.mark_read_done(l % 2)
        if l + 2 < self.c.layers:
            self._prefetch(l + 2)
        if l == self.c.layers - 1:
            self._step_open = False

    def _layer(self, l: int, L: LayerWeights):
        """Layer l's weights for this step. With offload, the layer's block from the pinned arena lands in slot
        l % 2 first (overlapped: the current stream waits for the copy started earlier; otherwise the copy is
        issued here, stream-ordered before the layer's kernels), and views of the slot come back with the
        resident scales and norms."""
        if not self.offload:
            return L, (self.gu_il[l] if hasattr(self, "gu_il") else None)
        off, n = self._blocks[l]
        if self.overlap_copy:
            self._begin_step()
            self.copies.wait(l % 2)
        else:
            self.slots[l % 2][:n].copy_(self.wstore.arena[off:off + n], non_blocking=True)
        v = self._slot_views[l % 2]
        Ls = LayerWeights(L.in_norm, L.post_norm, L.q_norm, L.k_norm, v["qkv_Wq"], L.qkv_scale, v["o_Wq"], L.o_scale,
                          v.get("gu_Wq", L.gu_Wq), L.gu_scale, v.get("down_Wq", L.down_Wq), L.down_scale,
                          L.down_T_Wq, L.down_T_scale)
        gu = (v["gu_il"], self.gu_il[l][1]) if "gu_il" in v else None
        return Ls, gu

    # ---- one layer ----
    def _mlp(self, l: int, L: LayerWeights):
        c = self.c
        H, I, gs = c.hidden, c.intermediate, c.group_size
        if self.mode == "dense":
            _C.gemv_w4a16_into(L.gu_Wq, L.gu_scale, self.h, self.gu, H, gs)
            _C.silu_mul_into(self.gu[:I], self.gu[I:], self.mlp_h)
            _C.gemv_w4a16_into(L.down_Wq, L.down_scale, self.mlp_h, self.down, I, gs)
            return
        gate = self.gu[:I]
        gW, gS = L.gate(I)
        _C.gemv_w4a16_into(gW, gS, self.h, gate, H, gs)
        if self.dip_dense_up:
            uW, uS = L.up(I)
            _C.gemv_w4a16_into(uW, uS, self.h, self.gu[I:], H, gs)
            _C.silu_mul_into(gate, self.gu[I:], self.mlp_h)  # h of every channel
            self._dense_down(l, gate, self.mlp_h)
            return
        if self.dip_gated:
            uW, uS = L.up(I)
            _C.gemv_w4a16_into(uW, uS, self.h, self.gu[I:], H, gs)
            if self.dip_gated_tr:
                _C.silu_mul_into(gate, self.gu[I:], self.mlp_h)  # h of every channel
                self._gated_down(l, L, gate, self.mlp_h)
            else:
                self._gated_down(l, L, gate, self.gu[I:])
            return
        _C.topk_threshold_select_f16abs_into(gate, self.k, self.idx, self.cnt)
        self._count_selection(l)
        if self.mode == "dip":
            uW, uS = L.up(I)
            _C.gemv_w4a16_indexed_into(uW, uS, self.idx, self.h, self.u_sel, H, gs)
            _C.silu_mul_indexed_into(gate, self.idx, self.u_sel, self.h_sel)
            _C.gemv_w4a16_indexed_accumulate_into(L.down_T_Wq, L.down_T_scale, self.idx, self.h_sel, self.down, H,
                                                  gs, self.sd_ws)
            return
        cache = self.caches[l]
        _, uS = L.up(I)
        if self.miss_path == "direct":
            _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, self.host_up[l], uS, cache.slot_of, self.idx,
                                       self.h, self.u_sel, H, gs)
            _C.silu_mul_indexed_into(gate, self.idx, self.u_sel, self.h_sel)
            _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, self.host_down[l], L.down_T_scale,
                                         cache.slot_of, self.idx, self.h_sel, self.down, H, gs, self.sd_ws)
            return
        self._fetch_misses(l, L, uS)
        _C.gemv_dip_fused_up_into(cache.up_Wq, cache.up_scale, self.st_up, self.st_up_s, self.desc, self.h,
                                  self.u_sel, H, gs)
        _C.silu_mul_indexed_into(gate, self.idx, self.u_sel, self.h_sel)
        _C.gemv_dip_fused_down_into(cache.down_Wq, cache.down_scale, self.st_dn, self.st_dn_s, self.desc,
                                    self.h_sel, self.down, H, gs, self.sd_ws)

    def _dense_down(self, l: int, gate: torch.Tensor, h: torch.Tensor, res: Optional[torch.Tensor] = None,
                    res_out: Optional[torch.Tensor] = None):
        """Selection + down of the dense-up schedule (h: fp16(silu(gate) * up) of every channel); the index list
        is written only for the eager consumers that read it (calibration counts, the layer hook). With res_out
        the launch also writes res + down there."""
        Wt, St = self.down_tt[l]
        want = self.counts is not None or self.layer_hook is not None
        _C.dip_select_dense_down_into(gate, h, self.k, Wt, St, self.idx if want else None,
                                      self.cnt if want else None, self.down, self.c.group_size,
                                      res if res_out is not None else None, res_out)
        self._count_selection(l)

    def _gated_down(self, l: int, L: LayerWeights, gate: torch.Tensor, hu: torch.Tensor,
                    res: Optional[torch.Tensor] = None, res_out: Optional[torch.Tensor] = None):
        """Selection + sparse down of the gated schedule. Over the transposed copy (hu = h of every channel) the
        index list is written only for the eager consumers that read it, and with res_out the launch also writes
        res + down there; over the selected rows (hu = up of every channel) h of the selected channels is formed
        on load, as the indexed up GEMV's SiLU epilogue rounds it."""
        c = self.c
        if self.dip_gated_tr:
            Wt, St = self.down_tt[l]
            want = self.counts is not None or self.layer_hook is not None
            _C.dip_select_down_ordered_into(gate, hu, self.k, Wt, St, self.idx if want else None,
                                            self.cnt if want else None, self.down, c.group_size,
                                            res if res_out is not None else None, res_out)
        else:
            assert res_out is None
            _C.dip_select_gated_down_into(gate, hu, self.k, L.down_T_Wq, L.down_T_scale, self.idx, self.cnt,
                                          self.down, c.hidden, c.group_size, self.sd_ws)
        self._count_selection(l)

    def _count_selection(self, l: int):
        """Calibration: add this layer's selected channels to its frequency counts."""
        if self.counts is not None:
            self.counts[l].index_add_(0, self.idx.long(), torch.ones(self.k, dtype=self.counts[l].dtype,
                                                                     device=self.device))

    def _fetch_misses(self, l: int, L: LayerWeights, uS: torch.Tensor):
        """Descriptors for this layer's selection, then the miss rows into staging: packed rows from pinned
        host memory (device gather through the host mapping), scale rows from HBM."""
        I = self.c.intermediate
        cache = self.caches[l]
        _C.build_dip_descriptors_into(self.idx, cache.slot_of, self.desc, self.miss_ch, self.miss_cnt)
        _C.gather_rows_device_counted(self.host_up_ptr[l], I, self.st_up.shape[1], self.miss_ch, self.miss_cnt,
                                      self.st_up)
        _C.gather_rows_device_counted(self.host_down_ptr[l], I, self.st_dn.shape[1], self.miss_ch, self.miss_cnt,
                                      self.st_dn)
        _C.gather_rows_device_counted(uS.data_ptr(), I, uS.shape[1] * 4, self.miss_ch, self.miss_cnt,
                                      self.st_up_s.view(torch.uint8))
        _C.gather_rows_device_counted(L.down_T_scale.data_ptr(), I, L.down_T_scale.shape[1] * 4, self.miss_ch,
                                      self.miss_cnt, self.st_dn_s.view(torch.uint8))

    def _layers(self):
        """Embedding of the device token, all layers at the device position, final norm; pos += 1."""
        if self.fused:
            self._layers_fused()
            return
        c, eps = self.c, self.c.rms_eps
        H, gs = c.hidden, c.group_size
        _C.embed_lookup_into(self.w.embed, self.token, self.x)
        for l, L in enumerate(self.w.layers):
            L, _ = self._layer(l, L)
            if l == 0:
                _C.rmsnorm_into(self.x, L.in_norm, self.h, eps)
            else:
                _C.residual_rmsnorm_(self.x, self.down, L.in_norm, self.h, eps)
            _C.gemv_w4a16_into(L.qkv_Wq, L.qkv_scale, self.h, self.qkv, H, gs)
            _C.qk_norm_rope_append(self.qkv, L.q_norm, L.k_norm, self.cos_t, self.sin_t, self.pos, self.q,
                                   self.k_cache[l], self.v_cache[l], eps)
            _C.decode_attention_at(self.q, self.k_cache[l], self.v_cache[l], self.pos, self.attn, self.attn_ws)
            _C.gemv_w4a16_into(L.o_Wq, L.o_scale, self.attn, self.o, c.q_heads * c.head_dim, gs)
            _C.residual_rmsnorm_(self.x, self.o, L.post_norm, self.h, eps)
            self._mlp(l, L)
            self._layer_done(l)
            if self.layer_hook is not None:
                self.layer_hook(l)
        _C.residual_rmsnorm_(self.x, self.down, self.w.final_norm, self.hn, eps)
        self._x_final = self.x
        _C.advance_position(self.pos, 1)

    def _layers_fused(self):
        """Same computation with the RMSNorm done inside the following GEMV (the residual stream alternates
        between two buffers), the SiLU gating in the up / gate|up GEMV epilogue and, with residual_epilogue,
        the residual adds in the producers' epilogues (the o projection, and the down projection of the dense
        and dense-up schedules, write residual + output into the other buffer); otherwise the consumer adds
        on load (reads residual and delta, writes the sum for the next add)."""
        c, eps = self.c, self.c.rms_eps
        H, gs = c.hidden, c.group_size
        cur, other = self.x, self.x2
        fold = self.residual_epilogue
        # the down launch writes the residual
        down_res = fold and (self.mode == "dense" or self.dip_dense_up or self.dip_gated_tr)
        last = len(self.w.layers) - 1
        _C.embed_lookup_into(self.w.embed, self.token, cur)
        for l, L in enumerate(self.w.layers):
            L, gu_il = self._layer(l, L)
            if l == 0 or down_res:
                _C.gemv_w4a16_rmsnorm_into(L.qkv_Wq, L.qkv_scale, cur, None, L.in_norm, eps, None, None, self.qkv,
                                           H, gs, False)
            else:
                _C.gemv_w4a16_rmsnorm_into(L.qkv_Wq, L.qkv_scale, cur, self.down, L.in_norm, eps, other, None,
                                           self.qkv, H, gs, False)
                cur, other = other, cur
            attn = self.attn.view(c.q_heads, c.head_dim)
            if self.step_ws is not None:
                step = _C.decode_attention_step_deferred if self.defer_combine else _C.decode_attention_step
                step(self.qkv, L.q_norm, L.k_norm, self.cos_t, self.sin_t, self.pos, self.k_cache[l],
                     self.v_cache[l], attn, eps, self.step_ws)
            else:
                _C.qk_norm_rope_append(self.qkv, L.q_norm, L.k_norm, self.cos_t, self.sin_t, self.pos, self.q,
                                       self.k_cache[l], self.v_cache[l], eps)
                _C.decode_attention_at(self.q, self.k_cache[l], self.v_cache[l], self.pos, self.attn, self.attn_ws)
            K_o = c.q_heads * c.head_dim
            res = (cur, other) if fold else (None, None)
            if self.defer_combine:
                _C.gemv_w4a16_attn_combine_into(L.o_Wq, L.o_scale, self.step_ws, attn, self.pos, c.kv_heads,
                                                c.max_seq, self.o, gs, *res)
            elif fold:
                _C.gemv_w4a16_residual_into(L.o_Wq, L.o_scale, self.attn, self.o, cur, other, K_o, gs)
            else:
                _C.gemv_w4a16_into(L.o_Wq, L.o_scale, self.attn, self.o, K_o, gs)
            if fold:
                cur, other = other, cur
                self._mlp_fused(l, L, gu_il, cur, None, None, other if down_res and l < last else None)
            else:
                self._mlp_fused(l, L, gu_il, cur, self.o, other, None)
            self._layer_done(l)
            if not fold or (down_res and l < last):
                cur, other = other, cur
            if self.layer_hook is not None:
                self.layer_hook(l)
        _C.final_norm_advance(cur, self.down, self.w.final_norm, self.hn, eps, self.pos)
        self._x_final = cur

    def _mlp_fused(self, l: int, L: LayerWeights, gu_il, x: torch.Tensor, delta: Optional[torch.Tensor],
                   x_out: Optional[torch.Tensor], res_out: Optional[torch.Tensor]):
        """Layer l's MLP on the residual x (+ delta, the sum written to x_out, when given) with the RMSNorm on
        load; the output lands in self.down. With res_out (dense and dense-up schedules only, no delta) the
        down launch also writes x + down there."""
        c, eps = self.c, self.c.rms_eps
        H, I, gs = c.hidden, c.intermediate, c.group_size
        if self.mode == "dense":
            gW, gS = gu_il
            _C.gemv_w4a16_rmsnorm_into(gW, gS, x, delta, L.post_norm, eps, x_out, None, self.mlp_h, H, gs, True)
            if res_out is not None:
                _C.gemv_w4a16_residual_into(L.down_Wq, L.down_scale, self.mlp_h, self.down, x, res_out, I, gs)
            else:
                _C.gemv_w4a16_into(L.down_Wq, L.down_scale, self.mlp_h, self.down, I, gs)
            return
        gate = self.gu[:I]
        if self.dip_dense_up:
            gW, gS = gu_il
            _C.gemv_w4a16_rmsnorm_swiglu_gate_into(gW, gS, x, delta, L.post_norm, eps, x_out, gate, self.gu[I:],
                                                   H, gs)
            self._dense_down(l, gate, self.gu[I:], x, res_out)
            return
        if self.dip_gated:
            gW, gS = gu_il
            if self.dip_gated_tr:  # gate and h of every channel, as the dense-up schedule's first launch
                _C.gemv_w4a16_rmsnorm_swiglu_gate_into(gW, gS, x, delta, L.post_norm, eps, x_out, gate,
                                                       self.gu[I:], H, gs)
            else:  # gate and up of every channel
                _C.gemv_w4a16_rmsnorm_gate_up_into(gW, gS, x, delta, L.post_norm, eps, x_out, gate, self.gu[I:],
                                                   H, gs)
            self._gated_down(l, L, gate, self.gu[I:], x, res_out)
            return
        assert res_out is None
        gW, gS = L.gate(I)
        _C.gemv_w4a16_rmsnorm_into(gW, gS, x, delta, L.post_norm, eps, x_out, self.h, gate, H, gs, False)
        _C.topk_threshold_select_f16abs_into(gate, self.k, self.idx, self.cnt)
        self._count_selection(l)
        uW, uS = L.up(I)
        if self.mode == "dip":
            _C.gemv_w4a16_indexed_silu_into(uW, uS, self.idx, self.h, gate, self.h_sel, H, gs)
            _C.gemv_w4a16_indexed_accumulate_into(L.down_T_Wq, L.down_T_scale, self.idx, self.h_sel, self.down,
                                                  H, gs, self.sd_ws)
            return
        cache = self.caches[l]
        if self.miss_path == "direct":
            # the up GEMV's waves also copy their down^T miss rows to staging (whole-row PCIe reads, overlapped
            # with the up rows); the down accumulate then reads hits from the cache and misses from staging
            cp = (self.host_down[l], self.st_dn) if self.down_copy else (None, None)
            _C.gemv_dip_cached_up_silu_into(cache.up_Wq, cache.up_scale, self.host_up[l], uS, cache.slot_of,
                                            self.idx, self.h, gate, self.h_sel, H, gs, *cp)
            _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, self.host_down[l], L.down_T_scale,
                                         cache.slot_of, self.idx, self.h_sel, self.down, H, gs, self.sd_ws,
                                         self.st_dn if self.down_copy else None)
            return
        self._fetch_misses(l, L, uS)
        _C.gemv_dip_fused_up_silu_into(cache.up_Wq, cache.up_scale, self.st_up, self.st_up_s, self.desc,
                                       self.idx, self.h, gate, self.h_sel, H, gs)
        _C.gemv_dip_fused_down_into(cache.down_Wq, cache.down_scale, self.st_dn, self.st_dn_s, self.desc,
                                    self.h_sel, self.down, H, gs, self.sd_ws)

    @property
    def x_final(self) -> torch.Tensor:
        """The residual stream after the last layer of the latest step."""
        return self._x_final

    def _head(self):
        """LM head on the final-normed hidden state and argmax into the device token (and the log)."""
        if self.head_q is not None:
            _C.gemv_w4a16_into(self.head_q[0], self.head_q[1], self.hn, self.logits, self.c.hidden,
                               self.c.group_size)
        else:
            _C.gemv_f16_into(self.w.lm_head, self.hn, self.logits)
        _C.argmax_f16_into(self.logits, self.token, self.log, self.log_len, self.argmax_ws)

    def _gen_step(self):
        """One generation step: LM head + argmax of the previous step, then the layers (an overlapped offload
        starts the copies of layers 0 and 1 first, so they run under the head)."""
        if self.offload:
            self._begin_step()
        self._head()
        self._layers()

    # ---- graphs ----
    def capture(self):
        """Capture the prompt step (layers), the generation step (head + layers) and GRAPH_CHUNK generation steps
        in a row as HIP graphs (the chunk graph saves a graph boundary per step: about 5 us, 0.7% of a token of the
        Qwen3-1.7B shape, measured)."""
        saved = (self.pos.clone(), self.log_len.clone(), self.token.clone())
        self._step_open = False  # a step's copies always start inside the step that uses them
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):  # warm up outside capture (first-launch costs)
            self._layers()
            self._gen_step()
        torch.cuda.current_stream(self.device).wait_stream(s)
        torch.cuda.synchronize(self.device)
        self._graph_layers = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph_layers):
            self._layers()
        self._graph_gen = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph_gen):
            self._gen_step()
        self._graph_gen_chunk = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self._graph_gen_chunk):
            for _ in range(GRAPH_CHUNK):
                self._gen_step()
        self.pos.copy_(saved[0])
        self.log_len.copy_(saved[1])
        self.token.copy_(saved[2])
        torch.cuda.synchronize(self.device)

    def reset(self):
        self.pos.zero_()
        self.log_len.zero_()
        self._step_open = False

    def prefill(self, prompt_ids, use_graph: bool = True):
        prompt = torch.as_tensor(list(prompt_ids), dtype=torch.int32, device=self.device)
        if prompt.numel() + 1 > self.c.max_seq:
            raise ValueError("prompt longer than the KV cache")
        for i in range(prompt.numel()):
            self.token.copy_(prompt[i:i + 1])
            if use_graph:
                self._graph_layers.replay()
            else:
                self._layers()

    def decode(self, n_new: int, use_graph: bool = True):
        if n_new > self.log.numel():
            raise ValueError("n_new exceeds max_new_tokens")
        if not use_graph:
            for _ in range(n_new):
                self._gen_step()
            return
        for _ in range(n_new // GRAPH_CHUNK):
            self._graph_gen_chunk.replay()
        for _ in range(n_new % GRAPH_CHUNK):
            self._graph_gen.replay()

    def generate(self, prompt_ids, n_new: int, use_graph: bool = True, eos_token_id: Optional[int] = None):
        """Greedy decoding: returns prompt_ids + the n_new generated tokens (cut after eos_token_id, as the
        reference's early stop; the device loop runs all n_new steps and the host truncates)."""
        if len(prompt_ids) + n_new > self.c.max_seq:
            raise ValueError("prompt + new tokens exceed the KV cache length")
        if use_graph and self._graph_gen is None:
            self.capture()
        self.reset()
        self.prefill(prompt_ids, use_graph)
        self.decode(n_new, use_graph)
        out = self.log[:n_new].tolist()
        if eos_token_id is not None and eos_token_id in out:
            out = out[:out.index(eos_token_id) + 1]
        return list(prompt_ids) + out


def calibrate_channel_counts(w: DecoderWeights, dip_k: int, calib_tokens) -> list:
    """Per layer, counts[c] = how many of the calib_tokens steps selected channel c, feeding the tokens one at a
    time through the DIP engine (eagerly) as the reference's calibrate_channel_frequencies does
    (generate.py:579-609). int64 [I] tensors on the engine's device; each sums to len(calib_tokens) * dip_k."""
    c = w.config
    eng = DecodeEngine(w, "dip", dip_k=dip_k, max_new_tokens=1)
    eng.counts = [torch.zeros(c.intermediate, dtype=torch.int64, device=eng.device) for _ in range(c.layers)]
    eng.reset()
    eng.prefill(calib_tokens, use_graph=False)
    counts = eng.counts
    del eng
    return counts


def calibrate_hot_channels(w: DecoderWeights, dip_k: int, calib_tokens, cache_fraction: float = 0.2):
    """Hot set per layer: the cache_fraction * I most frequently selected channels (ties to the lower index)
    while decoding calib_tokens with the DIP engine (calibrate_channel_counts; StaticFrequencyPolicy orders
    them, hot_cache.py:67-95 of the reference)."""
    from ..offload.hot_cache import StaticFrequencyPolicy

    C = int(round(cache_fraction * w.config.intermediate))
    return [StaticFrequencyPolicy(cnt.cpu(), C).hot_indices.tolist()
            for cnt in calibrate_channel_counts(w, dip_k, calib_tokens)]
