"""CPU restatement of the reference's batch-1 decode step (numpy, binary64 arithmetic).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the HIP decode
glue and the decode engine. The product never imports it.

Follows python/soinfer/runtime/generate.py of the reference:
  * layer (run_decoder_layer_streaming :141-182): rmsnorm -> q/k/v GEMVs ->
    per-head qk_norm -> RoPE (rotate-half, precompute_rope_cos_sin of
    python/soinfer/ops.py:222-227) -> KV append -> decode attention -> o GEMV
    -> residual add -> rmsnorm -> gate/up GEMVs -> fp16(silu(gate) * up) ->
    down GEMV -> residual add;
  * DIP MLP (run_decoder_layer_dip :276-310): gate GEMV, top-k rule A over
    |gate| as fp32, up GEMV over the selected rows, fp16(silu(gate[idx]) * u),
    sparse down accumulate over the selected rows of down^T;
  * generation (generate_streaming :429-463): prompt tokens one at a time,
    then final rmsnorm -> fp16 LM head GEMV -> argmax (first maximum).
Kernels restated: rmsnorm.cu:9-48 (x * rsqrt(mean(x^2) + eps) * w),
rope.cu:5-25, kv_cache.cu:7-27, gemv_fp16.cu:60-95, swiglu_fused.cu:15-51. Every op rounds its
output to binary16, as the reference's ops do; the arithmetic inside an op is
binary64 here (the reference's is fp32), so results agree to the fp16
rounding of each op, not bit for bit.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import oracle as O


def f16(a) -> np.ndarray:
    """Round binary64 values to binary16 (correctly rounded)."""
    return O.f64_to_f16(np.asarray(a, np.float64))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """rmsnorm.cu:9-48 per row of the last axis: fp16(x * 1/sqrt(mean(x^2) + eps) * w)."""
    v = np.asarray(x, np.float64)
    inv = 1.0 / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + eps)
    return f16(v * inv * np.asarray(w, np.float64))


def residual_add(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """binary16 a + b (generate.py:172 / :182)."""
    return f16(np.asarray(a, np.float64) + np.asarray(b, np.float64))


def rope_angles(head_dim: int, theta: float, pos: int) -> np.ndarray:
    """fp32 angles pos * inv_freq, inv_freq[i] = 1 / theta^(2i/head_dim) (ops.py:222-227)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.float32) / np.float32(head_dim)
    inv_freq = (np.float32(1.0) / (np.float32(theta) ** exponent)).astype(np.float32)
    return (np.float32(pos) * inv_freq).astype(np.float32)


def rope(x: np.ndarray, head_dim: int, theta: float, pos: int) -> np.ndarray:
    """rope.cu:5-25, rotate-half: [x1 c - x2 s, x2 c + x1 s] per head, fp16 out."""
    ang = rope_angles(head_dim, theta, pos).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    v = np.asarray(x, np.float64)
    half = head_dim // 2
    x1, x2 = v[..., :half], v[..., half:]
    return f16(np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1))


def silu(t: np.ndarray) -> np.ndarray:
    t = np.asarray(t, np.float64)
    return t / (1.0 + np.exp(-t))


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """fp16(silu(fp32 gate) * fp32 up) (generate.py:178, :304-305)."""
    return f16(silu(gate) * np.asarray(up, np.float64))


def gemv_f16(W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """gemv_fp16.cu:60-95 (the LM head): fp16(W @ x)."""
    return f16(np.asarray(W, np.float64) @ np.asarray(x, np.float64))


def swiglu_gate_up(gate_W: np.ndarray, up_W: np.ndarray, x: np.ndarray) -> np.ndarray:
    """swiglu_fused.cu:15-51 (ops.py:112-116): fp16(silu(gate_W @ x) * (up_W @ x)), silu on the unrounded gate
    sum (the kernel keeps both sums in fp32 and rounds only h)."""
    xd = np.asarray(x, np.float64)
    g = np.asarray(gate_W, np.float64) @ xd
    u = np.asarray(up_W, np.float64) @ xd
    return f16(silu(g) * u)


def argmax_first(v: np.ndarray) -> int:
    """torch.argmax order on a 1-D fp16 vector: NaN first, then the largest value, lowest index on ties."""
    v = np.asarray(v, np.float64)
    nan = np.flatnonzero(np.isnan(v))
    if nan.size:
        return int(nan[0])
    return int(np.flatnonzero(v == v.max())[0])


def int4_gemv(Wq: np.ndarray, scale: np.ndarray, x: np.ndarray, gs: int) -> np.ndarray:
    K = Wq.shape[1] * 2
    return f16(O.gemv_w4_f64(Wq, scale, np.asarray(x, np.float16), K, gs))


@dataclass
class OracleLayer:
    in_norm: np.ndarray
    post_norm: np.ndarray
    q_norm: np.ndarray
    k_norm: np.ndarray
    qkv_Wq: np.ndarray
    qkv_scale: np.ndarray
    o_Wq: np.ndarray
    o_scale: np.ndarray
    gu_Wq: np.ndarray
    gu_scale: np.ndarray
    down_Wq: np.ndarray
    down_scale: np.ndarray
    down_T_Wq: np.ndarray
    down_T_scale: np.ndarray


class OracleDecoder:
    """Greedy decoder over numpy copies of the weights; mode "dense" or "dip" (rule-A top-k of dip_k).
    lm_head_int4 = (packed rows, fp32 scales): the LM head as an INT4 group GEMV instead of the fp16 one."""

    def __init__(self, cfg, embed, lm_head, final_norm, layers, mode="dense", dip_k=None, lm_head_int4=None):
        self.c, self.embed, self.lm_head, self.final_norm, self.layers = cfg, embed, lm_head, final_norm, layers
        self.mode, self.k = mode, dip_k
        self.lm_head_int4 = lm_head_int4
        c = cfg
        self.kc = [np.zeros((c.kv_heads, c.max_seq, c.head_dim), np.float16) for _ in range(c.layers)]
        self.vc = [np.zeros((c.kv_heads, c.max_seq, c.head_dim), np.float16) for _ in range(c.layers)]
        self.pos = 0
        self.x = None

    def _mlp(self, L: OracleLayer, h3: np.ndarray) -> np.ndarray:
        c = self.c
        I, H, gs = c.intermediate, c.hidden, c.group_size
        if self.mode == "dense":
            gu = int4_gemv(L.gu_Wq, L.gu_scale, h3, gs)
            m = silu_mul(gu[:I], gu[I:])
            return int4_gemv(L.down_Wq, L.down_scale, m, gs)
        gate = int4_gemv(L.gu_Wq[:I], L.gu_scale[:I], h3, gs)
        idx = O.topk_rule_a(np.abs(gate.astype(np.float32)), self.k)
        u = int4_gemv(L.gu_Wq[I:][idx], L.gu_scale[I:][idx], h3, gs)
        hs = silu_mul(gate[idx], u)
        return f16(O.sparse_accumulate_f64(L.down_T_Wq[idx], L.down_T_scale[idx], hs, H, gs))

    def layer(self, l: int, x: np.ndarray) -> np.ndarray:
        c, L, pos = self.c, self.layers[l], self.pos
        NQ, NKV, hd, eps = c.q_heads, c.kv_heads, c.head_dim, c.rms_eps
        h = rmsnorm(x, L.in_norm, eps)
        qkv = int4_gemv(L.qkv_Wq, L.qkv_scale, h, c.group_size)
        q = qkv[:NQ * hd].reshape(NQ, hd)
        k = qkv[NQ * hd:(NQ + NKV) * hd].reshape(NKV, hd)
        v = qkv[(NQ + NKV) * hd:].reshape(NKV, hd)
        q = rope(rmsnorm(q, L.q_norm, eps), hd, c.rope_theta, pos)
        k = rope(rmsnorm(k, L.k_norm, eps), hd, c.rope_theta, pos)
        self.kc[l][:, pos, :] = k
        self.vc[l][:, pos, :] = v
        a = f16(O.decode_attention_f64(q, self.kc[l], self.vc[l], pos + 1)).reshape(-1)
        o = int4_gemv(L.o_Wq, L.o_scale, a, c.group_size)
        x2 = residual_add(x, o)
        h3 = rmsnorm(x2, L.post_norm, eps)
        return residual_add(x2, self._mlp(L, h3))

    def step(self, token: int) -> None:
        x = np.asarray(self.embed[token], np.float16)
        for l in range(self.c.layers):
            x = self.layer(l, x)
        self.x = x
        self.pos += 1

    def logits(self) -> np.ndarray:
        xn = rmsnorm(self.x, self.final_norm, self.c.rms_eps)
        if self.lm_head_int4 is not None:
            return int4_gemv(self.lm_head_int4[0], self.lm_head_int4[1], xn, self.c.group_size)
        return gemv_f16(self.lm_head, xn)


def from_device(weights) -> tuple:
    """numpy copies (embed, lm_head, final_norm, [OracleLayer]) of soinfer DecoderWeights."""
    def np_(t):
        return t.detach().cpu().numpy()

    layers = [OracleLayer(*(np_(getattr(L, f)) for f in OracleLayer.__dataclass_fields__)) for L in weights.layers]
    return np_(weights.embed), np_(weights.lm_head), np_(weights.final_norm), layers
