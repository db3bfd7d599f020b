"""Decoder parity against an implementation outside this repository: Hugging Face transformers' Qwen3 model
(`Qwen3ForCausalLM`, binary64 on the CPU) with the dequantized INT4 weights fl(q * s) of the same decoder.
The reference checks its own decoder against this model the same way (tests/test_layer_parity.py:90-119,
tests/test_end_to_end.py:120-132 of the reference; there with checkpoints, here with random weights).

* the oracle decoder (oracle/decoder.py, the CPU restatement of generate.py's layer order with the kernels'
  binary16 rounding points) on a random INT4 model quantized by the reference's quantizer (CPU, no GPU);
* the GPU decode engine (dense, and gated DIP at k = I, which selects every channel and so is the dense model
  with the down projection taken from the separately quantized down_proj^T) on its own random weights (GPU).

Both step through a 6-token prompt and 6 generated tokens, teacher-forced on the tested decoder's tokens: the
logits within 1e-2 of max|logit| of transformers' (half the reference's HF bound, its layer parity test's
`max rel err < 2e-2`; the difference is the binary16 rounding of every activation here against binary64 there,
about 1e-3 on this model, while swapping the q and k norm weights moves the oracle's logits by 3-5e-2 and a RoPE
position off by one by 0.15), and the same greedy token wherever transformers' top-2 margin exceeds twice that
bound; the GPU engines also over a 300-token prompt and 4 generated tokens (split attention), on two layers
of the Qwen3-1.7B shape, and with every weight INT4 g128, the LM head included (int4_head). transformers is in
this image; the tests skip where it is not importable.
"""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import decoder as OD
from oracle import oracle as O

TOL = 1e-2
TINY = dict(hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
            group_size=128, max_seq=64, rms_eps=1e-6, rope_theta=1_000_000.0)
# head size 128 (one rotation pair per lane in the attention step, the Qwen3 path), 2 query heads per KV head
WIDE = dict(hidden=512, layers=2, q_heads=8, kv_heads=4, head_dim=128, intermediate=1024, vocab=2000,
            group_size=128, max_seq=64, rms_eps=1e-6, rope_theta=1_000_000.0)
# one KV head shared by 4 query heads, 64-element quantization groups, a hidden size that is not a power of two
GQA4 = dict(hidden=384, layers=2, q_heads=4, kv_heads=1, head_dim=128, intermediate=768, vocab=1500,
            group_size=64, max_seq=64, rms_eps=1e-6, rope_theta=1_000_000.0)
CONFIGS = {"tiny": TINY, "hd128": WIDE, "gqa4_g64": GQA4}


def _hf_model(c, embed, lm_head, final_norm, layers, down_from_transposed=False):
    """transformers' Qwen3 with the dequantized weights; down_from_transposed: the down projection from the
    separately quantized down_proj^T that the DIP schedules read (its groups run along the hidden size, so its
    values differ from down_proj's by the INT4 rounding)."""
    tr = pytest.importorskip("transformers")
    cfg = tr.Qwen3Config(vocab_size=c.vocab, hidden_size=c.hidden, intermediate_size=c.intermediate,
                         num_hidden_layers=c.layers, num_attention_heads=c.q_heads, num_key_value_heads=c.kv_heads,
                         head_dim=c.head_dim, rms_norm_eps=c.rms_eps, rope_theta=c.rope_theta,
                         max_position_embeddings=c.max_seq, tie_word_embeddings=False, attention_bias=False,
                         hidden_act="silu")
    model = tr.Qwen3ForCausalLM(cfg).to(torch.float64).eval()
    H, I, gs = c.hidden, c.intermediate, c.group_size
    nq, nkv = c.q_heads * c.head_dim, c.kv_heads * c.head_dim

    def t(a):
        return torch.from_numpy(np.asarray(a, np.float64))

    def dq(Wq, s, K):
        return t(O.dequant_int4(Wq, s, K, gs))

    sd = {"model.embed_tokens.weight": t(embed), "lm_head.weight": t(lm_head), "model.norm.weight": t(final_norm)}
    for l, L in enumerate(layers):
        p = f"model.layers.{l}."
        qkv = dq(L.qkv_Wq, L.qkv_scale, H)
        gu = dq(L.gu_Wq, L.gu_scale, H)
        sd.update({
            p + "self_attn.q_proj.weight": qkv[:nq], p + "self_attn.k_proj.weight": qkv[nq:nq + nkv],
            p + "self_attn.v_proj.weight": qkv[nq + nkv:], p + "self_attn.o_proj.weight": dq(L.o_Wq, L.o_scale, nq),
            p + "self_attn.q_norm.weight": t(L.q_norm), p + "self_attn.k_norm.weight": t(L.k_norm),
            p + "mlp.gate_proj.weight": gu[:I], p + "mlp.up_proj.weight": gu[I:],
            p + "mlp.down_proj.weight": (dq(L.down_T_Wq, L.down_T_scale, H).T.contiguous() if down_from_transposed
                                         else dq(L.down_Wq, L.down_scale, I)),
            p + "input_layernorm.weight": t(L.in_norm), p + "post_attention_layernorm.weight": t(L.post_norm),
        })
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not unexpected and all("rotary" in m for m in missing), (missing, unexpected)
    return model


def _hf_logits(model, seq):
    with torch.no_grad():
        return model(input_ids=torch.tensor([seq])).logits[0, -1].numpy()


def _compare(label, step, ours, ref, tok):
    scale = np.abs(ref).max()
    err = np.abs(np.asarray(ours, np.float64) - ref).max()
    assert err <= TOL * scale, f"{label} step {step}: logits {err / scale:.2e} of max|logit| from transformers'"
    srt = np.sort(ref)
    if srt[-1] - srt[-2] > 2 * TOL * scale:
        assert tok == int(np.argmax(ref)), f"{label} step {step}: token {tok} != transformers' {int(np.argmax(ref))}"


def _prompt(n, vocab, seed=7):
    return np.random.default_rng(seed).integers(0, vocab, n).tolist()


def _random_oracle_model(c, seed):
    """Random fp32 weights quantized by the reference's quantizer (INT4 g128, AWQ packing)."""
    r = np.random.default_rng(seed)
    H, I, hd, gs = c.hidden, c.intermediate, c.head_dim, c.group_size

    def lin(N, K, std=0.05):
        q, s = O.quantize_group(r.standard_normal((N, K)).astype(np.float32) * np.float32(std), gs)
        return O.pack_int4(q), s

    def norm(n):
        return (1.0 + 0.1 * r.standard_normal(n)).astype(np.float16)

    layers = []
    for _ in range(c.layers):
        qkv, o = lin((c.q_heads + 2 * c.kv_heads) * hd, H), lin(H, c.q_heads * hd)
        gu, down = lin(2 * I, H), lin(H, I)
        layers.append(OD.OracleLayer(norm(H), norm(H), norm(hd), norm(hd), *qkv, *o, *gu, *down, *down))
    embed = (r.standard_normal((c.vocab, H)) * 0.5).astype(np.float16)
    lm_head = (r.standard_normal((c.vocab, H)) * 0.05).astype(np.float16)
    return embed, lm_head, norm(H), layers


@pytest.mark.parametrize("name", list(CONFIGS))
def test_oracle_decoder_matches_transformers(name):
    c = SimpleNamespace(**CONFIGS[name])
    embed, lm_head, final_norm, layers = _random_oracle_model(c, seed=5)
    model = _hf_model(c, embed, lm_head, final_norm, layers)
    ora = OD.OracleDecoder(c, embed, lm_head, final_norm, layers)
    seq = _prompt(6, c.vocab)
    for t in seq:
        ora.step(t)
    for i in range(6):
        ours = ora.logits()
        tok = OD.argmax_first(ours)
        _compare(f"oracle {name}", i, ours, _hf_logits(model, seq), tok)
        seq.append(tok)
        ora.step(tok)


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(CONFIGS))
@pytest.mark.parametrize("mode", ["dense", "gated"])
def test_engine_matches_transformers(cuda, mode, name):
    from soinfer.runtime import decoder as dec

    cfg = dec.DecoderConfig(**CONFIGS[name])
    w = dec.random_decoder(cfg, seed=3, linear_std=0.05, norm_jitter=0.1)
    embed, lm_head, final_norm, layers = OD.from_device(w)
    model = _hf_model(cfg, embed, lm_head, final_norm, layers, down_from_transposed=mode != "dense")
    if mode == "dense":
        eng = dec.DecodeEngine(w, "dense", max_new_tokens=6)
    else:  # k = I: every channel selected, the MLP of the dense model summed in the sparse down's order
        eng = dec.DecodeEngine(w, "dip", dip_k=cfg.intermediate, max_new_tokens=6, dip_schedule="gated")
    eng.reset()
    seq = _prompt(6, cfg.vocab)
    eng.prefill(seq, use_graph=False)
    for i in range(6):
        eng._head()
        tok = int(eng.token.item())
        _compare(f"engine {mode} {name}", i, eng.logits.float().cpu().numpy(), _hf_logits(model, seq), tok)
        seq.append(tok)
        eng._layers()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["dense", "gated"])
def test_engine_long_context_matches_transformers(cuda, mode):
    """A 300-token prompt (past one attention workgroup's rows, so the attention step splits the context and
    combines the splits) and 4 generated tokens on the head-size-128 model, by the same bound."""
    from soinfer.runtime import decoder as dec

    cfg = dec.DecoderConfig(**dict(WIDE, max_seq=320))
    w = dec.random_decoder(cfg, seed=13, linear_std=0.05, norm_jitter=0.1)
    embed, lm_head, final_norm, layers = OD.from_device(w)
    model = _hf_model(cfg, embed, lm_head, final_norm, layers, down_from_transposed=mode != "dense")
    if mode == "dense":
        eng = dec.DecodeEngine(w, "dense", max_new_tokens=4)
    else:
        eng = dec.DecodeEngine(w, "dip", dip_k=cfg.intermediate, max_new_tokens=4, dip_schedule="gated")
    eng.reset()
    seq = _prompt(300, cfg.vocab, seed=17)
    eng.prefill(seq, use_graph=False)
    for i in range(4):
        eng._head()
        tok = int(eng.token.item())
        _compare(f"engine {mode} long context", i, eng.logits.float().cpu().numpy(), _hf_logits(model, seq), tok)
        seq.append(tok)
        eng._layers()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["dense", "gated"])
def test_engine_qwen3_1p7b_width_matches_transformers(cuda, mode):
    """Two layers of the Qwen3-1.7B shape (hidden 2048, intermediate 6144, 16 query / 8 KV heads of 128, INT4 g128)
    with a 4096-token vocabulary: 6 prompt + 6 generated tokens, by the same bound."""
    from soinfer.runtime import decoder as dec

    cfg = dec.DecoderConfig(hidden=2048, layers=2, q_heads=16, kv_heads=8, head_dim=128, intermediate=6144,
                            vocab=4096, group_size=128, max_seq=64, rms_eps=1e-6, rope_theta=1_000_000.0)
    w = dec.random_decoder(cfg, seed=19, linear_std=0.03, norm_jitter=0.1)
    embed, lm_head, final_norm, layers = OD.from_device(w)
    model = _hf_model(cfg, embed, lm_head, final_norm, layers, down_from_transposed=mode != "dense")
    if mode == "dense":
        eng = dec.DecodeEngine(w, "dense", max_new_tokens=6)
    else:
        eng = dec.DecodeEngine(w, "dip", dip_k=cfg.intermediate, max_new_tokens=6, dip_schedule="gated")
    eng.reset()
    seq = _prompt(6, cfg.vocab, seed=21)
    eng.prefill(seq, use_graph=False)
    for i in range(6):
        eng._head()
        tok = int(eng.token.item())
        _compare(f"engine {mode} 1.7B width", i, eng.logits.float().cpu().numpy(), _hf_logits(model, seq), tok)
        seq.append(tok)
        eng._layers()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["dense", "gated"])
def test_engine_int4_head_matches_transformers(cuda, mode):
    """Every weight INT4 g128, the LM head included (int4_head=True): transformers' lm_head is the dequantized
    INT4 head the engine reads; head-size-128 model, 6 prompt + 6 generated tokens, by the same bound."""
    from soinfer.runtime import decoder as dec

    cfg = dec.DecoderConfig(**WIDE)
    w = dec.random_decoder(cfg, seed=23, linear_std=0.05, norm_jitter=0.1)
    kw = dict(int4_head=True, max_new_tokens=6)
    eng = (dec.DecodeEngine(w, "dense", **kw) if mode == "dense"
           else dec.DecodeEngine(w, "dip", dip_k=cfg.intermediate, dip_schedule="gated", **kw))
    hq, hs = (t.cpu().numpy() for t in dec.quantize_lm_head(w))
    embed, _, final_norm, layers = OD.from_device(w)
    head = O.dequant_int4(hq, hs, cfg.hidden, cfg.group_size)
    model = _hf_model(cfg, embed, head, final_norm, layers, down_from_transposed=mode != "dense")
    eng.reset()
    seq = _prompt(6, cfg.vocab, seed=25)
    eng.prefill(seq, use_graph=False)
    for i in range(6):
        eng._head()
        tok = int(eng.token.item())
        _compare(f"engine {mode} INT4 head", i, eng.logits.float().cpu().numpy(), _hf_logits(model, seq), tok)
        seq.append(tok)
        eng._layers()
