"""The decode engine on other Qwen3 shapes, two layers each and a 4096-token vocabulary (the head is not what is
tested here):

  Qwen3-0.6B  hidden 1024, I 3072,  16 query / 8 KV heads of 128
  Qwen3-4B    hidden 2560, I 9728,  32 / 8 heads (the o projection's K = 4096 is past the deferred attention
              combine's limit, so the attention launch combines its own splits)
  Qwen3-8B    hidden 4096, I 12288, 32 / 8 heads

* dense logits against the oracle decoder for 3 prompt + 3 new tokens, by the tolerance rule of
  tests/test_decode_engine_gpu.py;
* DIP (k = I/2), the first generated step teacher-forced layer by layer, as tests/test_decode_full_shape_gpu.py
  does at the 1.7B shape: the gate within the tolerance of tests/helpers.py of the binary64 oracle GEMV on the
  layer's own MLP input, the selection equal to the oracle's rule A on the kernel's own |gate|, the sparse down
  on the kernel's own h within the per-element bound, and the MLP output within 1e-3 (normalized) of the
  oracle's DIP MLP on the same input (free-running DIP logits are not compared: one |gate| at the selection
  boundary rounded to the other binary16 neighbour swaps a channel and moves the logits past any tight bound);
* over a 300-token context (split attention), the gated DIP schedule and cache-aware DIP (a calibrated 20% hot
  cache, misses read from pinned host memory) give DIP's tokens and final hidden state bit for bit, eager and
  graph replays.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import decoder as OD
from oracle import oracle as O
from test_decode_engine_gpu import prompt_ids, run_against_oracle
from test_decode_full_shape_gpu import _first_step_trace

pytestmark = pytest.mark.gpu

SHAPES = {
    "qwen3_0p6b": dict(hidden=1024, q_heads=16, kv_heads=8, intermediate=3072),
    "qwen3_4b": dict(hidden=2560, q_heads=32, kv_heads=8, intermediate=9728),
    "qwen3_8b": dict(hidden=4096, q_heads=32, kv_heads=8, intermediate=12288),
}


@pytest.fixture(scope="module")
def dec(cuda):
    from soinfer.runtime import decoder

    return decoder


@pytest.fixture(scope="module", params=list(SHAPES))
def model(request, dec):
    cfg = dec.DecoderConfig(layers=2, head_dim=128, vocab=4096, max_seq=320, **SHAPES[request.param])
    w = dec.random_decoder(cfg, seed=11, linear_std=0.03, norm_jitter=0.1)
    yield request.param, w
    del w
    torch.cuda.empty_cache()


def test_dense_matches_oracle(dec, model):
    name, w = model
    run_against_oracle(dec, w, "dense", None, n_prompt=3, n_new=3, tol=5e-3)


def test_dip_step_per_layer_matches_oracle(dec, model):
    name, w = model
    c = w.config
    I, H, gs = c.intermediate, c.hidden, c.group_size
    k = I // 2
    eng = dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=2)
    trace = _first_step_trace(eng, prompt_ids(3, c.vocab, seed=29))
    assert len(trace) == c.layers
    for l, t in enumerate(trace):
        L = w.layers[l]
        h = t["h"].cpu().numpy()
        gate = t["gate"].cpu().numpy()
        assert_close(t["gate"], O.gemv_w4_f64(L.gu_Wq[:I].cpu().numpy(), L.gu_scale[:I].cpu().numpy(), h, H, gs),
                     f"{name} layer {l} gate")
        idx = t["idx"].cpu().numpy()
        assert int(t["cnt"].item()) == k
        assert np.array_equal(idx, O.topk_rule_a(np.abs(gate.astype(np.float32)), k)), f"{name} layer {l} selection"
        dW, dS = L.down_T_Wq.cpu().numpy()[idx], L.down_T_scale.cpu().numpy()[idx]
        assert_close(t["down"], O.sparse_accumulate_f64(dW, dS, t["h_sel"].cpu().numpy(), H, gs),
                     f"{name} layer {l} sparse down")
        u = OD.int4_gemv(L.gu_Wq[I:].cpu().numpy()[idx], L.gu_scale[I:].cpu().numpy()[idx], h, gs)
        y_ref = O.sparse_accumulate_f64(dW, dS, OD.silu_mul(gate[idx], u), H, gs)
        err = np.abs(t["down"].float().cpu().numpy() - y_ref).max()
        assert err <= 1e-3 * np.abs(y_ref).max(), f"{name} layer {l} MLP: {err / np.abs(y_ref).max():.2e}"


def test_gated_and_cached_dip_bit_identical_to_dip(dec, model):
    name, w = model
    cfg = w.config
    k = cfg.intermediate // 2
    prompt = prompt_ids(300, cfg.vocab, seed=23)
    plain = dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=4)
    want = plain.generate(prompt, 4, use_graph=True)
    assert plain.defer_combine == (cfg.q_heads * cfg.head_dim <= 2048), name
    gated = dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=4, dip_schedule="gated")
    assert gated.dip_gated_tr, f"{name}: the ordered down should fit this shape"
    hot = dec.calibrate_hot_channels(w, k, prompt_ids(16, cfg.vocab, seed=1001), cache_fraction=0.2)
    cached = dec.DecodeEngine(w, "cached_dip", dip_k=k, hot_channels=hot, max_new_tokens=4)
    for eng, tag in ((gated, "gated"), (cached, "cached_dip")):
        for use_graph in (False, True):
            assert eng.generate(prompt, 4, use_graph=use_graph) == want, f"{name} {tag} graph={use_graph}"
            assert torch.equal(eng.x_final, plain.x_final), f"{name} {tag} graph={use_graph}: hidden state"
