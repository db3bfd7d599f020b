"""The decode engine over seeded random small decoder configurations (two layers each; hidden, head counts, head
size, intermediate size, vocabulary and group size drawn from a fixed generator, so the same configurations run
every time):

* dense logits against the oracle decoder for 3 prompt + 3 new tokens (the tolerance rule of
  tests/test_decode_engine_gpu.py), fused and unfused layers;
* DIP at a random k, the first generated step teacher-forced layer by layer against the oracle (the gate, the
  selection exactly, the sparse down on the kernel's own h, the MLP output);
* the gated DIP schedule and cache-aware DIP (a random hot set, misses read from pinned host memory) give DIP's
  tokens and final hidden state bit for bit over a context past one attention workgroup's rows (split
  attention), eager and graph replays.
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


def _config(r):
    kv = int(r.choice([1, 2, 4, 8]))
    rep = int(r.choice([1, 2, 4]))
    hd = int(r.choice([64, 128]))
    gs = int(r.choice([64, 128]))
    return dict(hidden=128 * int(r.integers(1, 9)), q_heads=kv * rep, kv_heads=kv, head_dim=hd,
                intermediate=128 * int(r.integers(2, 25)), vocab=int(r.integers(300, 3001)), group_size=gs,
                k_frac=float(r.uniform(0.1, 0.9)))


_rng = np.random.default_rng(909)
CONFIGS = [_config(_rng) for _ in range(6)]


@pytest.fixture(scope="module")
def dec(cuda):
    from soinfer.runtime import decoder

    return decoder


@pytest.fixture(scope="module", params=range(len(CONFIGS)), ids=lambda i: f"cfg{i}")
def model(request, dec):
    c = dict(CONFIGS[request.param])
    kf = c.pop("k_frac")
    cfg = dec.DecoderConfig(layers=2, max_seq=640, **c)
    w = dec.random_decoder(cfg, seed=100 + request.param, linear_std=0.04, norm_jitter=0.1)
    yield c, max(1, int(round(kf * cfg.intermediate))), w
    del w
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fused", [True, False])
def test_dense_matches_oracle(dec, model, fused):
    c, k, w = model
    run_against_oracle(dec, w, "dense", None, n_prompt=3, n_new=3, tol=5e-3, fused=fused)


def test_dip_step_per_layer_matches_oracle(dec, model):
    c, k, w = model
    cfg = w.config
    I, H, gs = cfg.intermediate, cfg.hidden, cfg.group_size
    eng = dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=2)
    trace = _first_step_trace(eng, prompt_ids(3, cfg.vocab, seed=31))
    for l, t in enumerate(trace):
        L = w.layers[l]
        h = t["h"].cpu().numpy()
        gate = t["gate"].cpu().numpy()
        assert_close(t["gate"], O.gemv_w4_f64(L.gu_Wq[:I].cpu().numpy(), L.gu_scale[:I].cpu().numpy(), h, H, gs),
                     f"{c} layer {l} gate")
        idx = t["idx"].cpu().numpy()
        assert int(t["cnt"].item()) == k
        assert np.array_equal(idx, O.topk_rule_a(np.abs(gate.astype(np.float32)), k)), f"{c} layer {l} selection"
        dW, dS = L.down_T_Wq.cpu().numpy()[idx], L.down_T_scale.cpu().numpy()[idx]
        assert_close(t["down"], O.sparse_accumulate_f64(dW, dS, t["h_sel"].cpu().numpy(), H, gs),
                     f"{c} layer {l} sparse down")
        u = OD.int4_gemv(L.gu_Wq[I:].cpu().numpy()[idx], L.gu_scale[I:].cpu().numpy()[idx], h, gs)
        y_ref = O.sparse_accumulate_f64(dW, dS, OD.silu_mul(gate[idx], u), H, gs)
        err = np.abs(t["down"].float().cpu().numpy() - y_ref).max()
        assert err <= 1e-3 * np.abs(y_ref).max(), f"{c} layer {l} MLP: {err / np.abs(y_ref).max():.2e}"


def test_gated_and_cached_dip_bit_identical_to_dip(dec, model):
    c, k, w = model
    cfg = w.config
    prompt = prompt_ids(540, cfg.vocab, seed=37)
    plain = dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=4)
    want = plain.generate(prompt, 4, use_graph=True)
    r = np.random.default_rng(cfg.intermediate + k)
    hot = [sorted(r.choice(cfg.intermediate, size=int(r.integers(0, cfg.intermediate + 1)), replace=False).tolist())
           for _ in range(cfg.layers)]
    engines = [("gated", dec.DecodeEngine(w, "dip", dip_k=k, max_new_tokens=4, dip_schedule="gated")),
               ("cached_dip", dec.DecodeEngine(w, "cached_dip", dip_k=k, hot_channels=hot, max_new_tokens=4))]
    for tag, eng in engines:
        for use_graph in (False, True):
            assert eng.generate(prompt, 4, use_graph=use_graph) == want, f"{c} {tag} graph={use_graph}"
            assert torch.equal(eng.x_final, plain.x_final), f"{c} {tag} graph={use_graph}: hidden state"
