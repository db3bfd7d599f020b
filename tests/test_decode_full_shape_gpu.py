"""Config 5 at the full Qwen3-1.7B shape (28 layers, hidden 2048, 16/8 heads, I = 6144, vocab 151936) on the GPU.

Counterpart of the reference's DIP / cache-aware DIP comparison (python/soinfer/runtime/generate.py:466-542,
tests/test_m8_cached_dip_pipeline.py:103-138) at the real shape, k/I = 0.5, with a 20% hot cache calibrated
from 64 seeded tokens (calibrate_hot_channels, generate.py:579-609):
  * DIP (indexed up GEMV) and cache-aware DIP with the misses read in place from pinned host memory (direct)
    or gathered into staging first (staged) generate the same tokens and end with bit-identical hidden states,
    from HIP-graph replays; DIP with the dense-up schedule (one-launch selection + gated down) sums its down
    terms in another order, so its tokens are checked for determinism (graph replay == eager run) only;
  * the first generated step, teacher-forced layer by layer: each layer's gate within 1e-3 of the binary64
    oracle GEMV on the layer's own MLP input, the selection equal to the oracle's rule A on the kernel's own
    |gate| (count = k), the gated up values h and the sparse down (on the kernel's own h) within the
    per-element bound of tests/helpers.py, and the whole MLP output within 1e-3 (normalized) of the oracle's
    DIP MLP on the same input; every other schedule gives the same selection and output bit for bit.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import decoder as OD
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DIP_K = 3072
N_PROMPT, N_NEW = 16, 8


@pytest.fixture(scope="module")
def setup(cuda):
    from soinfer.runtime import decoder as D

    w = D.random_decoder(D.QWEN3_1P7B, seed=0)
    V = w.config.vocab
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, V, (N_PROMPT,), generator=g).tolist()
    calib = torch.randint(0, V, (64,), generator=torch.Generator().manual_seed(1000)).tolist()
    hot = D.calibrate_hot_channels(w, DIP_K, calib, cache_fraction=0.2)
    assert all(len(h) == 1229 for h in hot)
    return D, w, prompt, hot


def _engines(D, w, hot):
    return {
        "dip": D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW),
        "dip_dense_up": D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW, dip_dense_up=True),
        "cached_direct": D.DecodeEngine(w, "cached_dip", dip_k=DIP_K, hot_channels=hot, max_new_tokens=N_NEW),
        "cached_staged": D.DecodeEngine(w, "cached_dip", dip_k=DIP_K, hot_channels=hot, max_new_tokens=N_NEW,
                                        miss_path="staged"),
    }


def test_config5_dip_and_cached_dip_generate_identically(setup):
    D, w, prompt, hot = setup
    engines = _engines(D, w, hot)
    ref = engines.pop("dip")
    want = ref.generate(prompt, N_NEW)
    assert len(want) == N_PROMPT + N_NEW and all(0 <= t < w.config.vocab for t in want)
    x_ref = ref.x_final.clone()
    for name, eng in engines.items():
        got = eng.generate(prompt, N_NEW)
        if name == "dip_dense_up":
            # its down sums the same terms in another order: on this random-init model the logits are nearly flat
            # and a 1e-3 difference in one layer's MLP output, carried through 28 layers, already moves the first
            # argmax, so tokens are not compared with DIP (its per-layer agreement with the oracle on its own
            # inputs is checked below); its own runs are deterministic: graph replays equal the eager run
            x_du = eng.x_final.clone()
            assert eng.generate(prompt, N_NEW, use_graph=False) == got
            assert torch.equal(eng.x_final, x_du), f"{name}: eager run differs from the graph replay"
            del eng
            continue
        assert got == want, f"{name}: tokens differ from DIP"
        assert torch.equal(eng.x_final, x_ref), f"{name}: final hidden state differs from DIP"
        del eng
    # a second replay of the same prompt gives the same tokens (graphs re-read device position and token)
    assert ref.generate(prompt, N_NEW) == want
    assert torch.equal(ref.x_final, x_ref)


def _first_step_trace(eng, prompt):
    """Prefill (graphs), then the first generated step eagerly with a per-layer snapshot of the MLP input,
    gate, selection, count and output."""
    I = eng.c.intermediate
    eng.capture()
    eng.reset()
    eng.prefill(prompt)
    trace = []

    def hook(l):
        trace.append({"h": eng.h.clone(), "gate": eng.gu[:I].clone(), "idx": eng.idx.clone(),
                      "cnt": eng.cnt.clone(), "h_sel": eng.h_sel.clone(), "down": eng.down.clone(),
                      "h_all": eng.gu[I:].clone()})

    eng._head()
    eng.layer_hook = hook
    eng._layers()
    eng.layer_hook = None
    torch.cuda.synchronize()
    return trace


def test_config5_first_step_per_layer_matches_oracle(setup):
    D, w, prompt, hot = setup
    c = w.config
    I, H, gs = c.intermediate, c.hidden, c.group_size
    engines = _engines(D, w, hot)
    traces = {name: _first_step_trace(eng, prompt) for name, eng in engines.items()}
    del engines
    ref = traces["dip"]
    assert len(ref) == c.layers
    for l, t in enumerate(ref):
        L = w.layers[l]
        h = t["h"].cpu().numpy()
        gate = t["gate"].cpu().numpy()
        gW, gS = L.gu_Wq[:I].cpu().numpy(), L.gu_scale[:I].cpu().numpy()
        assert_close(t["gate"], O.gemv_w4_f64(gW, gS, h, H, gs), f"layer {l} gate")
        idx = t["idx"].cpu().numpy()
        assert int(t["cnt"].item()) == DIP_K
        assert np.array_equal(idx, O.topk_rule_a(np.abs(gate.astype(np.float32)), DIP_K)), f"layer {l} selection"
        uW, uS = L.gu_Wq[I:].cpu().numpy()[idx], L.gu_scale[I:].cpu().numpy()[idx]
        u = OD.int4_gemv(uW, uS, h, gs)
        hs = OD.silu_mul(gate[idx], u)
        # the gated up values against the oracle's on the same gate and input: u and then h are each rounded to
        # binary16 on both sides, so they may sit up to two binary16 steps apart (2^-10 relative each)
        assert_close(t["h_sel"], hs.astype(np.float64), f"layer {l} gated up h", tol=2e-3)
        dW, dS = L.down_T_Wq.cpu().numpy()[idx], L.down_T_scale.cpu().numpy()[idx]
        # the sparse down on the kernel's own h: the full per-element bound
        assert_close(t["down"], O.sparse_accumulate_f64(dW, dS, t["h_sel"].cpu().numpy(), H, gs),
                     f"layer {l} sparse down")
        # the whole MLP from the layer's input against the oracle's MLP (h rounded independently there, so a few
        # h_j differ by one binary16 step): normalized bound
        y_ref = O.sparse_accumulate_f64(dW, dS, hs, H, gs)
        err = np.abs(t["down"].float().cpu().numpy() - y_ref).max()
        assert err <= 1e-3 * np.abs(y_ref).max(), f"layer {l} MLP: normalized error {err / np.abs(y_ref).max():.2e}"
        for name, tr in traces.items():
            o = tr[l]
            if name == "dip_dense_up":
                # its own inputs (the earlier layers' downs sum in another order): the selection is rule A on its own
                # gate, and the down is the oracle's sparse accumulate over that selection and its own h
                og = o["gate"].cpu().numpy()
                oi = o["idx"].cpu().numpy()
                assert int(o["cnt"].item()) == DIP_K
                assert np.array_equal(oi, O.topk_rule_a(np.abs(og.astype(np.float32)), DIP_K)), f"{name} layer {l}"
                oh = o["h_all"].cpu().numpy()[oi]
                assert_close(o["down"], O.sparse_accumulate_f64(L.down_T_Wq.cpu().numpy()[oi],
                                                                L.down_T_scale.cpu().numpy()[oi], oh, H, gs),
                             f"{name} layer {l} down")
                continue
            assert torch.equal(o["idx"], t["idx"]) and torch.equal(o["cnt"], t["cnt"]), f"{name} layer {l} idx"
            assert torch.equal(o["down"], t["down"]), f"{name} layer {l} MLP output"
            assert torch.equal(o["h"], t["h"]), f"{name} layer {l} MLP input"
            assert torch.equal(o["h_sel"], t["h_sel"]), f"{name} layer {l} gated up h"
