"""Config 5 at the full Qwen3-1.7B shape (28 layers, hidden 2048, 16/8 heads, I = 6144, vocab 151936) on the GPU.

Counterpart of the reference's DIP / cache-aware DIP comparison (python/soinfer/runtime/generate.py:466-542,
tests/test_m8_cached_dip_pipeline.py:103-138) at the real shape, k/I = 0.5, with a 20% hot cache calibrated
from 64 seeded tokens (calibrate_hot_channels, generate.py:579-609):
  * DIP (indexed up GEMV), DIP with the two-launch gated schedule and cache-aware DIP with the misses read in
    place from pinned host memory (direct) or gathered into staging first (staged) generate the same tokens and
    end with bit-identical hidden states, from HIP-graph replays; DIP with the dense-up schedule (one-launch selection + gated down) sums its down
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
        "dip_gated": D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW, dip_schedule="gated"),
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
            if name == "dip_gated":
                # normalizes on load and forms h inside the down launch: neither the normed input nor h_sel is
                # stored; its gate of every channel and the up values of the selected ones are
                assert torch.equal(o["gate"], t["gate"]), f"{name} layer {l} gate"
                continue
            assert torch.equal(o["h"], t["h"]), f"{name} layer {l} MLP input"
            assert torch.equal(o["h_sel"], t["h_sel"]), f"{name} layer {l} gated up h"


# BASELINE config 5 at its stated lengths: a 64-token prompt, then 128 greedy tokens (positions 0 .. 191)
N_PROMPT5, N_NEW5 = 64, 128


def _prompt5(V):
    return torch.randint(0, V, (N_PROMPT5,), generator=torch.Generator().manual_seed(7)).tolist()


def test_config5_full_length_cached_dip_equals_dip(setup):
    """64 + 128 tokens through 28 layers: cache-aware DIP (20% calibrated hot cache, misses from pinned host
    memory, direct and staged) and the gated DIP schedule generate DIP's tokens and end with its final hidden
    state, bit for bit."""
    D, w, _, hot = setup
    prompt = _prompt5(w.config.vocab)
    dip = D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW5)
    want = dip.generate(prompt, N_NEW5)
    x_ref = dip.x_final.clone()
    assert len(want) == N_PROMPT5 + N_NEW5 and int(dip.pos.item()) == N_PROMPT5 + N_NEW5
    del dip
    for path in ("direct", "staged"):
        eng = D.DecodeEngine(w, "cached_dip", dip_k=DIP_K, hot_channels=hot, max_new_tokens=N_NEW5, miss_path=path)
        got = eng.generate(prompt, N_NEW5)
        assert got == want, f"cached DIP ({path}): tokens differ from DIP"
        assert torch.equal(eng.x_final, x_ref), f"cached DIP ({path}): final hidden state differs from DIP"
        del eng
    # the two-launch gated schedule: the same tokens and final hidden state as well
    eng = D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW5, dip_schedule="gated")
    assert eng.generate(prompt, N_NEW5) == want, "gated DIP: tokens differ from DIP"
    assert torch.equal(eng.x_final, x_ref), "gated DIP: final hidden state differs from DIP"


def test_config5_last_step_per_layer_matches_oracle(setup):
    """The last step of the 64 + 128 token run (position 191), teacher-forced layer by layer on the engine's own
    state after 191 positions: q/k norm + RoPE + the attention over the engine's own KV cache of 192 positions
    against the binary64 oracle attention, the gate GEMV, rule-A selection, gated up values and sparse down
    against the oracle as in the first-step test. (defer_attention_combine=False so the attention output is in
    one buffer; the deferred form equals it bit for bit, tests/test_attn_combine_gpu.py.)"""
    D, w, _, hot = setup
    from soinfer import _C

    c = w.config
    I, H, gs, NQ, NKV, hd = c.intermediate, c.hidden, c.group_size, c.q_heads, c.kv_heads, c.head_dim
    eng = D.DecodeEngine(w, "dip", dip_k=DIP_K, max_new_tokens=N_NEW5, defer_attention_combine=False)
    eng.capture()
    eng.reset()
    eng.prefill(_prompt5(c.vocab))
    eng.decode(N_NEW5 - 1)
    torch.cuda.synchronize()
    pos = int(eng.pos.item())
    assert pos == N_PROMPT5 + N_NEW5 - 1 == 191
    trace = []

    def hook(l):
        trace.append({"h": eng.h.clone(), "gate": eng.gu[:I].clone(), "idx": eng.idx.clone(), "cnt": eng.cnt.clone(),
                      "h_sel": eng.h_sel.clone(), "down": eng.down.clone(), "qkv": eng.qkv.clone(),
                      "attn": eng.attn.clone()})

    eng._head()
    eng.layer_hook = hook
    eng._layers()
    eng.layer_hook = None
    torch.cuda.synchronize()
    assert len(trace) == c.layers
    p = torch.tensor([pos], dtype=torch.int32, device="cuda")
    for l, t in enumerate(trace):
        L = w.layers[l]
        # attention: q from the layer's own qkv by the q/k norm + RoPE op (tested against the oracle separately),
        # the K/V caches as the engine left them (the appended row at 191 included)
        q = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
        kc, vc = eng.k_cache[l].clone(), eng.v_cache[l].clone()
        _C.qk_norm_rope_append(t["qkv"], L.q_norm, L.k_norm, eng.cos_t, eng.sin_t, p, q, kc, vc, c.rms_eps)
        assert torch.equal(kc, eng.k_cache[l]) and torch.equal(vc, eng.v_cache[l]), f"layer {l}: KV row at 191"
        a_ref = O.decode_attention_f64(q.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), pos + 1)
        assert_close(t["attn"].view(NQ, hd), a_ref, f"layer {l} attention at L = {pos + 1}")
        # MLP
        h = t["h"].cpu().numpy()
        gate = t["gate"].cpu().numpy()
        assert_close(t["gate"], O.gemv_w4_f64(L.gu_Wq[:I].cpu().numpy(), L.gu_scale[:I].cpu().numpy(), h, H, gs),
                     f"layer {l} gate")
        idx = t["idx"].cpu().numpy()
        assert int(t["cnt"].item()) == DIP_K
        assert np.array_equal(idx, O.topk_rule_a(np.abs(gate.astype(np.float32)), DIP_K)), f"layer {l} selection"
        u = OD.int4_gemv(L.gu_Wq[I:].cpu().numpy()[idx], L.gu_scale[I:].cpu().numpy()[idx], h, gs)
        assert_close(t["h_sel"], OD.silu_mul(gate[idx], u).astype(np.float64), f"layer {l} gated up h", tol=2e-3)
        dW, dS = L.down_T_Wq.cpu().numpy()[idx], L.down_T_scale.cpu().numpy()[idx]
        assert_close(t["down"], O.sparse_accumulate_f64(dW, dS, t["h_sel"].cpu().numpy(), H, gs),
                     f"layer {l} sparse down")


def test_config5_int4_head_logits_match_oracle(setup):
    """The INT4 g128 LM head at the full vocabulary (151936 x 2048): logits on the engine's own final-normed
    state within the GEMV bound of the binary64 oracle, and the token their first maximum."""
    D, w, prompt, _ = setup
    c = w.config
    Wq, S = D.quantize_lm_head(w)
    eng = D.DecodeEngine(w, "dense", max_new_tokens=4, int4_head=True)
    eng.reset()
    eng.prefill(prompt[:2], use_graph=False)
    for i in range(2):
        eng._head()
        torch.cuda.synchronize()
        ref = O.gemv_w4_f64(Wq.cpu().numpy(), S.cpu().numpy(), eng.hn.cpu().numpy(), c.hidden, c.group_size)
        assert_close(eng.logits, ref, f"INT4 head step {i}")
        assert int(eng.token.item()) == OD.argmax_first(eng.logits.cpu().numpy())
        eng._layers()
