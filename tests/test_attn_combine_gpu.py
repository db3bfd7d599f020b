"""Deferred attention combine: the o projection finishes a split attention step (decode_attention.hip).

soi_decode_attention_step_deferred leaves a split context's per-split softmax states in the workspace, and
soi_gemv_w4a16_attn_combine combines them while loading the o projection's x. The pair must equal the
reference's decode_attention followed by the o_proj GEMV (generate.py:169-171) as this build computes them
(soi_decode_attention_step, then soi_gemv_w4a16_group_lop3 on its output), bit for bit:
  * y (and res_out = res + y with the residual epilogue) identical at every context length, on both sides of
    the split boundary (8 kernel passes), at the longest context, and with more splits than one load batch
    holds (one KV head: up to 64 splits);
  * both KV caches identical (the step's append is unchanged), the attention output identical where the
    context does not split;
  * the general (several-pass, ragged-row, per-word-scale) forms as well as the K = 2048 one-pass form;
  * shapes outside the form rejected.
"""
import pytest
import torch

from helpers import int4_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def C(cuda):
    from soinfer import _C

    return _C


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


def rnd(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).half()


def _split(L, NKV, hd):
    """Whether the attention kernel splits a context of L timesteps (more than 8 passes of 8 waves)."""
    step = (64 // (hd // 8)) * 8
    return L > 8 * step


@pytest.mark.parametrize("NQ,NKV,hd,S,N,gs,lengths", [
    (16, 8, 128, 2048, 2048, 128, [1, 7, 256, 257, 300, 1024, 1025, 2048]),  # Qwen3-1.7B, one-pass form
    (4, 2, 64, 1024, 256, 128, [100, 512, 513, 1024]),                        # several passes: K = 256
    (8, 1, 128, 4096, 1000, 128, [256, 257, 2000, 4096]),                     # one KV head: 64 splits; ragged N
    (16, 8, 128, 2048, 2048, 16, [200, 300, 2048]),                           # per-word scales (gs % 32 != 0)
    (16, 8, 128, 16384, 2048, 128, [200, 4096, 8193, 16384]),                 # long contexts: many passes per split
])
def test_deferred_step_and_combine_equal_step_and_gemv(C, ops, NQ, NKV, hd, S, N, gs, lengths):
    K = NQ * hd
    cos_t, sin_t = ops.rope_tables(hd, 1e6, S, "cuda")
    qn, kn = (rnd((hd,), 22) * 0.1 + 1).half().cuda(), (rnd((hd,), 23) * 0.1 + 1).half().cuda()
    kc_a, vc_a = rnd((NKV, S, hd), 24).cuda(), rnd((NKV, S, hd), 25).cuda()
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    Wo = int4_problem(N, K, gs, seed=26 + N)
    ws_a = torch.zeros(C.decode_attention_step_workspace_bytes(NQ, NKV, hd, S), dtype=torch.uint8, device="cuda")
    ws_b = torch.zeros_like(ws_a)
    out_a = torch.zeros(NQ, hd, dtype=torch.float16, device="cuda")
    out_b = torch.zeros_like(out_a)
    y = torch.empty(N, dtype=torch.float16, device="cuda")
    res = rnd((N,), 27, 4.0).cuda()
    res_out = torch.empty_like(res)
    y2 = torch.empty_like(y)
    for i, L in enumerate(lengths):
        qkv = rnd(((NQ + 2 * NKV) * hd,), 200 + i, 2.0).cuda()
        pos = torch.tensor([L - 1], dtype=torch.int32, device="cuda")
        print(f"case NQ={NQ} NKV={NKV} hd={hd} N={N} gs={gs} L={L}", flush=True)
        C.decode_attention_step(qkv, qn, kn, cos_t, sin_t, pos, kc_a, vc_a, out_a, 1e-6, ws_a)
        y_ref = ops.gemv_w4a16_group_lop3(Wo["Wq_d"], Wo["s_d"], out_a.view(-1), K, gs)
        C.decode_attention_step_deferred(qkv, qn, kn, cos_t, sin_t, pos, kc_b, vc_b, out_b, 1e-6, ws_b)
        C.gemv_w4a16_attn_combine_into(Wo["Wq_d"], Wo["s_d"], ws_b, out_b, pos, NKV, S, y, gs)
        C.gemv_w4a16_attn_combine_into(Wo["Wq_d"], Wo["s_d"], ws_b, out_b, pos, NKV, S, y2, gs, res, res_out)
        assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b), f"caches at length {L}"
        if not _split(L, NKV, hd):
            assert torch.equal(out_a, out_b), f"unsplit attention output at length {L}"
        assert torch.equal(y, y_ref), f"y at length {L}"
        assert torch.equal(y2, y_ref), f"y (residual form) at length {L}"
        assert torch.equal(res_out.cpu(), res.cpu() + y_ref.cpu()), f"res_out at length {L}"
    assert any(_split(L, NKV, hd) for L in lengths) and not all(_split(L, NKV, hd) for L in lengths)


def test_attn_combine_rejections(C, ops):
    NQ, NKV, hd, S = 32, 8, 128, 512  # K = 4096 > 2048
    ws = torch.zeros(C.decode_attention_step_workspace_bytes(NQ, NKV, hd, S), dtype=torch.uint8, device="cuda")
    out = torch.zeros(NQ, hd, dtype=torch.float16, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    Wo = int4_problem(64, NQ * hd, 128, seed=3)
    y = torch.empty(64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="at most 2048"):
        C.gemv_w4a16_attn_combine_into(Wo["Wq_d"], Wo["s_d"], ws, out, pos, NKV, S, y, 128)
    NQ = 16
    ws = torch.zeros(C.decode_attention_step_workspace_bytes(NQ, NKV, hd, S), dtype=torch.uint8, device="cuda")
    out = torch.zeros(NQ, hd, dtype=torch.float16, device="cuda")
    Wo = int4_problem(64, NQ * hd, 128, seed=4)
    with pytest.raises(RuntimeError, match="go together"):
        C.gemv_w4a16_attn_combine_into(Wo["Wq_d"], Wo["s_d"], ws, out, pos, NKV, S, y, 128, y.clone(), None)
    with pytest.raises(RuntimeError, match="workspace"):
        C.gemv_w4a16_attn_combine_into(Wo["Wq_d"], Wo["s_d"], ws[:64], out, pos, NKV, S, y, 128)
    with pytest.raises(RuntimeError, match="not supported"):  # head_dim 96 is not a power of two
        out96 = torch.zeros(NQ, 96, dtype=torch.float16, device="cuda")
        W96 = int4_problem(64, NQ * 96, 128, seed=5)
        C.gemv_w4a16_attn_combine_into(W96["Wq_d"], W96["s_d"], ws, out96, pos, NKV, S, y, 128)


@pytest.fixture(scope="module")
def dec(cuda):
    from soinfer.runtime import decoder

    return decoder


@pytest.mark.parametrize("mode,k", [("dense", None), ("dip", 128)])
def test_engine_deferred_combine_bit_identical(dec, mode, k):
    """A decoder whose context crosses the split boundary (512 timesteps at head_dim 64): tokens and the final
    hidden state with the combine in the o projection == with the combine in the attention launch, eager and
    under graph replay."""
    cfg = dec.DecoderConfig(hidden=256, layers=2, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                            group_size=128, max_seq=1024)
    w = dec.random_decoder(cfg, seed=5, linear_std=0.05, norm_jitter=0.1)
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, cfg.vocab, (530,), generator=g).tolist()
    n_new = 6
    kw = dict(dip_k=k, max_new_tokens=n_new, dip_dense_up=mode == "dip")
    ref = dec.DecodeEngine(w, mode, defer_attention_combine=False, **kw)
    assert not ref.defer_combine
    want = ref.generate(prompt, n_new, use_graph=True)
    x_ref = ref.x_final.clone()
    for use_graph in (True, False):
        eng = dec.DecodeEngine(w, mode, defer_attention_combine=True, **kw)
        assert eng.defer_combine
        got = eng.generate(prompt, n_new, use_graph=use_graph)
        assert got == want, f"{mode} graph={use_graph}: tokens differ"
        assert torch.equal(eng.x_final, x_ref), f"{mode} graph={use_graph}: hidden state differs"
