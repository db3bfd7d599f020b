"""Residual add in the producer's epilogue (soi_gemv_w4a16_residual, soi_dip_select_dense_down_residual).

The reference adds the o projection and the MLP output to the residual stream in PyTorch (generate.py:172
`h2 = residual + o`, :182 / :310 `residual2 + down`): one binary16 addition of the two fp16 vectors. The
producer launches that also write res_out must
  * leave y exactly as the plain launch writes it (and the index list of the dense down);
  * write res_out = res + y as PyTorch's CPU fp16 addition rounds it, including at overflow to inf, through
    subnormals, signed zeros and NaN rows, and the value the RMSNorm-fused GEMV writes as x_out from
    (res, delta = y);
  * work in place (res_out = res), on ragged row counts and with K off the vector path;
and the decode engine with the adds moved into the producers must give bit-identical tokens and hidden
states to the engine that adds on load, eager and under graph replay, in every schedule.
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


def _residual(N, seed):
    """fp16 residual values across binades with the special cases the add must round like PyTorch."""
    g = torch.Generator().manual_seed(seed)
    mag = torch.exp2(torch.randint(-20, 15, (N,), generator=g).float())
    r = (torch.randn(N, generator=g) * mag).half()
    special = torch.tensor([65504.0, -65504.0, 2.0 ** -24, -(2.0 ** -24), 0.0, -0.0, 2048.0, 1.0],
                           dtype=torch.float16)
    r[: min(N, special.numel())] = special[: min(N, special.numel())]
    return r


def _torch_add(res, y):
    """The reference's `residual + o`: PyTorch fp16 addition on the CPU."""
    return res.cpu() + y.cpu()


@pytest.mark.parametrize("N,K,gs", [(2048, 2048, 128), (2048, 6144, 128), (1000, 256, 128), (37, 96, 32),
                                    (4096, 2048, 128), (130, 200, 40)])
def test_gemv_residual_matches_plain_gemv_and_add(C, ops, N, K, gs):
    p = int4_problem(N, K, gs, seed=N + K)
    res = _residual(N, seed=7 + N).cuda()
    y_ref = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)
    y, res_out = ops.gemv_w4a16_residual(p["Wq_d"], p["s_d"], p["x_d"], res, p["K"], gs)
    assert torch.equal(y, y_ref), "y differs from the plain GEMV"
    assert torch.equal(res_out.cpu(), _torch_add(res, y)), "res_out differs from the fp16 add"
    # the value the RMSNorm-fused GEMV writes as x_out from (res, delta = y) when N is its K
    if N == 2048:
        Wn = int4_problem(64, N, 128, seed=5)
        xo = torch.empty_like(res)
        yn = torch.empty(64, dtype=torch.float16, device="cuda")
        nw = torch.ones(N, dtype=torch.float16, device="cuda")
        C.gemv_w4a16_rmsnorm_into(Wn["Wq_d"], Wn["s_d"], res, y, nw, 1e-6, xo, None, yn, N, 128, False)
        assert torch.equal(xo, res_out), "res_out differs from the fused GEMV's residual sum"
    # in place: res_out = res
    r2 = res.clone()
    y2 = torch.empty_like(y)
    C.gemv_w4a16_residual_into(p["Wq_d"], p["s_d"], p["x_d"], y2, r2, r2, p["K"], gs)
    assert torch.equal(y2, y) and torch.equal(r2, res_out)


def test_gemv_residual_overflow_and_nan_rows(C, ops):
    """Sums past the binary16 range become inf with the sign of the sum; a NaN residual stays NaN."""
    N, K, gs = 256, 256, 128
    p = int4_problem(N, K, gs, seed=3, std=4.0)  # |y| of order 100: sums with +-65504 cross 65520
    y = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)
    res = torch.where(y > 0, torch.full_like(y, 65504.0), torch.full_like(y, -65504.0))
    res[:4] = float("nan")
    y2, res_out = ops.gemv_w4a16_residual(p["Wq_d"], p["s_d"], p["x_d"], res, p["K"], gs)
    assert torch.equal(y2, y)
    ref = _torch_add(res, y)
    got = res_out.cpu()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    m = ~torch.isnan(ref)
    assert torch.equal(got[m], ref[m])
    assert torch.isinf(ref).any(), "the case must reach the overflow"


def test_gemv_residual_rejects_bad_arguments(C, ops):
    p = int4_problem(64, 128, 64, seed=1)
    res = torch.zeros(64, dtype=torch.float16, device="cuda")
    y = torch.empty(64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="res and res_out"):
        C.gemv_w4a16_residual_into(p["Wq_d"], p["s_d"], p["x_d"], y, res[:63], res, p["K"], 64)
    with pytest.raises(RuntimeError, match="alias"):
        C.gemv_w4a16_residual_into(p["Wq_d"], p["s_d"], p["x_d"], y, res, y, p["K"], 64)


@pytest.mark.parametrize("I,H,k", [(6144, 2048, 3072), (6144, 2048, 768), (96, 384, 50), (3008, 2176, 1111)])
def test_dense_down_residual_matches_plain_launch_and_add(C, ops, I, H, k):
    down = int4_problem(I, H, 128, seed=31 + k)
    Wt, St = ops.transposed_down_T(down["Wq_d"], down["s_d"], H)
    g = torch.Generator().manual_seed(32 + k)
    gate = (torch.randn(I, generator=g) * 2).half().cuda()
    up = (torch.randn(I, generator=g) * 2).half().cuda()
    h = torch.empty_like(gate)
    C.silu_mul_into(gate, up, h)
    res = _residual(H, seed=33 + k).cuda()
    y_ref, idx_ref, cnt_ref = ops.dip_select_dense_down(gate, h, k, Wt, St, 128)
    y, res_out, idx, cnt = ops.dip_select_dense_down_residual(gate, h, k, Wt, St, 128, res)
    assert torch.equal(y, y_ref) and torch.equal(idx, idx_ref) and torch.equal(cnt, cnt_ref)
    assert torch.equal(res_out.cpu(), _torch_add(res, y))
    y2, res_out2, _, _ = ops.dip_select_dense_down_residual(gate, h, k, Wt, St, 128, res, with_indices=False)
    assert torch.equal(y2, y) and torch.equal(res_out2, res_out)
    r2 = res.clone()  # in place
    y3 = torch.empty_like(y)
    C.dip_select_dense_down_into(gate, h, k, Wt, St, None, None, y3, 128, r2, r2)
    assert torch.equal(y3, y) and torch.equal(r2, res_out)
    with pytest.raises(RuntimeError, match="go together"):
        C.dip_select_dense_down_into(gate, h, k, Wt, St, None, None, y3, 128, res, None)


@pytest.fixture(scope="module")
def dec(cuda):
    from soinfer.runtime import decoder

    return decoder


@pytest.fixture(scope="module")
def tiny(dec):
    cfg = dec.DecoderConfig(hidden=256, layers=3, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
                            group_size=128, max_seq=64)
    return dec.random_decoder(cfg, seed=3, linear_std=0.05, norm_jitter=0.1)


@pytest.mark.parametrize("mode,k,extra", [("dense", None, {}), ("dip", 256, {}), ("dip", 256, {"dip_dense_up": True}),
                                          ("cached_dip", 256, {"hot_channels": "third"}),
                                          ("dense", None, {"offload": True})])
def test_engine_residual_epilogue_bit_identical(dec, tiny, mode, k, extra):
    """Tokens and the final hidden state with the adds in the producers == with the adds on load."""
    prompt, n_new = [3, 17, 5, 9, 2, 611], 6
    kw = dict(dip_k=k, max_new_tokens=n_new, **extra)
    if kw.get("hot_channels") == "third":
        I = tiny.config.intermediate
        kw["hot_channels"] = [list(range(0, I, 3)) for _ in range(tiny.config.layers)]
    ref = dec.DecodeEngine(tiny, mode, residual_epilogue=False, **kw)
    out_ref = ref.generate(prompt, n_new, use_graph=False)
    x_ref = ref.x_final.clone()
    for use_graph in (False, True):
        eng = dec.DecodeEngine(tiny, mode, residual_epilogue=True, **kw)
        out = eng.generate(prompt, n_new, use_graph=use_graph)
        assert out == out_ref, f"{mode} {extra} graph={use_graph}: tokens differ"
        assert torch.equal(eng.x_final, x_ref), f"{mode} {extra} graph={use_graph}: hidden state differs"
