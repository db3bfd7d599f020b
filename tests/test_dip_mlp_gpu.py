"""The single-launch DIP MLP (soinfer._C.dip_mlp_into, C ABI soi_dip_mlp) on the GPU.

It must return exactly what the four launches it replaces return (the reference's DIP MLP op sequence,
generate.py:276-310: gate GEMV with the residual add + RMSNorm on load, rule-A top-k over |gate|, the indexed up
GEMV with the SiLU gating, the sparse down accumulate): gate, indices, count, gated h, y, the next residual and
the normed input, compared with torch.equal, at the Qwen3-1.7B shape for k/I = 0.125 ... 1, at small and maximal
intermediate sizes, on tie-heavy gates, on repeated calls through one workspace (the grid-barrier epochs
advance) and from HIP-graph replays. y is also checked against the binary64 oracle, the barrier error flag stays
clear, and the argument checks raise.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import oracle as O

pytestmark = pytest.mark.gpu
H, GS = 2048, 128


@pytest.fixture(scope="module")
def C(cuda):
    from soinfer import _C

    return _C


def _weights(I, seed, gs=GS, tie_blocks=0):
    mats = []
    for i in range(3):
        p = int4_problem(I, H, gs, seed=seed * 10 + i)
        mats.append((p["Wq_d"], p["s_d"]))
    if tie_blocks:  # gate rows repeated in blocks of tie_blocks: many exactly equal gates
        W, S = mats[0]
        rep = torch.arange(I, device="cuda") // tie_blocks * tie_blocks
        mats[0] = (W[rep].contiguous(), S[rep].contiguous())
    return mats


def _inputs(seed, with_delta=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(H, generator=g).half().cuda()
    d = (torch.randn(H, generator=g) * 0.5).half().cuda() if with_delta else None
    nw = (torch.randn(H, generator=g) * 0.1 + 1).half().cuda()
    return x, d, nw


def _four_launches(C, mats, x, d, nw, k, gs):
    (gW, gS), (uW, uS), (dW, dS) = mats
    I = gW.shape[0]
    f16 = dict(dtype=torch.float16, device="cuda")
    out = {"x_out": torch.empty(H, **f16), "h_out": torch.empty(H, **f16), "gate": torch.empty(I, **f16),
           "idx": torch.full((k,), -1, dtype=torch.int32, device="cuda"),
           "cnt": torch.zeros(1, dtype=torch.int32, device="cuda"), "h_sel": torch.empty(k, **f16),
           "y": torch.empty(H, **f16)}
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    C.gemv_w4a16_rmsnorm_into(gW, gS, x, d, nw, 1e-6, out["x_out"], out["h_out"], out["gate"], H, gs, False)
    C.topk_threshold_select_f16abs_into(out["gate"], k, out["idx"], out["cnt"])
    C.gemv_w4a16_indexed_silu_into(uW, uS, out["idx"], out["h_out"], out["gate"], out["h_sel"], H, gs)
    C.gemv_w4a16_indexed_accumulate_into(dW, dS, out["idx"], out["h_sel"], out["y"], H, gs, ws)
    return out


def _fused(C, mats, x, d, nw, k, gs, ws=None, out=None):
    (gW, gS), (uW, uS), (dW, dS) = mats
    I = gW.shape[0]
    f16 = dict(dtype=torch.float16, device="cuda")
    if out is None:
        out = {"x_out": torch.empty(H, **f16), "h_out": torch.empty(H, **f16), "gate": torch.empty(I, **f16),
               "idx": torch.full((k,), -1, dtype=torch.int32, device="cuda"),
               "cnt": torch.zeros(1, dtype=torch.int32, device="cuda"), "h_sel": torch.empty(k, **f16),
               "y": torch.empty(H, **f16)}
    if ws is None:
        ws = torch.zeros(C.dip_mlp_workspace_bytes(k), dtype=torch.uint8, device="cuda")
    C.dip_mlp_into(x, d, nw, 1e-6, out["x_out"], out["h_out"], gW, gS, uW, uS, dW, dS, k, out["gate"], out["idx"],
                   out["cnt"], out["h_sel"], out["y"], gs, ws)
    return out, ws


def _assert_same(a, b, label):
    for key in ("x_out", "h_out", "gate", "idx", "cnt", "h_sel", "y"):
        assert torch.equal(a[key], b[key]), f"{label}: {key} differs from the four launches"


@pytest.mark.parametrize("k", [768, 1536, 3072, 6144, 1, 4097])
def test_qwen3_shape_bit_identical_to_four_launches(C, k):
    mats = _weights(6144, seed=1)
    x, d, nw = _inputs(2)
    want = _four_launches(C, mats, x, d, nw, k, GS)
    got, ws = _fused(C, mats, x, d, nw, k, GS)
    _assert_same(got, want, f"k={k}")
    assert int(got["cnt"].item()) == k
    C.dip_mlp_check(ws)


def test_oracle_parity_and_selection_rule(C):
    I, k = 6144, 3072
    mats = _weights(I, seed=3)
    x, d, nw = _inputs(4)
    got, _ = _fused(C, mats, x, d, nw, k, GS)
    (gW, gS), (uW, uS), (dW, dS) = [(W.cpu().numpy(), S.cpu().numpy()) for W, S in mats]
    h = got["h_out"].cpu().numpy()
    assert_close(got["gate"], O.gemv_w4_f64(gW, gS, h, H, GS), "gate")
    gate = got["gate"].cpu().numpy()
    idx = got["idx"].cpu().numpy()
    assert np.array_equal(idx, O.topk_rule_a(np.abs(gate.astype(np.float32)), k))
    assert_close(got["y"], O.sparse_accumulate_f64(dW[idx], dS[idx], got["h_sel"].cpu().numpy(), H, GS), "y")


@pytest.mark.parametrize("I,k,gs,ties,with_delta", [
    (512, 1, 128, 0, True), (512, 100, 128, 0, False), (512, 512, 64, 0, True), (1024, 333, 32, 0, True),
    (12288, 6000, 128, 0, True),  # 24 gates per thread, 24 positions per workgroup
    (6144, 3072, 128, 16, True), (6144, 1000, 128, 64, True),  # blocks of exactly equal gates
])
def test_other_shapes_and_ties_bit_identical(C, I, k, gs, ties, with_delta):
    mats = _weights(I, seed=I + k, gs=gs, tie_blocks=ties)
    x, d, nw = _inputs(k, with_delta)
    want = _four_launches(C, mats, x, d, nw, k, gs)
    got, ws = _fused(C, mats, x, d, nw, k, gs)
    _assert_same(got, want, f"I={I} k={k} gs={gs} ties={ties}")
    C.dip_mlp_check(ws)


def test_repeated_calls_and_graph_replays(C):
    """One workspace across many calls (the barrier epochs advance every call) and across graph replays with
    eager work and other calls in between; every result equals the four launches on the same inputs."""
    mats = _weights(6144, seed=7)
    k = 3072
    ws = torch.zeros(C.dip_mlp_workspace_bytes(k), dtype=torch.uint8, device="cuda")
    for s in range(12):
        x, d, nw = _inputs(100 + s)
        got, _ = _fused(C, mats, x, d, nw, k, GS, ws=ws)
        _assert_same(got, _four_launches(C, mats, x, d, nw, k, GS), f"call {s}")
    x, d, nw = _inputs(200)
    want = _four_launches(C, mats, x, d, nw, k, GS)
    f16 = dict(dtype=torch.float16, device="cuda")
    out = {"x_out": torch.empty(H, **f16), "h_out": torch.empty(H, **f16), "gate": torch.empty(6144, **f16),
           "idx": torch.zeros(k, dtype=torch.int32, device="cuda"),
           "cnt": torch.zeros(1, dtype=torch.int32, device="cuda"), "h_sel": torch.empty(k, **f16),
           "y": torch.empty(H, **f16)}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        _fused(C, mats, x, d, nw, k, GS, ws=ws, out=out)
    other = _inputs(300)
    for rep in range(3):
        for t in out.values():
            t.zero_()
        g.replay()
        torch.cuda.synchronize()
        _assert_same(out, want, f"replay {rep}")
        _ = torch.zeros(1 << 20, device="cuda").sum()
        _fused(C, mats, *other, k, GS, ws=ws)  # an eager call on the same workspace between replays
    C.dip_mlp_check(ws)


def test_rejects_bad_arguments(C):
    mats = _weights(512, seed=9)
    x, d, nw = _inputs(9)
    with pytest.raises(RuntimeError):
        _fused(C, mats, x, d, nw, 513, GS)  # k > I
    with pytest.raises(RuntimeError):
        (gW, gS), u, dn = mats
        _fused(C, [(gW[:510].contiguous(), gS[:510].contiguous()), u, dn], x, d, nw, 10, GS)  # I not a multiple of 4
    small = [int4_problem(512, 1024, GS, seed=i) for i in range(3)]
    x1k = torch.zeros(1024, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):  # hidden size 1024
        _fused(C, [(p["Wq_d"], p["s_d"]) for p in small], x1k, None, torch.ones_like(x1k), 10, GS)
    with pytest.raises(RuntimeError):
        _fused(C, mats, x, d, nw, 10, GS, ws=torch.zeros(64, dtype=torch.uint8, device="cuda"))  # workspace
    buf = torch.empty(H + 8, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):
        _fused(C, mats, buf[1:1 + H], d, nw, 10, GS)  # misaligned x
