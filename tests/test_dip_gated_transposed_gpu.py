"""The DIP selection + down over the transposed copy of down_proj^T in the sparse accumulate's own order
(dip_select_down_ordered, dip_dense_down.hip), from gate and h = fp16(silu(gate) * up) of every channel,
against the row form (dip_select_gated_down, sparse_down.hip, from gate and up), which equals the top-k launch
followed by the gated sparse down:

  * indices, count and y equal the row form bit for bit: the Qwen3-1.7B MLP shape at k = 1 .. n, fp16 gates
    with boundary ties, tie-heavy gates (more than k channels at the threshold), NaN gates (fewer than k kept),
    ragged H with per-word scales, small n, and column counts whose plan has up to 64 row chunks;
  * channel counts past the row form's reach (up to 24576, the largest packed-row stride): y and the selection
    equal the indexed schedule's three launches;
  * y does not depend on whether the index outputs are requested; res_out = res + y as one binary16 add;
  * y also equals the indexed schedule's three launches (top-k, indexed up GEMV with the SiLU epilogue, sparse
    down) on the same gate and up, and lies within the sparse-down tolerance of the binary64 oracle;
  * shapes outside the kernel's limits are rejected (and report 0 LDS bytes).
"""
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import oracle as O

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


def _problem(ops, I, H, seed, gs):
    down = int4_problem(I, H, gs, seed=seed)  # down_proj^T: I rows of H
    Wt, St = ops.transposed_down_T(down["Wq_d"], down["s_d"], H)
    return down, Wt, St


def _row_form(C, gate, up, k, down, H, gs):
    idx = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    cnt = torch.zeros(1, dtype=torch.int32, device="cuda")
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(1, C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device="cuda")
    C.dip_select_gated_down_into(gate, up, k, down["Wq_d"], down["s_d"], idx, cnt, y, H, gs, ws)
    return idx, cnt, y


def _transposed(C, gate, up, k, Wt, St, H, gs, want_idx=True, res=None):
    h = torch.empty_like(gate)
    C.silu_mul_into(gate, up, h)  # h of every channel, the rounding of the SwiGLU epilogues
    idx = torch.full((k,), -7, dtype=torch.int32, device="cuda") if want_idx else None
    cnt = torch.zeros(1, dtype=torch.int32, device="cuda") if want_idx else None
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    res_out = torch.empty(H, dtype=torch.float16, device="cuda") if res is not None else None
    C.dip_select_down_ordered_into(gate, h, k, Wt, St, idx, cnt, y, gs, res, res_out)
    return idx, cnt, y, res_out


def _check(C, gate, up, k, down, Wt, St, H, gs, label):
    assert C.dip_select_down_ordered_lds_bytes(H, gate.numel(), k) > 0, label
    ri, rc, ry = _row_form(C, gate, up, k, down, H, gs)
    res = rnd((H,), 99, 4.0).cuda()
    ti, tc, ty, ro = _transposed(C, gate, up, k, Wt, St, H, gs, res=res)
    n_kept = int(rc.item())
    assert int(tc.item()) == n_kept, f"{label}: count"
    assert torch.equal(ti[:n_kept], ri[:n_kept]), f"{label}: indices"
    assert torch.equal(ty, ry), f"{label}: y differs from the row form"
    assert torch.equal(ro, (res.float() + ty.float()).half()), f"{label}: res_out"
    _, _, ty2, _ = _transposed(C, gate, up, k, Wt, St, H, gs, want_idx=False)
    assert torch.equal(ty2, ty), f"{label}: y depends on the index outputs"
    return ri[:n_kept], ty


@pytest.mark.parametrize("k", [1, 768, 1536, 3072, 4097, 6144])
def test_qwen_shape_equals_row_form(C, ops, k):
    I, H, gs = 6144, 2048, 128
    down, Wt, St = _problem(ops, I, H, seed=11 + k, gs=gs)
    gate, up = rnd((I,), 20 + k, 0.9).cuda(), rnd((I,), 30 + k).cuda()
    idx, y = _check(C, gate, up, k, down, Wt, St, H, gs, f"k={k}")
    # the indexed schedule's three launches on the same gate and up
    idx3 = torch.empty(k, dtype=torch.int32, device="cuda")
    cnt3 = torch.empty(1, dtype=torch.int32, device="cuda")
    C.topk_threshold_select_f16abs_into(gate, k, idx3, cnt3)
    assert torch.equal(idx3, idx)
    h_sel = torch.empty(k, dtype=torch.float16, device="cuda")
    C.silu_mul_indexed_into(gate, idx3, up.index_select(0, idx3.long()), h_sel)
    y3 = torch.empty(H, dtype=torch.float16, device="cuda")
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    C.gemv_w4a16_indexed_accumulate_into(down["Wq_d"], down["s_d"], idx3, h_sel, y3, H, gs, ws)
    assert torch.equal(y3, y), "differs from top-k + SiLU gating + sparse down"
    # and against the binary64 oracle on the same selection and h
    sel = idx.cpu().numpy()
    ref = O.sparse_accumulate_f64(down["Wq"][sel], down["s"][sel], h_sel.cpu().numpy(), H, gs)
    assert_close(y, ref, f"k={k} vs oracle")


def test_tie_heavy_and_nan_gates(C, ops):
    I, H, gs = 6144, 2048, 128
    down, Wt, St = _problem(ops, I, H, seed=41, gs=gs)
    up = rnd((I,), 42).cuda()
    g = torch.Generator().manual_seed(43)
    # few distinct magnitudes: far more than k channels sit at the threshold
    ties = (torch.randint(0, 6, (I,), generator=g).float() * 0.25 * torch.sign(torch.randn(I, generator=g))).half()
    _check(C, ties.cuda(), up, 3072, down, Wt, St, H, gs, "ties")
    # NaN gates are never selected: with 4000 NaNs only 2144 channels can be kept for k = 3072
    nan = rnd((I,), 44, 0.9)
    nan[torch.randperm(I, generator=g)[:4000]] = float("nan")
    idx, _ = _check(C, nan.cuda(), up, 3072, down, Wt, St, H, gs, "nan")
    assert idx.numel() == I - 4000


@pytest.mark.parametrize("I,H,gs,ks", [
    (1024, 256, 128, [1, 100, 512, 1024]),   # one slice: the plan's floor of 64 row chunks
    (640, 200, 8, [7, 320, 640]),            # ragged H, per-word scales (gs % 32 != 0)
    (32, 64, 32, [1, 17, 32]),               # one 32-channel chunk
    (8192, 1024, 64, [2048, 4096]),          # four 4-channel groups per thread
    (2048, 5120, 128, [1024]),               # wide H (Qwen3-14B hidden)
])
def test_other_shapes_equal_row_form(C, ops, I, H, gs, ks):
    down, Wt, St = _problem(ops, I, H, seed=I + H + gs, gs=gs)
    for k in ks:
        gate, up = rnd((I,), 50 + k, 0.9).cuda(), rnd((I,), 60 + k).cuda()
        _check(C, gate, up, k, down, Wt, St, H, gs, f"I={I} H={H} gs={gs} k={k}")


@pytest.mark.parametrize("I,H,gs,ks", [
    (24576, 2048, 128, [512, 2048]),         # 12 packed-row KB per wave: the largest row stride the kernel takes
    (20480, 512, 64, [1000]),                # 10 KB rows, gs 64
    (10240, 1024, 128, [5120]),              # 5 KB rows
])
def test_wide_rows_equal_indexed_schedule(C, ops, I, H, gs, ks):
    """Channel counts past the row form's reach (it takes n <= 6144): y and the selection against the indexed
    schedule's three launches (top-k, SiLU gating of the selected channels, indexed sparse down) and y against the
    binary64 oracle on the same selection."""
    down, Wt, St = _problem(ops, I, H, seed=I + H, gs=gs)
    for k in ks:
        assert C.dip_select_down_ordered_lds_bytes(H, I, k) > 0, (I, H, k)
        gate, up = rnd((I,), 70 + k, 0.9).cuda(), rnd((I,), 80 + k).cuda()
        ti, tc, ty, _ = _transposed(C, gate, up, k, Wt, St, H, gs)
        idx3 = torch.empty(k, dtype=torch.int32, device="cuda")
        cnt3 = torch.empty(1, dtype=torch.int32, device="cuda")
        C.topk_threshold_select_f16abs_into(gate, k, idx3, cnt3)
        assert int(tc.item()) == int(cnt3.item()) == k
        assert torch.equal(ti, idx3), f"I={I} k={k}: indices"
        h_sel = torch.empty(k, dtype=torch.float16, device="cuda")
        C.silu_mul_indexed_into(gate, idx3, up.index_select(0, idx3.long()), h_sel)
        y3 = torch.empty(H, dtype=torch.float16, device="cuda")
        ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
        C.gemv_w4a16_indexed_accumulate_into(down["Wq_d"], down["s_d"], idx3, h_sel, y3, H, gs, ws)
        assert torch.equal(ty, y3), f"I={I} H={H} k={k}: differs from the indexed schedule"
        sel = idx3.cpu().numpy()
        ref = O.sparse_accumulate_f64(down["Wq"][sel], down["s"][sel], h_sel.cpu().numpy(), H, gs)
        assert_close(ty, ref, f"I={I} H={H} k={k} vs oracle")


def test_outside_limits_rejected(C, ops):
    """H = 256 (one column slice) with n = k = 24576: the row form's plan has 128 row chunks (> 64)."""
    I, H, gs = 24576, 256, 128
    assert C.dip_select_down_ordered_lds_bytes(H, I, I) == 0
    assert C.dip_select_down_ordered_lds_bytes(2048, 6144, 3072) > 0
    assert C.dip_select_down_ordered_lds_bytes(2048, 6143, 3072) == 0  # n not a multiple of 32
    Wt = torch.zeros(H, I // 2, dtype=torch.uint8, device="cuda")
    St = torch.ones(H // gs, I, device="cuda")
    gate, up = rnd((I,), 1).cuda(), rnd((I,), 2).cuda()
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="row chunks"):
        C.dip_select_down_ordered_into(gate, up, I, Wt, St, None, None, y, gs)
    with pytest.raises(RuntimeError):
        C.dip_select_down_ordered_into(gate, up, 0, Wt, St, None, None, y, gs)
