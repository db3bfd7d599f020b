"""One-launch DIP selection + down projection over transposed resident weights (dip_dense_down.hip).

The reference's DIP down projection (generate.py:304-308: h = fp16(silu(gate) * up) over the rule-A top-k
selection of |gate|, then gemv_w4a16_sparse_accumulate over down_proj^T rows) computed as a GEMV over a
transposed copy of the same quantized values:
  * the transposed copy holds exactly the transpose of down_proj^T's INT4 values and scales;
  * the gate|up GEMV's SwiGLU form that also writes the gate equals the interleaved gate|up GEMV and the SwiGLU
    GEMV, bit for bit;
  * indices and count equal the oracle's rule-A selection and the top-k kernel's, including tie-heavy gates
    where more than k channels reach the threshold and NaN gates;
  * y within the sparse-down tolerance of the binary64 oracle over that selection, identical with and without
    the index outputs, and close to the position-partitioned sparse accumulate on the same (idx, h);
  * coefficients across many binades (the power-of-two scale and the hi / lo split), k = 1 and k = n, ragged
    and small sizes, rejections.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import decoder as OD
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


def _gated_all(C, gate, up):
    h = torch.empty_like(gate)
    C.silu_mul_into(gate, up, h)
    return h


def _problem(ops, I, H, seed, gs=128):
    down = int4_problem(I, H, gs, seed=seed)  # down_proj^T: I rows of H
    Wt, St = ops.transposed_down_T(down["Wq_d"], down["s_d"], H)
    return down, Wt, St


def test_transposed_copy_is_the_transpose(ops):
    """Wt unpacks to the transpose of down_proj^T's INT4 values; St is the transposed scale matrix."""
    from soinfer.quant import pack

    I, H = 640, 384
    down, Wt, St = _problem(ops, I, H, seed=3)
    assert Wt.shape == (H, I // 2) and St.shape == (H // 128, I)
    q = torch.from_numpy(down["q"][:, :H]).cuda()
    assert torch.equal(pack.unpack_int4(Wt, I), q.t().contiguous())
    assert torch.equal(St, down["s_d"].t().contiguous())


def test_rmsnorm_swiglu_gate_equals_gate_up_and_swiglu(C):
    """gate_out = the gate half of the interleaved gate|up GEMV; y = the SwiGLU form's output."""
    H, I = 2048, 1024
    x, d = rnd((H,), 61).cuda(), rnd((H,), 62).cuda()
    nw = (rnd((H,), 63) * 0.1 + 1).half().cuda()
    g = int4_problem(I, H, 128, seed=64)
    u = int4_problem(I, H, 128, seed=65)
    t = torch.arange(I // 4)
    perm = torch.stack([4 * t + i for i in range(4)] + [I + 4 * t + i for i in range(4)], 1).reshape(-1).cuda()
    W = torch.cat([g["Wq_d"], u["Wq_d"]]).index_select(0, perm).contiguous()
    S = torch.cat([g["s_d"], u["s_d"]]).index_select(0, perm).contiguous()
    gate, y = torch.empty(I, dtype=torch.float16, device="cuda"), torch.empty(I, dtype=torch.float16, device="cuda")
    xo = torch.empty_like(x)
    C.gemv_w4a16_rmsnorm_swiglu_gate_into(W, S, x, d, nw, 1e-6, xo, gate, y, H, 128)
    gref, uref = torch.empty_like(gate), torch.empty_like(gate)
    C.gemv_w4a16_rmsnorm_gate_up_into(W, S, x, d, nw, 1e-6, None, gref, uref, H, 128)
    yref = torch.empty_like(y)
    C.gemv_w4a16_rmsnorm_into(W, S, x, d, nw, 1e-6, None, None, yref, H, 128, True)
    assert torch.equal(gate, gref) and torch.equal(y, yref)
    assert torch.equal(y, _gated_all(C, gref, uref))
    assert torch.equal(xo, (x.float() + d.float()).half())


@pytest.mark.parametrize("I,H,k,ties", [(6144, 2048, 3072, False), (6144, 2048, 768, True), (6144, 2048, 1536, False),
                                        (6144, 2048, 6144, False), (6144, 2048, 1, False), (1024, 256, 333, True),
                                        (8192, 1024, 4096, True), (9728, 2048, 4864, False), (96, 384, 50, False),
                                        (3008, 2176, 1111, False), (17408, 5120, 8704, False),
                                        (24576, 1024, 12288, True)])
def test_dense_down_matches_oracle_and_topk(C, ops, I, H, k, ties):
    """Selection = the oracle's rule A = the top-k kernel; y = the binary64 sum over it within the sparse-down
    tolerance, the same without the index outputs, and close to the sparse accumulate on the same (idx, h)."""
    down, Wt, St = _problem(ops, I, H, seed=81 + k)
    g = rnd((I,), 82 + k) * 2
    if ties:
        g = ((g.float() * 4).round() / 4).half()
    u = rnd((I,), 83 + k) * 2
    gate, up = g.cuda(), u.cuda()
    h_all = _gated_all(C, gate, up)
    y, idx, cnt = ops.dip_select_dense_down(gate, h_all, k, Wt, St, 128)
    idx2 = torch.empty(k, dtype=torch.int32, device="cuda")
    cnt2 = torch.empty(1, dtype=torch.int32, device="cuda")
    C.topk_threshold_select_f16abs_into(gate, k, idx2, cnt2)
    assert torch.equal(idx, idx2) and torch.equal(cnt, cnt2)
    ref_idx = O.topk_rule_a(np.abs(g.float().numpy()), k)
    assert int(cnt.item()) == ref_idx.size == k
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    h = h_all.index_select(0, idx.long())
    assert_close(h, OD.silu_mul(g.numpy()[ref_idx], u.numpy()[ref_idx]).astype(np.float64), "gated h")
    y_ref = O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h.cpu().numpy(), H, 128)
    assert_close(y, y_ref, f"dense down I={I} H={H} k={k}")
    y_noidx, _, _ = ops.dip_select_dense_down(gate, h_all, k, Wt, St, 128, with_indices=False)
    assert torch.equal(y, y_noidx), "y depends on whether the index list is written"
    ws = torch.zeros(max(1, C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device="cuda")
    y_sd = torch.empty(H, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_indexed_accumulate_into(down["Wq_d"], down["s_d"], idx, h, y_sd, H, 128, ws)
    scale = max(float(y_sd.float().abs().max()), 1e-30)
    assert float((y.float() - y_sd.float()).abs().max()) <= 2e-3 * scale
    # a second launch gives the same bytes (no state carried between launches)
    assert torch.equal(ops.dip_select_dense_down(gate, h_all, k, Wt, St, 128)[0], y)


@pytest.mark.parametrize("k", [1, 700, 2047, 2048, 2049, 3000, 6143])
def test_dense_down_ties_beyond_k(C, ops, k):
    """Gates of three magnitudes only: more than k channels reach the threshold and rule A keeps the first k in
    index order (the cut falls inside a tie group, in a wave and position that vary with k)."""
    I, H = 6144, 2048
    down, Wt, St = _problem(ops, I, H, seed=500 + k)
    mags = torch.tensor([0.5, 1.0, 2.0]).repeat_interleave(I // 3)
    perm = torch.randperm(I, generator=torch.Generator().manual_seed(k))
    sign = torch.where(torch.rand(I, generator=torch.Generator().manual_seed(k + 1)) < 0.5, -1.0, 1.0)
    g = (mags[perm] * sign).half()
    u = rnd((I,), 600 + k)
    gate, up = g.cuda(), u.cuda()
    absg = np.abs(g.float().numpy())
    ref_idx = O.topk_rule_a(absg, k)
    if k != 2048:
        assert int((absg >= absg[ref_idx].min()).sum()) > k, "the case must have ties beyond k"
    h_all = _gated_all(C, gate, up)
    y, idx, cnt = ops.dip_select_dense_down(gate, h_all, k, Wt, St, 128)
    assert int(cnt.item()) == k and np.array_equal(idx.cpu().numpy(), ref_idx)
    h = h_all.index_select(0, idx.long())
    assert_close(y, O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h.cpu().numpy(), H, 128),
                 f"ties k={k}")


def test_dense_down_fewer_than_k_selected(C, ops):
    """NaN gates are never selected: with fewer than k valid channels the count says how many, only those
    indices are written, and y sums over exactly those rows."""
    I, H, k = 1024, 256, 1019
    down, Wt, St = _problem(ops, I, H, seed=91)
    g = rnd((I,), 92) * 2
    g[torch.arange(3, I, 97)] = float("nan")  # 11 NaN gates: 1013 valid channels
    u = rnd((I,), 93) * 2
    h_all = _gated_all(C, g.cuda(), u.cuda())
    idx = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    cnt = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    C.dip_select_dense_down_into(g.cuda(), h_all, k, Wt, St, idx, cnt, y, 128)
    ref_idx = O.topk_rule_a(np.abs(g.float().numpy()), k)
    n = int(cnt.item())
    assert n == ref_idx.size == 1013
    assert np.array_equal(idx[:n].cpu().numpy(), ref_idx)
    assert bool((idx[n:] == -7).all()), "entries past the count were written"
    h = h_all.index_select(0, idx[:n].long())
    assert_close(y, O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h.cpu().numpy(), H, 128),
                 "NaN gates")


@pytest.mark.parametrize("spread", [0, 8, 20])
def test_dense_down_coefficients_across_binades(C, ops, spread):
    """h spanning 2^-spread .. 2^spread (and tiny / large scales): the power-of-two scale and the binary16
    hi / lo split keep every coefficient h * s to fp32 accuracy, so y matches the binary64 oracle as closely as
    the fp32 sparse accumulate does."""
    I, H, k = 2048, 512, 1024
    down, Wt, St = _problem(ops, I, H, seed=700 + spread)
    g = rnd((I,), 701) * 2
    e = torch.randint(-spread, spread + 1, (I,), generator=torch.Generator().manual_seed(702)).float()
    hv = (rnd((I,), 703).float() * torch.exp2(e)).clamp(-6e4, 6e4).half()
    gate, h_all = g.cuda(), hv.cuda()
    y, idx, cnt = ops.dip_select_dense_down(gate, h_all, k, Wt, St, 128)
    sel = idx.long().cpu().numpy()
    h = hv.numpy()[sel]
    y_ref = O.sparse_accumulate_f64(down["Wq"][sel], down["s"][sel], h, H, 128)
    assert_close(y, y_ref, f"binades spread={spread}")
    ws = torch.zeros(max(1, C.sparse_accumulate_workspace_bytes(H, k)), dtype=torch.uint8, device="cuda")
    y_sd = torch.empty(H, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_indexed_accumulate_into(down["Wq_d"], down["s_d"], idx, h_all.index_select(0, idx.long()), y_sd,
                                         H, 128, ws)
    err = (y.double().cpu() - torch.from_numpy(y_ref)).abs().max().item()
    err_sd = (y_sd.double().cpu() - torch.from_numpy(y_ref)).abs().max().item()
    ulp = float(np.abs(y_ref).max()) * 2.0 ** -10
    assert err <= err_sd + ulp, (err, err_sd)


def test_dense_down_rejections(C, ops):
    I, H = 1024, 256
    down, Wt, St = _problem(ops, I, H, seed=41)
    gate, h = rnd((I,), 42).cuda(), rnd((I,), 43).cuda()
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):
        C.dip_select_dense_down_into(gate, h, 0, Wt, St, None, None, y, 128)
    with pytest.raises(RuntimeError, match="group_size"):
        C.dip_select_dense_down_into(gate, h, 10, Wt, St, None, None, y, 24)
    with pytest.raises(RuntimeError, match="Wt"):
        C.dip_select_dense_down_into(gate, h, 10, Wt[:, :100], St, None, None, y, 128)
    g_odd = rnd((I - 8,), 44).cuda()
    W_odd = torch.zeros(H, (I - 8) // 2, dtype=torch.uint8, device="cuda")
    S_odd = torch.zeros(H // 128, I - 8, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        C.dip_select_dense_down_into(g_odd, g_odd, 10, W_odd, S_odd, None, None, y, 128)
    n_big = 24576 + 32  # past the 12 four-channel groups per thread
    g_big = torch.zeros(n_big, dtype=torch.float16, device="cuda")
    W_big = torch.zeros(H, n_big // 2, dtype=torch.uint8, device="cuda")
    S_big = torch.zeros(H // 128, n_big, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 32"):
        C.dip_select_dense_down_into(g_big, g_big, 10, W_big, S_big, None, None, y, 128)


def test_dense_down_unselected_infinite_h(C, ops):
    """An unselected channel whose h overflowed to +-inf (or is NaN) must not change y: the power-of-two scale
    comes from the finite coefficients only, so y over the selected channels matches the oracle and is finite."""
    I, H, k = 2048, 512, 1024
    down, Wt, St = _problem(ops, I, H, seed=901)
    g = rnd((I,), 902) * 2
    hv = rnd((I,), 903) * 4
    absg = np.abs(g.float().numpy())
    ref_idx = O.topk_rule_a(absg, k)
    unsel = np.setdiff1d(np.arange(I), ref_idx)
    hv[int(unsel[0])] = float("inf")
    hv[int(unsel[len(unsel) // 2])] = float("-inf")
    hv[int(unsel[-1])] = float("nan")
    y, idx, cnt = ops.dip_select_dense_down(g.cuda(), hv.cuda(), k, Wt, St, 128)
    assert int(cnt.item()) == k and np.array_equal(idx.cpu().numpy(), ref_idx)
    y_ref = O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], hv.numpy()[ref_idx], H, 128)
    assert_close(y, y_ref, "unselected inf / NaN h")


@pytest.mark.parametrize("I,H,k", [(1024, 200, 333), (2048, 2056, 1000), (1024, 204, 512), (512, 36, 100)])
def test_dense_down_group_size_8_ragged_h(C, ops, I, H, k):
    """group_size 8 with H not a multiple of 128 (grids of 25, 257, 26 and 5 workgroups, not multiples of 8: the
    identity tile order) and H not a multiple of 8 (a last tile with rows past H): selection and y against the
    oracle, and nothing written past y[H - 1] or res_out[H - 1]."""
    gs = 8
    down = int4_problem(I, H, gs, seed=950 + H)
    Wt, St = ops.transposed_down_T(down["Wq_d"], down["s_d"], H)
    assert St.shape == (-(-H // gs), I)
    g = rnd((I,), 951 + H) * 2
    u = rnd((I,), 952 + H) * 2
    gate, up = g.cuda(), u.cuda()
    h_all = _gated_all(C, gate, up)
    sentinel = 0x7bff  # fp16 65504, never a value of these sums
    y_buf = torch.full((H + 24,), sentinel, dtype=torch.int16, device="cuda").view(torch.float16)
    r_buf = torch.full((H + 24,), sentinel, dtype=torch.int16, device="cuda").view(torch.float16)
    res = rnd((H,), 953 + H).cuda()
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    cnt = torch.empty(1, dtype=torch.int32, device="cuda")
    C.dip_select_dense_down_into(gate, h_all, k, Wt, St, idx, cnt, y_buf[:H], gs, res, r_buf[:H])
    ref_idx = O.topk_rule_a(np.abs(g.float().numpy()), k)
    assert int(cnt.item()) == k and np.array_equal(idx.cpu().numpy(), ref_idx)
    h = h_all.index_select(0, idx.long())
    y_ref = O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h.cpu().numpy(), H, gs)
    assert_close(y_buf[:H], y_ref, f"gs=8 H={H}")
    assert torch.equal(r_buf[:H], (res.float() + y_buf[:H].float()).half()), "residual output"
    tail = torch.full((24,), sentinel, dtype=torch.int16, device="cuda")
    assert torch.equal(y_buf[H:].view(torch.int16), tail), "y written past H"
    assert torch.equal(r_buf[H:].view(torch.int16), tail), "res_out written past H"
