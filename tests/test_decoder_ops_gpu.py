"""Decode-step glue on the GPU against the CPU oracle (oracle/decoder.py), op by op on identical inputs
(counterpart of the reference's tests/test_m2_kernels.py and test_m5_kernels.py for rmsnorm, gemv_fp16,
rope, kv_cache_append).

Tolerance for floating-point outputs: the rule of tests/helpers.py (1e-3 relative). Integer / byte outputs
(argmax index, KV rows, embedding rows) are compared exactly. Engine forms (device position / token,
fused residual add, fused q/k norm + RoPE + append) are checked against the separate reference-named ops,
bit for bit where they share the arithmetic.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import decoder as OD
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


@pytest.fixture(scope="module")
def C(cuda):
    from soinfer import _C

    return _C


def rnd(shape, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).half()


@pytest.mark.parametrize("rows,hidden", [(1, 2048), (16, 128), (8, 128), (3, 1000), (1, 6)])
def test_rmsnorm_matches_oracle(ops, rows, hidden):
    x, w = rnd((rows, hidden), 1, 3.0), rnd((hidden,), 2) + 1
    y = ops.rmsnorm(x.cuda(), w.half().cuda(), 1e-6)
    ref = OD.rmsnorm(x.numpy(), w.numpy(), 1e-6)
    assert_close(y, ref.astype(np.float64), f"rmsnorm {rows}x{hidden}")


def test_rmsnorm_rejects_bad_arguments(ops):
    with pytest.raises(RuntimeError):
        ops.rmsnorm(rnd((2, 7), 0).cuda(), rnd((7,), 1).cuda())  # odd hidden (reference requires even)
    with pytest.raises(RuntimeError):
        ops.rmsnorm(rnd((2, 8), 0).cuda(), rnd((6,), 1).cuda())  # weight shape


@pytest.mark.parametrize("hidden", [2048, 1000])
def test_residual_rmsnorm_equals_add_then_rmsnorm(C, ops, hidden):
    x, d, w = rnd((hidden,), 3), rnd((hidden,), 4), rnd((hidden,), 5) + 1
    xd, dd, wd = x.cuda(), d.cuda(), w.half().cuda()
    out = torch.empty_like(xd)
    C.residual_rmsnorm_(xd, dd, wd, out, 1e-6)
    s = (x.float() + d.float()).half()  # binary16 add, rounded once
    assert torch.equal(xd.cpu(), s), "x must hold the binary16 sum"
    assert torch.equal(out, ops.rmsnorm(s.cuda().view(1, -1), wd, 1e-6).view(-1))
    assert np.array_equal(s.numpy(), OD.residual_add(x.numpy(), d.numpy()))


@pytest.mark.parametrize("heads,hd,pos", [(16, 128, 0), (16, 128, 1), (8, 128, 2047), (4, 64, 77)])
def test_rope_matches_oracle(ops, heads, hd, pos):
    x = rnd((heads, hd), 6 + pos, 2.0)
    cos_v, sin_v = ops.precompute_rope_cos_sin(hd, 1e6, pos, "cuda")
    y = ops.apply_rope(x.cuda(), cos_v, sin_v)
    ref = OD.rope(x.numpy(), hd, 1e6, pos)
    assert_close(y, ref.astype(np.float64), f"rope pos {pos}")
    if pos == 0:
        assert torch.equal(y.cpu(), x), "angle 0 is the identity"


def test_rope_tables_match_single_position(ops):
    cos_t, sin_t = ops.rope_tables(128, 1e6, 300, "cuda")
    for p in (0, 1, 17, 299):
        c, s = ops.precompute_rope_cos_sin(128, 1e6, p, "cuda")
        assert torch.equal(cos_t[p], c) and torch.equal(sin_t[p], s)


def test_kv_cache_append_exact(ops):
    kc = torch.zeros(8, 64, 128, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    k, v = rnd((8, 128), 10).cuda(), rnd((8, 128), 11).cuda()
    ops.kv_cache_append(kc, vc, k, v, 37)
    assert torch.equal(kc[:, 37], k) and torch.equal(vc[:, 37], v)
    assert kc[:, :37].abs().sum() == 0 and kc[:, 38:].abs().sum() == 0
    with pytest.raises(RuntimeError):
        ops.kv_cache_append(kc, vc, k, v, 64)  # pos == max_seq


@pytest.mark.parametrize("N,K", [(151936 // 16, 2048), (1000, 256), (37, 2048), (5, 24), (7, 100)])
def test_gemv_fp16_matches_oracle(ops, C, N, K):
    W, x = rnd((N, K), 12, 0.05), rnd((K,), 13)
    ref = OD.gemv_f16(W.numpy(), x.numpy())
    if K % 8 == 0:
        y = ops.gemv_fp16_v3(W.cuda(), x.cuda())
    else:
        y = torch.empty(N, dtype=torch.float16, device="cuda")
        C.gemv_f16_into(W.cuda(), x.cuda(), y)
    assert_close(y, ref.astype(np.float64), f"gemv_f16 {N}x{K}")


def test_gemv_fp16_v3_requires_k_multiple_of_8(ops):
    with pytest.raises(RuntimeError):
        ops.gemv_fp16_v3(rnd((4, 12), 0).cuda(), rnd((12,), 1).cuda())


# (6144, 2048): the Qwen3-1.7B MLP (full tiles, 4 passes); (2048, 6144): 12 passes; (4095, 256): a ragged last
# tile; (33, 64): one partial pass; (7, 8): a single chunk per row
@pytest.mark.parametrize("I,H", [(6144, 2048), (2048, 6144), (4095, 256), (33, 64), (7, 8)])
def test_swiglu_gate_up_matches_oracle(ops, I, H):
    Wg, Wu, x = rnd((I, H), 30 + I, 0.05), rnd((I, H), 31 + H, 0.05), rnd((H,), 32)
    h = ops.swiglu_gate_up(Wg.cuda(), Wu.cuda(), x.cuda())
    assert h.dtype == torch.float16 and h.shape == (I,)
    assert_close(h, OD.swiglu_gate_up(Wg.numpy(), Wu.numpy(), x.numpy()).astype(np.float64), f"swiglu {I}x{H}")


def test_swiglu_gate_up_unaligned_rows(ops):
    """Weights starting 8 bytes into their storage take the per-element kernel; same results to the tolerance."""
    I, H = 100, 512
    Wg_s, Wu_s, x = rnd((I * H + 4,), 33, 0.05), rnd((I * H + 4,), 34, 0.05), rnd((H,), 35)
    Wg, Wu = Wg_s[4:].view(I, H), Wu_s[4:].view(I, H)
    h = ops.swiglu_gate_up(Wg_s.cuda()[4:].view(I, H), Wu_s.cuda()[4:].view(I, H), x.cuda())
    assert_close(h, OD.swiglu_gate_up(Wg.numpy(), Wu.numpy(), x.numpy()).astype(np.float64), "swiglu unaligned")


def test_swiglu_gate_up_rejects_bad_arguments(ops):
    W, x = rnd((16, 64), 36).cuda(), rnd((64,), 37).cuda()
    with pytest.raises(RuntimeError, match="same shape"):
        ops.swiglu_gate_up(W, rnd((8, 64), 38).cuda(), x)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        ops.swiglu_gate_up(rnd((4, 12), 0).cuda(), rnd((4, 12), 1).cuda(), rnd((12,), 2).cuda())
    with pytest.raises(RuntimeError, match="matching"):
        ops.swiglu_gate_up(W, W, rnd((32,), 39).cuda())
    with pytest.raises(RuntimeError):
        ops.swiglu_gate_up(W.float(), W.float(), x)


def test_fused_swiglu_mlp_equals_gate_up_then_down(ops):
    H, I = 2048, 6144
    Wg, Wu, Wd, x = (rnd((I, H), 40, 0.05).cuda(), rnd((I, H), 41, 0.05).cuda(), rnd((H, I), 42, 0.02).cuda(),
                     rnd((H,), 43).cuda())
    y = ops.fused_swiglu_mlp(Wg, Wu, Wd, x)
    assert torch.equal(y, ops.gemv_fp16_v3(Wd, ops.swiglu_gate_up(Wg, Wu, x)))
    # against the binary64 MLP: h is rounded to fp16 between the two kernels, so each h_j may carry up to one
    # binary16 rounding (2^-11 relative) plus its fp32 sums' error; the down sum propagates that as at most
    # 2^-10 sum_j |Wd_ij h_j|, and y itself rounds once more (2^-11 |y_i|)
    Wg64, Wu64, Wd64 = (t.cpu().numpy().astype(np.float64) for t in (Wg, Wu, Wd))
    x64 = x.cpu().numpy().astype(np.float64)
    g = Wg64 @ x64
    h64 = g / (1 + np.exp(-g)) * (Wu64 @ x64)
    y64 = Wd64 @ h64
    bound = 2.0 ** -10 * (np.abs(Wd64) @ np.abs(h64)) + 2.0 ** -11 * np.abs(y64) + 2.0 ** -24
    err = np.abs(y.cpu().numpy().astype(np.float64) - y64)
    assert (err <= bound).all(), f"fused_swiglu_mlp: {int((err > bound).sum())} outputs beyond the propagated bound"


def test_fused_qkv_projection_equals_separate_gemvs(ops):
    H, q_dim, kv_dim = 2048, 2048, 1024
    Wq, Wk, Wv = rnd((q_dim, H), 44, 0.05), rnd((kv_dim, H), 45, 0.05), rnd((kv_dim, H), 46, 0.05)
    x = rnd((H,), 47).cuda()
    qkv_W = ops.concat_qkv_weights(Wq.cuda(), Wk.cuda(), Wv.cuda())
    assert qkv_W.shape == (q_dim + 2 * kv_dim, H) and qkv_W.is_contiguous()
    q, k, v = ops.fused_qkv_projection(qkv_W, x, q_dim, kv_dim)
    # each output row is the same row-independent GEMV whichever matrix holds the row
    assert torch.equal(q, ops.gemv_fp16_v3(Wq.cuda(), x))
    assert torch.equal(k, ops.gemv_fp16_v3(Wk.cuda(), x))
    assert torch.equal(v, ops.gemv_fp16_v3(Wv.cuda(), x))
    with pytest.raises(RuntimeError):
        ops.fused_qkv_projection(qkv_W, x, q_dim, kv_dim + 1)


def argmax_dev(C, x):
    ws = torch.empty(C.argmax_workspace_bytes(x.numel()), dtype=torch.uint8, device="cuda")
    out = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    C.argmax_f16_into(x, out, None, None, ws)
    return int(out.item())


def test_argmax_first_maximum(C):
    x = rnd((151936,), 14)
    assert argmax_dev(C, x.cuda()) == OD.argmax_first(x.numpy()) == int(torch.argmax(x.float()))
    t = torch.zeros(10000, dtype=torch.float16)
    t[[17, 4099, 9000]] = 3.0  # ties in different workgroups -> lowest index
    assert argmax_dev(C, t.cuda()) == 17
    t[5000] = float("nan")
    assert argmax_dev(C, t.cuda()) == 5000 == OD.argmax_first(t.numpy())
    assert argmax_dev(C, torch.full((1,), -2.0, dtype=torch.float16).cuda()) == 0
    odd = rnd((9999,), 24)  # not a multiple of 8: element-wise path
    odd[[3, 9998]] = 9.0
    assert argmax_dev(C, odd.cuda()) == 3


def test_argmax_log(C):
    x = rnd((3000,), 15).cuda()
    ws = torch.empty(C.argmax_workspace_bytes(3000), dtype=torch.uint8, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    log = torch.full((2,), -1, dtype=torch.int32, device="cuda")
    n = torch.zeros(1, dtype=torch.int32, device="cuda")
    for _ in range(3):  # the third call finds the log full and leaves it unchanged
        C.argmax_f16_into(x, out, log, n, ws)
    want = int(torch.argmax(x.float()))
    assert log.tolist() == [want, want] and n.item() == 2 and out.item() == want


def test_silu_mul_matches_oracle(C):
    g, u = rnd((6144,), 16, 3.0), rnd((6144,), 17)
    out = torch.empty(6144, dtype=torch.float16, device="cuda")
    C.silu_mul_into(g.cuda(), u.cuda(), out)
    assert_close(out, OD.silu_mul(g.numpy(), u.numpy()).astype(np.float64), "silu_mul")
    ref_torch = (torch.nn.functional.silu(g.float()) * u.float()).half()
    diff = (out.cpu().float() - ref_torch.float()).abs()
    assert (diff <= 1e-3 * ref_torch.float().abs() + 1e-6).all(), "torch F.silu glue agrees to the fp16 rounding"


def test_silu_mul_indexed(C):
    g, u = rnd((512,), 18, 2.0), rnd((5,), 19)
    idx = torch.tensor([3, 0, 511, 100, 512], dtype=torch.int32)  # 512 is out of range -> NaN
    out = torch.empty(5, dtype=torch.float16, device="cuda")
    C.silu_mul_indexed_into(g.cuda(), idx.cuda(), u.cuda(), out)
    ref = OD.silu_mul(g.numpy()[idx[:4].numpy()], u.numpy()[:4])
    assert_close(out[:4], ref.astype(np.float64), "silu_mul_indexed")
    assert torch.isnan(out[4])


def test_embed_lookup(C):
    table = rnd((1000, 256), 20).cuda()
    out = torch.empty(256, dtype=torch.float16, device="cuda")
    for t in (0, 999, 417):
        C.embed_lookup_into(table, torch.tensor([t], dtype=torch.int32, device="cuda"), out)
        assert torch.equal(out, table[t])
    C.embed_lookup_into(table, torch.tensor([1000], dtype=torch.int32, device="cuda"), out)
    assert out.abs().sum() == 0, "an out-of-range token gives zeros"


@pytest.mark.parametrize("NQ,NKV,hd,S,pos", [(16, 8, 128, 2048, 0), (16, 8, 128, 2048, 1500), (4, 2, 64, 64, 63)])
def test_qk_norm_rope_append_equals_separate_ops(C, ops, NQ, NKV, hd, S, pos):
    qkv = rnd(((NQ + 2 * NKV) * hd,), 21 + pos, 2.0).cuda()
    qn, kn = (rnd((hd,), 22) * 0.1 + 1).half().cuda(), (rnd((hd,), 23) * 0.1 + 1).half().cuda()
    cos_t, sin_t = ops.rope_tables(hd, 1e6, S, "cuda")
    kc = torch.zeros(NKV, S, hd, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    q_out = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
    C.qk_norm_rope_append(qkv, qn, kn, cos_t, sin_t, torch.tensor([pos], dtype=torch.int32, device="cuda"), q_out,
                          kc, vc, 1e-6)
    q = qkv[:NQ * hd].view(NQ, hd).contiguous()
    k = qkv[NQ * hd:(NQ + NKV) * hd].view(NKV, hd).contiguous()
    v = qkv[(NQ + NKV) * hd:].view(NKV, hd)
    c, s = ops.precompute_rope_cos_sin(hd, 1e6, pos, "cuda")
    q_ref = ops.apply_rope(ops.qk_norm(q, qn), c, s)
    k_ref = ops.apply_rope(ops.qk_norm(k, kn), c, s)
    # same binary16 rounding points; only the fp32 sum order of the norm differs
    # Two binary16 rounding points (norm, then RoPE). One ulp of the normalised value (fp32 rsqrt here,
    # binary64 in the oracle) moves a RoPE output by up to ~1e-3 of the row scale, which can be large relative
    # to an output that cancels to near zero, so the bound is normalised by the row scale.
    ref_q = OD.rope(OD.rmsnorm(q.cpu().numpy(), qn.cpu().numpy(), 1e-6), hd, 1e6, pos).astype(np.float64)
    err = np.abs(q_out.float().cpu().numpy() - ref_q)
    assert err.max() <= 2e-3 * np.abs(ref_q).max(), f"q: normalized error {err.max() / np.abs(ref_q).max():.2e}"
    assert (q_out.float() - q_ref.float()).abs().max() <= 2e-3 * q_ref.float().abs().max()
    assert (kc[:, pos].float() - k_ref.float()).abs().max() <= 2e-3 * k_ref.float().abs().max()
    assert torch.equal(vc[:, pos], v)
    C.qk_norm_rope_append(qkv, qn, kn, cos_t, sin_t, torch.tensor([S], dtype=torch.int32, device="cuda"), q_out,
                          kc, vc, 1e-6)  # position past the cache: nothing written, no fault


@pytest.mark.parametrize("NQ,NKV,hd,S,L", [(16, 8, 128, 2048, 1), (16, 8, 128, 2048, 192), (16, 8, 128, 2048, 2048),
                                           (4, 2, 64, 64, 40)])
def test_decode_attention_at_matches_oracle(C, NQ, NKV, hd, S, L):
    q = rnd((NQ, hd), 30).cuda()
    kc, vc = rnd((NKV, S, hd), 31).cuda(), rnd((NKV, S, hd), 32).cuda()
    ws = torch.zeros(max(1, C.decode_attention_workspace_bytes(NQ, NKV, hd, S)), dtype=torch.uint8, device="cuda")
    out = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
    C.decode_attention_at(q, kc, vc, torch.tensor([L - 1], dtype=torch.int32, device="cuda"), out, ws)
    ref = O.decode_attention_f64(q.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy(), L)
    assert_close(out, ref, f"attention at len {L}")


def test_topk_f16abs_equals_fp32_abs(C, ops):
    g = rnd((6144,), 40, 0.9)
    g[::97] = 0.0
    g[1::89] = -g[2::89][: g[1::89].numel()]  # +/- pairs: equal |g|
    gd = g.cuda()
    for k in (768, 1536, 3072, 6144, 1):
        idx = torch.empty(k, dtype=torch.int32, device="cuda")
        cnt = torch.empty(1, dtype=torch.int32, device="cuda")
        C.topk_threshold_select_f16abs_into(gd, k, idx, cnt)
        ref = ops.topk_threshold_select(gd.float().abs().contiguous(), k)
        assert torch.equal(idx, ref) and cnt.item() == k
        assert np.array_equal(idx.cpu().numpy(), O.topk_rule_a(np.abs(g.float().numpy()), k))


def test_counted_device_gather(C):
    src = torch.randint(0, 256, (300, 64), dtype=torch.uint8, device="cuda")
    idx = torch.tensor([5, 299, 0, 7, 8], dtype=torch.int32, device="cuda")
    dst = torch.full((5, 64), 0xAB, dtype=torch.uint8, device="cuda")
    C.gather_rows_device_counted(src.data_ptr(), 300, 64, idx, torch.tensor([3], dtype=torch.int32, device="cuda"),
                                 dst)
    assert torch.equal(dst[:3], src[idx[:3].long()])
    assert (dst[3:] == 0xAB).all(), "rows at or past count are not written"


def test_counted_gather_from_pinned_host(C):
    host = torch.randint(0, 256, (256, 1024), dtype=torch.uint8).pin_memory()
    ptr = C.host_device_pointer(host)
    idx = torch.tensor([255, 3, 128, 0], dtype=torch.int32, device="cuda")
    dst = torch.zeros(4, 1024, dtype=torch.uint8, device="cuda")
    C.gather_rows_device_counted(ptr, 256, 1024, idx, torch.tensor([4], dtype=torch.int32, device="cuda"), dst)
    torch.cuda.synchronize()
    assert torch.equal(dst.cpu(), host[idx.cpu().long()])
    with pytest.raises(RuntimeError):
        C.host_device_pointer(torch.zeros(16, dtype=torch.uint8))  # not pinned


@pytest.mark.parametrize("row", [16, 48, 1024, 1040, 2560, 4096])
def test_counted_gather_from_pinned_host_row_sizes(C, row):
    """The host-row gather form (16 lanes per row, 64 bytes per lane per KB): every row size that is a multiple of
    16 bytes, partial last KB included; a row count not a multiple of 4 (the rows per workgroup); out-of-range
    indices give zero rows; rows at or past the device count stay unwritten."""
    n, k = 97, 11
    host = torch.randint(0, 256, (n, row), dtype=torch.uint8, generator=torch.Generator().manual_seed(row))
    host = host.pin_memory()
    ptr = C.host_device_pointer(host)
    idx_l = [96, 0, 5, 5, -1, 97, 50, 1, 2, 3, 4]
    idx = torch.tensor(idx_l, dtype=torch.int32, device="cuda")
    dst = torch.full((k, row), 0xAB, dtype=torch.uint8, device="cuda")
    C.gather_rows_device_counted(ptr, n, row, idx, torch.tensor([9], dtype=torch.int32, device="cuda"), dst)
    torch.cuda.synchronize()
    got = dst.cpu()
    for j, r in enumerate(idx_l[:9]):
        want = host[r] if 0 <= r < n else torch.zeros(row, dtype=torch.uint8)
        assert torch.equal(got[j], want), f"row {j} (index {r})"
    assert (got[9:] == 0xAB).all(), "rows at or past count are not written"


# ---------------------------------------------------------------------------
# fused decode-step GEMVs: each equals the separate ops on the same values
# ---------------------------------------------------------------------------

def int4_mat(N, K, seed, gs=128):
    from helpers import int4_problem

    return int4_problem(N, K, gs, seed=seed)


@pytest.mark.parametrize("N,with_delta", [(4096, True), (6144, False), (1000, True), (37, True), (2050, False),
                                          (1030, True)])
def test_gemv_rmsnorm_equals_norm_then_gemv(C, ops, N, with_delta):
    K = 2048
    p = int4_mat(N, K, 50 + N)
    x, d, w = rnd((K,), 51, 2.0).cuda(), rnd((K,), 52).cuda(), (rnd((K,), 53) * 0.2 + 1).half().cuda()
    x_out, h_out = torch.empty_like(x), torch.empty_like(x)
    y = torch.empty(N, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_rmsnorm_into(p["Wq_d"], p["s_d"], x, d if with_delta else None, w, 1e-6, x_out, h_out, y, K, 128,
                              False)
    s = (x.float() + d.float()).half() if with_delta else x
    assert torch.equal(x_out, s), "x_out = x + delta in binary16"
    # h_out is rmsnorm(s) up to the fp32 sum order of the mean square: within one binary16 rounding
    h_ref = ops.rmsnorm(s.view(1, -1), w, 1e-6).view(-1)
    assert (h_out.float() - h_ref.float()).abs().max() <= 1e-3 * h_ref.float().abs().max()
    # the GEMV consumed exactly h_out
    assert torch.equal(y, ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], h_out, K, 128))


def test_gemv_rmsnorm_swiglu_equals_gemv_then_silu_mul(C, ops):
    K, I = 2048, 1024
    g, u = int4_mat(I, K, 60), int4_mat(I, K, 61)
    t = torch.arange(I // 4, device="cuda")
    perm = torch.stack([4 * t + i for i in range(4)] + [I + 4 * t + i for i in range(4)], 1).reshape(-1)
    W = torch.cat([g["Wq_d"], u["Wq_d"]]).index_select(0, perm).contiguous()
    S = torch.cat([g["s_d"], u["s_d"]]).index_select(0, perm).contiguous()
    x, d, w = rnd((K,), 62).cuda(), rnd((K,), 63).cuda(), (rnd((K,), 64) * 0.2 + 1).half().cuda()
    h_out = torch.empty_like(x)
    y = torch.empty(I, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_rmsnorm_into(W, S, x, d, w, 1e-6, None, h_out, y, K, 128, True)
    gate = ops.gemv_w4a16_group_lop3(g["Wq_d"], g["s_d"], h_out, K, 128)
    up = ops.gemv_w4a16_group_lop3(u["Wq_d"], u["s_d"], h_out, K, 128)
    want = torch.empty_like(y)
    C.silu_mul_into(gate, up, want)
    assert torch.equal(y, want)


def test_gemv_rmsnorm_gate_up_equals_separate_gemvs(C, ops):
    """The interleaved gate|up GEMV writing both halves == rmsnorm then the plain GEMV of the gate rows and of the
    up rows, bit for bit."""
    H, I = 2048, 1024
    x, d = rnd((H,), 61).cuda(), rnd((H,), 62).cuda()
    nw = (rnd((H,), 63) * 0.1 + 1).half().cuda()
    g = int4_problem(I, H, 128, seed=64)
    u = int4_problem(I, H, 128, seed=65)
    t = torch.arange(I // 4)
    perm = torch.stack([4 * t + i for i in range(4)] + [I + 4 * t + i for i in range(4)], 1).reshape(-1).cuda()
    W = torch.cat([g["Wq_d"], u["Wq_d"]]).index_select(0, perm).contiguous()
    S = torch.cat([g["s_d"], u["s_d"]]).index_select(0, perm).contiguous()
    gate = torch.empty(I, dtype=torch.float16, device="cuda")
    up = torch.empty_like(gate)
    xo = torch.empty_like(x)
    C.gemv_w4a16_rmsnorm_gate_up_into(W, S, x, d, nw, 1e-6, xo, gate, up, H, 128)
    hx = torch.empty_like(x)
    gref = torch.empty_like(gate)
    C.gemv_w4a16_rmsnorm_into(g["Wq_d"], g["s_d"], x, d, nw, 1e-6, None, hx, gref, H, 128, False)
    uref = ops.gemv_w4a16_group_lop3(u["Wq_d"], u["s_d"], hx, H, 128)
    assert torch.equal(gate, gref) and torch.equal(up, uref)
    assert torch.equal(xo, (x.float() + d.float()).half())


def test_indexed_accumulate_gated_equals_silu_then_accumulate(C, ops):
    """h_sel computed inside the sparse down == the indexed SiLU GEMV's h_sel, so y is identical; an index outside
    the channel range gives NaN."""
    H, I, k = 2048, 6144, 3072
    down = int4_problem(I, H, 128, seed=71)
    gate = (rnd((I,), 72) * 2).cuda()
    up = (rnd((I,), 73) * 2).cuda()
    idx = torch.sort(torch.randperm(I, generator=torch.Generator().manual_seed(74))[:k]).values.int().cuda()
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_indexed_accumulate_gated_into(down["Wq_d"], down["s_d"], idx, gate, up, y, H, 128, ws)
    h = torch.empty(k, dtype=torch.float16, device="cuda")
    C.silu_mul_indexed_into(gate, idx, up.index_select(0, idx.long()), h)
    y2 = torch.empty_like(y)
    C.gemv_w4a16_indexed_accumulate_into(down["Wq_d"], down["s_d"], idx, h, y2, H, 128, ws)
    assert torch.equal(y, y2)
    bad = idx.clone()
    bad[5] = I + 3
    C.gemv_w4a16_indexed_accumulate_gated_into(down["Wq_d"], down["s_d"], bad, gate, up, y, H, 128, ws)
    assert torch.isnan(y.float()).all()


def _fused_select_down(C, gate, up, k, down, H, ws):
    idx = torch.full((k,), -7, dtype=torch.int32, device="cuda")
    cnt = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    y = torch.full((H,), float("nan"), dtype=torch.float16, device="cuda")
    C.dip_select_gated_down_into(gate, up, k, down["Wq_d"], down["s_d"], idx, cnt, y, H, 128, ws)
    return idx, cnt, y


@pytest.mark.parametrize("I,H,k,ties", [(6144, 2048, 3072, False), (6144, 2048, 768, True), (6144, 2048, 1536, False),
                                        (6144, 2048, 6144, False), (6144, 2048, 1, False), (1000, 256, 333, True),
                                        (8192, 1024, 4096, True), (9728, 2048, 4864, False)])
def test_dip_select_gated_down_equals_topk_then_gated_down(C, I, H, k, ties):
    """One-launch selection + gated sparse down == the top-k launch followed by the gated down, bit for bit
    (indices, count, y); the indices are the oracle's rule-A selection and y matches the oracle's binary64 sum
    over them. Ragged sizes, tie-heavy gates (quarter steps), k = 1 and k = n; 9728 channels exceed the fused
    kernel and run the two-kernel path."""
    down = int4_problem(I, H, 128, seed=81 + k)
    g = rnd((I,), 82 + k) * 2
    if ties:
        g = ((g.float() * 4).round() / 4).half()
    u = rnd((I,), 83 + k) * 2
    gate, up = g.cuda(), u.cuda()
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    idx, cnt, y = _fused_select_down(C, gate, up, k, down, H, ws)
    idx2 = torch.empty(k, dtype=torch.int32, device="cuda")
    cnt2 = torch.empty(1, dtype=torch.int32, device="cuda")
    C.topk_threshold_select_f16abs_into(gate, k, idx2, cnt2)
    y2 = torch.empty(H, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_indexed_accumulate_gated_into(down["Wq_d"], down["s_d"], idx2, gate, up, y2, H, 128, ws)
    assert torch.equal(idx, idx2) and torch.equal(cnt, cnt2) and torch.equal(y, y2)
    ref_idx = O.topk_rule_a(np.abs(g.float().numpy()), k)
    assert int(cnt.item()) == ref_idx.size == k
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    h = OD.silu_mul(g.numpy()[ref_idx], u.numpy()[ref_idx])
    y_ref = O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h, H, 128)
    assert_close(y, y_ref, f"fused select + down I={I} k={k}")
    # the arrival counters are left at zero: a second call on the same workspace is identical
    assert all(torch.equal(a, b) for a, b in zip(_fused_select_down(C, gate, up, k, down, H, ws), (idx, cnt, y)))


def test_dip_select_gated_down_fewer_than_k_selected(C):
    """With NaN gates fewer than k channels can be selected: the count says how many, only those indices are
    written, and y sums over exactly those rows (as the oracle's sum over the rule-A selection)."""
    I, H, k = 1000, 256, 995
    down = int4_problem(I, H, 128, seed=91)
    g = rnd((I,), 92) * 2
    g[torch.arange(3, I, 97)] = float("nan")  # 11 NaN gates: 989 valid channels
    u = rnd((I,), 93) * 2
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    idx, cnt, y = _fused_select_down(C, g.cuda(), u.cuda(), k, down, H, ws)
    ref_idx = O.topk_rule_a(np.abs(g.float().numpy()), k)
    n = ref_idx.size
    assert n == 989 and int(cnt.item()) == n
    assert np.array_equal(idx[:n].cpu().numpy(), ref_idx) and bool((idx[n:] == -7).all())
    h = OD.silu_mul(g.numpy()[ref_idx], u.numpy()[ref_idx])
    assert_close(y, O.sparse_accumulate_f64(down["Wq"][ref_idx], down["s"][ref_idx], h, H, 128), "fused, count < k")


def test_dip_select_gated_down_rejections(C):
    I, H, k = 1024, 256, 100
    down = int4_problem(I, H, 128, seed=94)
    gate, up = (rnd((I,), 95)).cuda(), (rnd((I,), 96)).cuda()
    ws = torch.zeros(C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):  # k = 0
        _fused_select_down(C, gate, up, 0, down, H, ws)
    with pytest.raises(RuntimeError):  # k > n
        _fused_select_down(C, gate, up, I + 1, down, H, ws)
    with pytest.raises(RuntimeError):  # fewer down^T rows than channels
        short = {"Wq_d": down["Wq_d"][: I - 1], "s_d": down["s_d"][: I - 1]}
        _fused_select_down(C, gate, up, k, short, H, ws)
    with pytest.raises(RuntimeError):  # workspace too small
        _fused_select_down(C, gate, up, k, down, H, ws[:16])
    with pytest.raises(RuntimeError):  # up shorter than gate
        _fused_select_down(C, gate, up[:-1], k, down, H, ws)


def test_gemv_rmsnorm_rejects_aliasing(C):
    K = 256
    p = int4_mat(64, K, 70)
    x, w = rnd((K,), 71).cuda(), rnd((K,), 72).cuda()
    y = torch.empty(64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):
        C.gemv_w4a16_rmsnorm_into(p["Wq_d"], p["s_d"], x, None, w, 1e-6, x, None, y, K, 128, False)
    with pytest.raises(RuntimeError):  # SwiGLU needs N % 8 == 0
        q = int4_mat(12, K, 73)
        C.gemv_w4a16_rmsnorm_into(q["Wq_d"], q["s_d"], x, None, w, 1e-6, None, None, y[:6], K, 128, True)


def test_indexed_silu_equals_indexed_then_silu(C, ops):
    K, I = 2048, 6144
    u = int4_mat(I, K, 80)
    x, gate = rnd((K,), 81).cuda(), rnd((I,), 82, 2.0).cuda()
    idx = torch.sort(torch.randperm(I, generator=torch.Generator().manual_seed(83))[:3072]).values.int().cuda()
    h = torch.empty(3072, dtype=torch.float16, device="cuda")
    C.gemv_w4a16_indexed_silu_into(u["Wq_d"], u["s_d"], idx, x, gate, h, K, 128)
    u_sel = ops.gemv_w4a16_indexed(u["Wq_d"], u["s_d"], idx, x, K, 128)
    want = torch.empty_like(h)
    C.silu_mul_indexed_into(gate, idx, u_sel, want)
    assert torch.equal(h, want)


def test_fused_up_silu_equals_fused_up_then_silu(C, ops):
    K, I = 2048, 512
    u = int4_mat(I, K, 90)
    x, gate = rnd((K,), 91).cuda(), rnd((I,), 92, 2.0).cuda()
    sel = torch.arange(0, I, 2, dtype=torch.int32, device="cuda")
    hot = torch.arange(0, I, 3, device="cuda")
    slot_of = torch.full((I,), -1, dtype=torch.int32, device="cuda")
    slot_of[hot] = torch.arange(hot.numel(), dtype=torch.int32, device="cuda")
    desc, miss, mc = ops.build_dip_descriptors(sel, slot_of)
    m = int(mc.item())
    cW, cS = u["Wq_d"][hot].contiguous(), u["s_d"][hot].contiguous()
    sW, sS = u["Wq_d"][miss[:m].long()].contiguous(), u["s_d"][miss[:m].long()].contiguous()
    h = torch.empty(sel.numel(), dtype=torch.float16, device="cuda")
    C.gemv_dip_fused_up_silu_into(cW, cS, sW, sS, desc, sel, x, gate, h, K, 128)
    want = torch.empty_like(h)
    C.silu_mul_indexed_into(gate, sel, ops.gemv_dip_fused_up(cW, cS, sW, sS, desc, x, K, 128), want)
    assert torch.equal(h, want)


@pytest.mark.parametrize("NQ,NKV,hd,S,positions", [(16, 8, 128, 2048, [0, 1, 63, 64, 65, 254, 255, 256, 700]),
                                                   (4, 2, 64, 64, [0, 5, 63]), (8, 8, 128, 256, [0, 200])])
def test_attention_step_equals_separate_ops(C, ops, NQ, NKV, hd, S, positions):
    """One-launch attention == qk_norm_rope_append + decode_attention_at, bit for bit (outputs and both caches),
    over a sequence of positions (the counters left zero by each call make the next one correct)."""
    cos_t, sin_t = ops.rope_tables(hd, 1e6, S, "cuda")
    qn, kn = (rnd((hd,), 22) * 0.1 + 1).half().cuda(), (rnd((hd,), 23) * 0.1 + 1).half().cuda()
    kc_a = rnd((NKV, S, hd), 24).cuda()
    vc_a = rnd((NKV, S, hd), 25).cuda()
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    ws_step = torch.zeros(C.decode_attention_step_workspace_bytes(NQ, NKV, hd, S), dtype=torch.uint8, device="cuda")
    ws_at = torch.zeros(max(1, C.decode_attention_workspace_bytes(NQ, NKV, hd, S)), dtype=torch.uint8, device="cuda")
    q = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
    out_a = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
    out_b = torch.empty_like(out_a)
    for i, p in enumerate(positions):
        qkv = rnd(((NQ + 2 * NKV) * hd,), 100 + i, 2.0).cuda()
        pos = torch.tensor([p], dtype=torch.int32, device="cuda")
        C.decode_attention_step(qkv, qn, kn, cos_t, sin_t, pos, kc_a, vc_a, out_a, 1e-6, ws_step)
        C.qk_norm_rope_append(qkv, qn, kn, cos_t, sin_t, pos, q, kc_b, vc_b, 1e-6)
        C.decode_attention_at(q, kc_b, vc_b, pos, out_b, ws_at)
        assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b), f"caches at position {p}"
        assert torch.equal(out_a, out_b), f"attention output at position {p}"
    tail = ws_step[-256:]
    assert tail.sum() == 0, "the counters are left at zero"


@pytest.mark.parametrize("NQ,NKV,hd,S", [(16, 8, 128, 2048), (4, 2, 64, 64), (8, 1, 128, 1024)])
def test_attention_device_position_equals_host_length(C, ops, NQ, NKV, hd, S):
    """The device-position form plans its splits at run time with the host form's formula: identical outputs."""
    q = rnd((NQ, hd), 40).cuda()
    kc, vc = rnd((NKV, S, hd), 41).cuda(), rnd((NKV, S, hd), 42).cuda()
    ws = torch.zeros(max(1, C.decode_attention_workspace_bytes(NQ, NKV, hd, S)), dtype=torch.uint8, device="cuda")
    out = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
    for L in sorted(L for L in {1, 2, 15, 16, 17, 100, 255, 256, 257, S // 2, S - 1, S} if L <= S):
        C.decode_attention_at(q, kc, vc, torch.tensor([L - 1], dtype=torch.int32, device="cuda"), out, ws)
        assert torch.equal(out, ops.decode_attention(q, kc, vc, L)), f"length {L}"
