"""Size-independent properties at the full Qwen3-1.7B shapes (3 and 5), checked exactly.

Doubling an input of these kernels doubles every binary16 input, fp32 product, fp32 partial sum and the final
binary16 rounding (no overflow at these magnitudes), so the outputs double exactly, except that a binary16
subnormal output (|y| < 2^-14, rounded on a fixed 2^-24 grid) may move by that one step. Negating an input negates every term; IEEE round-to-nearest is sign-symmetric, so kernels
that accumulate with fmaf (sparse down, attention's P.V) negate exactly, while the GEMVs' v_dot2_f32_f16 chains do
not round to nearest and negate up to one binary16 rounding step. GEMV rows are
independent, so permuting the rows of W permutes y; attention heads read only their own KV head. These hold for
any size, so they check the kernels at the real shapes without an oracle run.
"""
import pytest
import torch

from helpers import int4_problem

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


def _eq(a: torch.Tensor, b: torch.Tensor, label: str):
    assert torch.equal(a, b), f"{label}: {int((a != b).sum())} elements differ"


def _doubled(y2: torch.Tensor, y: torch.Tensor, label: str):
    """y2 == 2 y exactly wherever y is a normal binary16 number; in the subnormal range (|y| < 2^-14) rounding is on
    a fixed grid of 2^-24, so fp16(2a) and 2 fp16(a) may differ by that one step."""
    want = (y.float() * 2).half()
    normal = y.float().abs() >= 2.0 ** -14
    _eq(y2[normal], want[normal], label)
    assert bool(((y2.float() - want.float()).abs() <= 2.0 ** -24).all()), f"{label}: subnormal outputs differ"


def _nearly(a: torch.Tensor, b: torch.Tensor, label: str):
    """Per element at most one binary16 rounding step of b apart (2^-10 |b|), plus 1e-5 of max |b| for the few
    outputs that cancel to near zero."""
    af, bf = a.float(), b.float()
    bound = (2.0 ** -10) * bf.abs() + 1e-5 * float(bf.abs().max())
    bad = int(((af - bf).abs() > bound).sum())
    assert bad == 0, f"{label}: {bad} elements more than one binary16 step apart"


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144), (2048, 2048), (1024, 2048)])
def test_int4_gemv_scaling_sign_and_row_permutation(ops, N, K):
    p = int4_problem(N, K, 128, seed=N * 3 + K)
    W, s, x = p["Wq_d"], p["s_d"], p["x_d"]
    y = ops.gemv_w4a16_group_lop3(W, s, x, K, 128)
    _doubled(ops.gemv_w4a16_group_lop3(W, s, x * 2, K, 128), y, "x -> 2x")
    _doubled(ops.gemv_w4a16_group_lop3(W, s * 2, x, K, 128), y, "scales -> 2 scales")
    # v_dot2_f32_f16 does not round to nearest (it is not sign-symmetric: probe over 2^20 random inputs, 14% of
    # results differ under negation, by one fp32 ulp), so negation holds up to that rounding only
    _nearly(ops.gemv_w4a16_group_lop3(W, s, -x, K, 128), -y, "x -> -x")
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(N)).cuda()
    _eq(ops.gemv_w4a16_group_lop3(W[perm].contiguous(), s[perm].contiguous(), x, K, 128), y[perm], "row permutation")
    _eq(ops.gemv_w4a16_group(W, s, x, K, 128), y, "scalar vs bitfield dequant")


@pytest.mark.parametrize("N,K", [(6144, 2048), (2048, 6144)])
def test_int8_gemv_scaling_sign_and_row_permutation(ops, N, K):
    g = torch.Generator().manual_seed(N + 5 * K)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).cuda()
    s = (torch.rand(N, K // 128, generator=g) * 1e-3).cuda()
    x = torch.randn(K, generator=g).half().cuda()
    y = ops.gemv_w8a16(q, s, x, 128)
    _doubled(ops.gemv_w8a16(q, s, x * 2, 128), y, "x -> 2x")
    _nearly(ops.gemv_w8a16(q, s, -x, 128), -y, "x -> -x")
    perm = torch.randperm(N, generator=g).cuda()
    _eq(ops.gemv_w8a16(q[perm].contiguous(), s[perm].contiguous(), x, 128), y[perm], "row permutation")


@pytest.mark.parametrize("k", [768, 3072, 6144])
def test_sparse_down_scaling_and_sign(ops, k):
    H, I = 2048, 6144
    p = int4_problem(I, H, 128, seed=k)
    idx = torch.sort(torch.randperm(I, generator=torch.Generator().manual_seed(k))[:k]).values.int().cuda()
    h = torch.randn(k, generator=torch.Generator().manual_seed(k + 1)).half().cuda()
    y = ops.gemv_w4a16_indexed_accumulate(p["Wq_d"], p["s_d"], idx, h, H, 128)
    _doubled(ops.gemv_w4a16_indexed_accumulate(p["Wq_d"], p["s_d"], idx, h * 2, H, 128), y, "h -> 2h")
    _eq(ops.gemv_w4a16_indexed_accumulate(p["Wq_d"], p["s_d"], idx, -h, H, 128), -y, "h -> -h")
    # the gathered form over the same logical rows is the same computation
    il = idx.long()
    _eq(ops.gemv_w4a16_sparse_accumulate(p["Wq_d"][il].contiguous(), p["s_d"][il].contiguous(), h, H, 128), y,
        "index-driven vs gathered")


@pytest.mark.parametrize("L", [1, 192, 2048])
def test_attention_value_scaling_and_head_independence(ops, L):
    NQ, NKV, hd, S = 16, 8, 128, 2048
    g = torch.Generator().manual_seed(L)
    q = torch.randn(NQ, hd, generator=g).half().cuda()
    kc = torch.randn(NKV, S, hd, generator=g).half().cuda()
    vc = torch.randn(NKV, S, hd, generator=g).half().cuda()
    out = ops.decode_attention(q, kc, vc, L)
    _doubled(ops.decode_attention(q, kc, vc * 2, L), out, "V -> 2V")
    _eq(ops.decode_attention(q, kc, -vc, L), -out, "V -> -V")
    # rewriting KV head 3 (query heads 6, 7) and everything past L leaves every other head bit-identical
    kc2, vc2 = kc.clone(), vc.clone()
    kc2[3].normal_(generator=torch.Generator(device="cuda").manual_seed(1))
    vc2[:, L:] = 7.0
    out2 = ops.decode_attention(q, kc2, vc2, L)
    keep = [h for h in range(NQ) if h // (NQ // NKV) != 3]
    _eq(out2[keep], out[keep], "heads of untouched KV heads")
