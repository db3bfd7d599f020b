"""Seeded random-shape sweeps of the hot-path operators against the oracle, beside the hand-picked grids of the
other test files: shapes, group sizes, selection sizes and context lengths drawn from a fixed generator (the
same cases every run), each within the operator's documented limits.

  * INT4 g GEMV (both dequant forms, bit-identical to each other): N in [1, 3000], K in [1, 5000], group sizes
    8 .. 256, against the binary64 oracle;
  * rule-A top-k over fp32 |gate| (normal, few distinct magnitudes, with NaN and +inf) and over binary16
    gates: indices and count equal to the oracle exactly;
  * the sparse down from an index list: H in [1, 6000], k in [1, 4000] rows of a larger down^T, against the
    binary64 sparse accumulate;
  * the ordered down (selection + the sparse accumulate's order over the transposed copy) where its limits
    allow, bit-identical to the row form;
  * decode attention: query / KV head counts, head sizes (fast and general kernels), cache sizes and lengths
    against the binary64 softmax attention;
  * INT8 GEMV (per-tensor, per-channel, group scales) against the binary64 oracle;
  * the cache-aware chain: a random selection and hot set, build_dip_descriptors equal to the oracle (exact),
    then the descriptor-driven up and down (hot rows from the cache copy, misses from a staging copy)
    bit-identical to the index-driven GEMVs over the resident rows, and within the oracle's tolerance.
"""
import numpy as np
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


def _cases(seed, n, draw):
    rng = np.random.default_rng(seed)
    return [draw(rng) for _ in range(n)]


GEMV = _cases(101, 24, lambda r: (int(r.integers(1, 3001)), int(r.integers(1, 5001)),
                                  int(r.choice([8, 16, 32, 64, 128, 256]))))


@pytest.mark.parametrize("N,K,gs", GEMV)
def test_int4_gemv(ops, N, K, gs):
    p = int4_problem(N, K, gs, seed=N * 7 + K)
    ref = O.gemv_w4_f64(p["Wq"], p["s"], p["x"], p["K"], gs)
    y = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)
    assert_close(y, ref, f"int4 {N}x{K} gs={gs}", floor=5e-5)
    assert torch.equal(y, ops.gemv_w4a16_group(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)), "dequant forms differ"


def _gates(r, n):
    kind = int(r.integers(0, 3))
    g = r.standard_normal(n).astype(np.float32) * np.float32(r.uniform(0.05, 3.0))
    if kind == 1:  # few distinct magnitudes: many ties at the threshold
        g = (r.integers(0, 6, n) * 0.25 * np.sign(r.standard_normal(n))).astype(np.float32)
    elif kind == 2:  # NaN and +inf entries
        m = r.random(n)
        g[m < 0.05] = np.nan
        g[(m >= 0.05) & (m < 0.07)] = np.inf
    return g


TOPK = _cases(202, 24, lambda r: (int(r.integers(1, 20001)), float(r.uniform(0.0, 1.0)), int(r.integers(0, 1 << 30))))


@pytest.mark.parametrize("n,kf,seed", TOPK)
def test_topk_rule_a(C, n, kf, seed):
    r = np.random.default_rng(seed)
    k = max(1, min(n, int(round(kf * n))))
    g = _gates(r, n)
    a = np.abs(g)
    ref = O.topk_rule_a(a, k)
    idx, cnt = C.topk_threshold_select(torch.from_numpy(a).cuda(), k)
    assert int(cnt.item()) == ref.size, f"n={n} k={k}: count"
    assert np.array_equal(idx.cpu().numpy()[:ref.size], ref), f"n={n} k={k}: indices"
    # the decode form over binary16 gates (|gate| read from the half bits): rule A on the same values
    h = torch.from_numpy(g).half()
    ref16 = O.topk_rule_a(np.abs(h.float().numpy()), k)
    i16 = torch.empty(k, dtype=torch.int32, device="cuda")
    c16 = torch.empty(1, dtype=torch.int32, device="cuda")
    C.topk_threshold_select_f16abs_into(h.cuda(), k, i16, c16)
    assert int(c16.item()) == ref16.size and np.array_equal(i16.cpu().numpy()[:ref16.size], ref16), \
        f"n={n} k={k}: binary16 form"


DOWN = _cases(303, 20, lambda r: (int(r.integers(1, 6001)), int(r.integers(1, 4001)),
                                  int(r.choice([8, 16, 32, 64, 128]))))


@pytest.mark.parametrize("H,k,gs", DOWN)
def test_sparse_down_indexed(C, H, k, gs):
    rows = k + int(np.random.default_rng(H + k).integers(0, 2000))
    p = int4_problem(rows, H, gs, seed=H * 3 + k)  # down^T: rows of H
    Hp = p["K"]
    r = np.random.default_rng(k)
    sel = np.sort(r.choice(rows, size=k, replace=False)).astype(np.int32)
    h = torch.from_numpy(r.standard_normal(k).astype(np.float32)).half()
    ref = O.sparse_accumulate_f64(p["Wq"][sel], p["s"][sel], h.numpy(), Hp, gs)
    y = torch.empty(Hp, dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(1, C.sparse_accumulate_workspace_bytes(Hp, k)), dtype=torch.uint8, device="cuda")
    C.gemv_w4a16_indexed_accumulate_into(p["Wq_d"], p["s_d"], torch.from_numpy(sel).cuda(), h.cuda(), y, Hp, gs, ws)
    assert_close(y, ref, f"sparse down H={Hp} k={k} gs={gs}")


ORDERED = _cases(404, 16, lambda r: (int(r.integers(1, 3001)), 32 * int(r.integers(1, 257)),
                                     float(r.uniform(0.0, 1.0)), int(r.choice([8, 16, 32, 64, 128]))))


@pytest.mark.parametrize("H,n,kf,gs", ORDERED)
def test_ordered_down_equals_row_form(C, ops, H, n, kf, gs):
    k = max(1, min(n, int(round(kf * n))))
    p = int4_problem(n, H, gs, seed=H + n)
    Hp = p["K"]
    if C.dip_select_down_ordered_lds_bytes(Hp, n, k) == 0:
        pytest.skip("outside the ordered kernel's limits (the engine uses the row form there)")
    Wt, St = ops.transposed_down_T(p["Wq_d"], p["s_d"], Hp)
    r = np.random.default_rng(n + k)
    gate = torch.from_numpy(r.standard_normal(n).astype(np.float32)).half().cuda()
    up = torch.from_numpy(r.standard_normal(n).astype(np.float32)).half().cuda()
    idx = torch.empty(k, dtype=torch.int32, device="cuda")
    cnt = torch.empty(1, dtype=torch.int32, device="cuda")
    y_row = torch.empty(Hp, dtype=torch.float16, device="cuda")
    ws = torch.zeros(max(1, C.sparse_accumulate_workspace_bytes(Hp, k)), dtype=torch.uint8, device="cuda")
    C.dip_select_gated_down_into(gate, up, k, p["Wq_d"], p["s_d"], idx, cnt, y_row, Hp, gs, ws)
    h = torch.empty_like(gate)
    C.silu_mul_into(gate, up, h)
    y = torch.empty(Hp, dtype=torch.float16, device="cuda")
    C.dip_select_down_ordered_into(gate, h, k, Wt, St, None, None, y, gs)
    assert torch.equal(y, y_row), f"H={Hp} n={n} k={k} gs={gs}"


def _attn_case(r):
    nkv = int(r.choice([1, 2, 4, 8]))
    rep = int(r.choice([1, 2, 3, 4, 8]))
    hd = int(r.choice([8, 16, 32, 64, 128, 256, 24, 40, 100]))
    S = int(r.integers(1, 3001))
    return nkv * rep, nkv, hd, S, int(r.integers(1, S + 1))


ATTN = _cases(505, 20, _attn_case)


@pytest.mark.parametrize("NQ,NKV,hd,S,L", ATTN)
def test_decode_attention(ops, NQ, NKV, hd, S, L):
    g = torch.Generator().manual_seed(NQ * 31 + hd + S + L)
    q = torch.randn(NQ, hd, generator=g).half()
    k = torch.randn(NKV, S, hd, generator=g).half()
    v = torch.randn(NKV, S, hd, generator=g).half()
    ref = O.decode_attention_f64(q.numpy(), k.numpy(), v.numpy(), L)
    out = ops.decode_attention(q.cuda(), k.cuda(), v.cuda(), L)
    assert_close(out, ref, f"attention {NQ}/{NKV} hd={hd} S={S} L={L}")


INT8 = _cases(606, 16, lambda r: (int(r.integers(1, 3001)), int(r.integers(1, 4097)),
                                  str(r.choice(["per_tensor", "per_channel", "group"])),
                                  int(r.choice([8, 16, 32, 64, 128]))))


@pytest.mark.parametrize("N,K,gran,gs", INT8)
def test_int8_gemv(ops, N, K, gran, gs):
    g = torch.Generator().manual_seed(N + K)
    if gran == "group":
        K = max(gs, K // gs * gs)  # group scales: K a multiple of the group size
    w = (torch.randn(N, K, generator=g)).numpy()
    q, sc = O.quantize_group(w, gs, bits=8) if gran == "group" else O.quantize_simple(w, gran, bits=8)
    q = q[:, :K].copy()
    x = torch.randn(K, generator=g).half()
    gsz = gs if gran == "group" else K
    ref = O.gemv_w8_f64(q, sc, x.numpy(), gsz)
    y = ops.gemv_w8a16(torch.from_numpy(q).cuda(), torch.from_numpy(np.ascontiguousarray(sc)).cuda(), x.cuda(), gsz)
    assert_close(y, ref, f"int8 {gran} {N}x{K} gs={gsz}")


CACHED = _cases(707, 12, lambda r: (int(r.integers(32, 8193)), int(r.integers(8, 3001)), float(r.uniform(0.0, 1.0)),
                                    float(r.uniform(0.0, 1.0)), int(r.choice([32, 64, 128]))))


@pytest.mark.parametrize("I,H,kf,hot,gs", CACHED)
def test_cache_aware_chain(ops, I, H, kf, hot, gs):
    k = max(1, min(I, int(round(kf * I))))
    r = np.random.default_rng(I + H)
    up = int4_problem(I, H, gs, seed=I * 5 + H)        # up_proj: I rows of H
    dn = int4_problem(I, H, gs, seed=I * 5 + H + 1)    # down_proj^T: I rows of H
    Hp = up["K"]
    sel = np.sort(r.choice(I, size=k, replace=False)).astype(np.int32)
    hot_ch = np.sort(r.choice(I, size=int(round(hot * I)), replace=False)).astype(np.int32)
    slot_of = np.full(I, -1, np.int32)
    slot_of[hot_ch] = np.arange(hot_ch.size, dtype=np.int32)
    d_ref, m_ref, mc_ref = O.build_dip_descriptors(sel, slot_of)
    sel_d = torch.from_numpy(sel).cuda()
    desc, miss, mc = ops.build_dip_descriptors(sel_d, torch.from_numpy(slot_of).cuda())
    assert int(mc.item()) == mc_ref and np.array_equal(desc.cpu().numpy(), d_ref), f"I={I} k={k}: descriptors"
    assert np.array_equal(miss.cpu().numpy()[:mc_ref], m_ref[:mc_ref]), f"I={I} k={k}: miss list"
    hot_t = torch.from_numpy(hot_ch).long().cuda()
    miss_t = torch.from_numpy(m_ref[:mc_ref]).long().cuda()
    for name, p in (("up", up), ("down", dn)):
        W, S = p["Wq_d"], p["s_d"]
        cW, cS = W.index_select(0, hot_t).contiguous(), S.index_select(0, hot_t).contiguous()
        sW, sS = W.index_select(0, miss_t).contiguous(), S.index_select(0, miss_t).contiguous()
        if name == "up":
            y = ops.gemv_dip_fused_up(cW, cS, sW, sS, desc, up["x_d"], Hp, gs)
            assert torch.equal(y, ops.gemv_w4a16_indexed(W, S, sel_d, up["x_d"], Hp, gs)), f"I={I} k={k}: up"
            assert_close(y, O.gemv_w4_f64(up["Wq"][sel], up["s"][sel], up["x"], Hp, gs), f"I={I} k={k}: up", floor=5e-5)
        else:
            h = torch.from_numpy(r.standard_normal(k).astype(np.float32)).half()
            y = ops.gemv_dip_fused_down(cW, cS, sW, sS, desc, h.cuda(), Hp, gs)
            assert torch.equal(y, ops.gemv_w4a16_indexed_accumulate(W, S, sel_d, h.cuda(), Hp, gs)), \
                f"I={I} k={k}: down"
            assert_close(y, O.sparse_accumulate_f64(dn["Wq"][sel], dn["s"][sel], h.numpy(), Hp, gs),
                         f"I={I} k={k}: down")
