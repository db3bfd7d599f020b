"""Sparse / cache-aware DIP parity on the GPU.

Counterpart of the reference's tests/test_m7_sparse_gemv.py, tests/test_gather_rows.py,
tests/test_m8_fused_gemv.py and tests/test_m8_cached_dip_pipeline.py:
  * gather_rows_{staged,naive,device}: byte-exact against the oracle gather;
  * gemv_w4a16_sparse_accumulate: one-hot rows exact, random within 1e-3 of the binary64 oracle;
  * build_dip_descriptors: the reference's hand cases and random selections, exact;
  * fused up/down with mixed cache/staging sources within 1e-3 of the oracle, and bit-identical
    to the plain kernels on the same logical rows;
  * index-driven (resident) sparse GEMVs bit-identical to gather-then-GEMV;
  * the DIP MLP of one Qwen3-1.7B layer: resident == gathered == cache-aware, torch.equal.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


def _desc_int32(is_staging: bool, off: int) -> int:
    return int(np.array([off | (0x80000000 if is_staging else 0)], np.uint32).view(np.int32)[0])


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("num_rows,row_nbytes,k", [(6144, 1024, 3072), (17408, 2560, 8704), (1024, 64, 1),
                                                   (1024, 64, 1024), (256, 8, 37)])
def test_gather_rows_host_variants(ops, num_rows, row_nbytes, k):
    g = torch.Generator().manual_seed(0)
    matrix = torch.randint(0, 256, (num_rows, row_nbytes), dtype=torch.uint8, generator=g).pin_memory()
    idx = torch.randperm(num_rows, generator=g)[:k].contiguous()
    expect = O.gather_rows(matrix.numpy(), idx.numpy())
    staging = torch.empty(k, row_nbytes, dtype=torch.uint8).pin_memory()
    d1 = torch.empty(k, row_nbytes, dtype=torch.uint8, device="cuda")
    d2 = torch.empty(k, row_nbytes, dtype=torch.uint8, device="cuda")
    ops.gather_rows_staged(matrix, idx, staging, d1)
    ops.gather_rows_naive(matrix, idx, d2)
    torch.cuda.synchronize()
    assert np.array_equal(d1.cpu().numpy(), expect)
    assert np.array_equal(d2.cpu().numpy(), expect)
    d3 = torch.empty(k, row_nbytes, dtype=torch.uint8, device="cuda")
    ops.gather_rows_device(matrix.cuda(), idx.int().cuda(), d3)
    assert np.array_equal(d3.cpu().numpy(), expect)


def test_gather_rows_rejections(ops):
    m = torch.randint(0, 256, (256, 8), dtype=torch.uint8)
    dst = torch.empty(10, 8, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        ops.gather_rows_naive(m, torch.arange(10), dst)  # not pinned
    mp = m.pin_memory()
    with pytest.raises(RuntimeError):
        ops.gather_rows_staged(mp, torch.arange(10), torch.empty(5, 8, dtype=torch.uint8).pin_memory(), dst)
    with pytest.raises(RuntimeError):
        ops.gather_rows_naive(mp, torch.tensor([0, 256]), dst)  # index out of range


# ---------------------------------------------------------------------------
# sparse accumulate
# ---------------------------------------------------------------------------

def test_sparse_accumulate_one_hot_exact(ops):
    p = int4_problem(20, 256, 64, seed=0, std=3.0)
    Wd = O.dequant_int4(p["Wq"], p["s"], 256, 64).astype(np.float16)
    for i0 in range(0, 20, 3):
        h = torch.zeros(20, dtype=torch.float16, device="cuda")
        h[i0] = 1.0
        y = ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, 256, 64)
        assert np.array_equal(y.cpu().numpy(), Wd[i0]), f"one-hot row {i0}"


@pytest.mark.parametrize("k,H,gs", [(64, 512, 128), (37, 256, 64), (3072, 2048, 128), (1536, 2048, 128),
                                    (768, 2048, 128), (200, 5120, 128), (50, 100, 8), (0, 256, 64),
                                    (8704, 5120, 128)])  # Qwen3-14B shape at k/I = 0.5: 20 slices x 46 row chunks
def test_sparse_accumulate_matches_oracle(ops, k, H, gs):
    p = int4_problem(max(k, 1), H, gs, seed=k + H)
    Wq, s = p["Wq"][:k], p["s"][:k]
    h = torch.randn(k, generator=torch.Generator().manual_seed(k)).half()
    ref = O.sparse_accumulate_f64(Wq, s, h.numpy(), p["K"], gs)
    y = ops.gemv_w4a16_sparse_accumulate(torch.from_numpy(Wq).cuda(), torch.from_numpy(s).cuda(), h.cuda(), p["K"], gs)
    if k == 0:
        assert torch.equal(y.cpu(), torch.zeros(p["K"], dtype=torch.float16))
    else:
        assert_close(y, ref, f"sparse_accumulate k={k} H={H}")


def test_sparse_accumulate_rejections(ops):
    p = int4_problem(16, 128, 32, seed=1)
    h = torch.randn(16, device="cuda").half()
    with pytest.raises(RuntimeError):
        ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, 136, 32)
    with pytest.raises(RuntimeError):
        ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h[:-1].contiguous(), 128, 32)
    with pytest.raises(RuntimeError):
        ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"][:-1].contiguous(), h, 128, 32)
    with pytest.raises(RuntimeError):
        ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, 128, 5)


# ---------------------------------------------------------------------------
# descriptors
# ---------------------------------------------------------------------------

def test_build_dip_descriptors_golden(ops):
    for c in json.loads((GOLDEN / "dip_descriptor_cases.json").read_text()):
        slot_of = torch.full((c["num_channels"],), -1, dtype=torch.int32)
        for slot, ch in enumerate(c["cached"]):
            slot_of[ch] = slot
        desc, miss, mc = ops.build_dip_descriptors(torch.tensor(c["selected"], dtype=torch.int32).cuda(),
                                                   slot_of.cuda())
        mc = int(mc.item())
        assert mc == c["expect_miss_count"], c["name"]
        assert miss[:mc].tolist() == c["expect_miss_channels"], c["name"]
        got = [[bool(d & 0x80000000), int(d & 0x7FFFFFFF)] for d in desc.cpu().numpy().view(np.uint32).tolist()]
        assert got == c["expect_desc"], c["name"]


@pytest.mark.parametrize("I,k,C", [(6144, 3072, 1229), (6144, 768, 0), (6144, 1536, 6144), (17408, 8704, 3000),
                                   (100, 100, 50)])
def test_build_dip_descriptors_random(ops, I, k, C):
    g = torch.Generator().manual_seed(I + k + C)
    sel = torch.sort(torch.randperm(I, generator=g)[:k]).values.int()
    hot = torch.sort(torch.randperm(I, generator=g)[:C]).values
    slot_of = torch.full((I,), -1, dtype=torch.int32)
    slot_of[hot] = torch.arange(C, dtype=torch.int32)
    d_ref, m_ref, mc_ref = O.build_dip_descriptors(sel.numpy(), slot_of.numpy())
    desc, miss, mc = ops.build_dip_descriptors(sel.cuda(), slot_of.cuda())
    assert int(mc.item()) == mc_ref
    assert np.array_equal(desc.cpu().numpy(), d_ref)
    assert np.array_equal(miss.cpu().numpy()[:mc_ref], m_ref[:mc_ref])


# ---------------------------------------------------------------------------
# fused GEMVs
# ---------------------------------------------------------------------------

def _split(k, seed):
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(k, generator=g).tolist()
    return sorted(perm[: k // 2]), perm[k // 2:]


def _descs(k, cache_rows, stage_rows):
    d = np.empty(k, np.int32)
    for slot, j in enumerate(cache_rows):
        d[j] = _desc_int32(False, slot)
    for pos, j in enumerate(stage_rows):
        d[j] = _desc_int32(True, pos)
    return torch.from_numpy(d).cuda()


@pytest.mark.parametrize("k,H,gs", [(24, 256, 64), (3072, 2048, 128), (40, 136, 8)])
def test_fused_up_and_down_mixed_sources(ops, k, H, gs):
    p = int4_problem(k, H, gs, seed=k * 3)
    cr, sr = _split(k, seed=k)
    desc = _descs(k, cr, sr)
    Wd, sd = p["Wq_d"], p["s_d"]
    cW, cS, sW, sS = Wd[cr].contiguous(), sd[cr].contiguous(), Wd[sr].contiguous(), sd[sr].contiguous()
    up = ops.gemv_dip_fused_up(cW, cS, sW, sS, desc, p["x_d"], p["K"], gs)
    assert_close(up, O.gemv_w4_f64(p["Wq"], p["s"], p["x"], p["K"], gs), "fused up")
    assert torch.equal(up, ops.gemv_w4a16_group_lop3(Wd, sd, p["x_d"], p["K"], gs))
    h = torch.randn(k, generator=torch.Generator().manual_seed(9)).half()
    down = ops.gemv_dip_fused_down(cW, cS, sW, sS, desc, h.cuda(), p["K"], gs)
    assert_close(down, O.sparse_accumulate_f64(p["Wq"], p["s"], h.numpy(), p["K"], gs), "fused down")
    assert torch.equal(down, ops.gemv_w4a16_sparse_accumulate(Wd, sd, h.cuda(), p["K"], gs))


def test_fused_degenerate_sources_equal_plain(ops):
    p = int4_problem(16, 128, 32, seed=2)
    empty_W = torch.empty(0, p["Wq_d"].shape[1], dtype=torch.uint8, device="cuda")
    empty_s = torch.empty(0, p["s_d"].shape[1], dtype=torch.float32, device="cuda")
    all_cache = torch.arange(16, dtype=torch.int32, device="cuda")
    up = ops.gemv_dip_fused_up(p["Wq_d"], p["s_d"], empty_W, empty_s, all_cache, p["x_d"], 128, 32)
    assert torch.equal(up, ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], 128, 32))
    all_stage = torch.arange(16, dtype=torch.int32, device="cuda") | (1 << 31)
    h = torch.randn(16, device="cuda").half()
    down = ops.gemv_dip_fused_down(empty_W, empty_s, p["Wq_d"], p["s_d"], all_stage, h, 128, 32)
    assert torch.equal(down, ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, 128, 32))


def test_fused_bad_descriptor_gives_nan_not_a_fault(ops):
    p = int4_problem(8, 64, 32, seed=3)
    empty_W = torch.empty(0, p["Wq_d"].shape[1], dtype=torch.uint8, device="cuda")
    empty_s = torch.empty(0, p["s_d"].shape[1], dtype=torch.float32, device="cuda")
    desc = torch.tensor([0, 1, 99, 2], dtype=torch.int32, device="cuda")  # 99: beyond the 8 cache rows
    up = ops.gemv_dip_fused_up(p["Wq_d"], p["s_d"], empty_W, empty_s, desc, p["x_d"], 64, 32)
    assert torch.isnan(up[2]) and torch.isfinite(up[[0, 1, 3]]).all()


def test_fused_rejections(ops):
    p = int4_problem(8, 64, 32, seed=7)
    desc = torch.arange(8, dtype=torch.int32, device="cuda")
    bad_s = torch.empty(0, p["s_d"].shape[1] + 1, dtype=torch.float32, device="cuda")
    empty_W = torch.empty(0, p["Wq_d"].shape[1], dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        ops.gemv_dip_fused_up(p["Wq_d"], p["s_d"], empty_W, bad_s, desc, p["x_d"], 64, 32)
    q65 = int4_problem(8, 65, 32, seed=8)
    bs = q65["s_d"][:, :2].contiguous()
    with pytest.raises(RuntimeError):
        ops.gemv_dip_fused_up(q65["Wq_d"], bs, empty_W, torch.empty(0, 2, device="cuda"), desc, q65["x_d"],
                              q65["K"], 32)


# ---------------------------------------------------------------------------
# resident (index-driven) sparse GEMVs and the DIP MLP
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("k", [768, 1536, 3072])
def test_indexed_equals_gathered(ops, k):
    p = int4_problem(6144, 2048, 128, seed=k)
    idx = torch.sort(torch.randperm(6144, generator=torch.Generator().manual_seed(k))[:k]).values
    idx_d = idx.int().cuda()
    sel_W = p["Wq_d"].index_select(0, idx.cuda())
    sel_s = p["s_d"].index_select(0, idx.cuda())
    u1 = ops.gemv_w4a16_indexed(p["Wq_d"], p["s_d"], idx_d, p["x_d"], 2048, 128)
    u2 = ops.gemv_w4a16_group_lop3(sel_W, sel_s, p["x_d"], 2048, 128)
    assert torch.equal(u1, u2)
    assert_close(u1, O.gemv_w4_f64(p["Wq"][idx.numpy()], p["s"][idx.numpy()], p["x"], 2048, 128), "indexed up")
    h = torch.randn(k, generator=torch.Generator().manual_seed(1)).half().cuda()
    y1 = ops.gemv_w4a16_indexed_accumulate(p["Wq_d"], p["s_d"], idx_d, h, 2048, 128)
    y2 = ops.gemv_w4a16_sparse_accumulate(sel_W, sel_s, h, 2048, 128)
    assert torch.equal(y1, y2)


def test_sparse_down_workspace_reused_across_calls(ops):
    """One zero-filled workspace serves calls of different k at the same H: the arrival counters at its start are
    left at zero by every call, and each result equals a call with a fresh workspace (and the oracle)."""
    from soinfer import _C

    H, gs, I = 2048, 128, 6144
    p = int4_problem(I, H, gs, seed=11)
    ws = torch.zeros(_C.sparse_accumulate_workspace_bytes(H, 3072), dtype=torch.uint8, device="cuda")
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    g = torch.Generator().manual_seed(3)
    for k in (3072, 768, 3072, 100, 1, 1536):
        idx = torch.sort(torch.randperm(I, generator=g)[:k]).values
        h = torch.randn(k, generator=g).half().cuda()
        _C.gemv_w4a16_indexed_accumulate_into(p["Wq_d"], p["s_d"], idx.int().cuda(), h, y, H, gs, ws)
        fresh = ops.gemv_w4a16_indexed_accumulate(p["Wq_d"], p["s_d"], idx.int().cuda(), h, H, gs)
        assert torch.equal(y, fresh), f"k={k}"
        assert_close(y, O.sparse_accumulate_f64(p["Wq"][idx.numpy()], p["s"][idx.numpy()], h.cpu().numpy(), H, gs),
                     f"sparse down k={k}")
        assert int(ws[:256].count_nonzero()) == 0, "arrival counters left non-zero"


def _layer(H=2048, I=6144, gs=128, seed=0):
    from soinfer.runtime.dip import DipMLPWeights

    mats = {}
    for i, name in enumerate(("gate", "up", "down_T")):
        p = int4_problem(I, H, gs, seed=seed * 10 + i)
        mats[name] = (p["Wq_d"], p["s_d"])
    return DipMLPWeights(mats["gate"][0], mats["gate"][1], mats["up"][0], mats["up"][1], mats["down_T"][0],
                         mats["down_T"][1], hidden_size=H, group_size=gs)


@pytest.mark.parametrize("frac", [0.125, 0.25, 0.5])
def test_dip_mlp_paths_bit_identical_and_match_oracle(ops, frac):
    from soinfer.offload.hot_cache import HotCache, StaticFrequencyPolicy
    from soinfer.runtime import dip

    w = _layer()
    k = int(6144 * frac)
    x = torch.randn(2048, generator=torch.Generator().manual_seed(7)).half().cuda()
    y_res, idx = dip.dip_mlp(w, x, k)
    y_gat, idx2 = dip.dip_mlp_gathered(w, x, k)
    assert torch.equal(idx, idx2) and torch.equal(y_res, y_gat)
    # selection = rule A on the kernel's own gate output
    gate = ops.gemv_w4a16_group_lop3(w.gate_Wq, w.gate_scale, x, 2048, 128)
    assert np.array_equal(idx.cpu().numpy(), O.topk_rule_a(gate.float().abs().cpu().numpy(), k))
    # down output against the binary64 oracle on the kernel's own h
    u = ops.gemv_w4a16_indexed(w.up_Wq, w.up_scale, idx, x, 2048, 128)
    h = dip.silu_gate(gate, idx, u)
    sel = idx.long().cpu().numpy()
    ref = O.sparse_accumulate_f64(w.down_T_Wq.cpu().numpy()[sel], w.down_T_scale.cpu().numpy()[sel],
                                  h.cpu().numpy(), 2048, 128)
    assert_close(y_res, ref, f"DIP down k/I={frac}")
    # cache-aware DIP with hot caches of 0%, 20% (calibrated) and 100%
    xs = torch.randn(8, 2048, generator=torch.Generator().manual_seed(11)).half().cuda()
    counts = dip.calibrate_channel_frequencies(w, xs, k)
    for C in (0, 1229, 6144):
        hot = StaticFrequencyPolicy(counts.cpu(), C).hot_indices
        cache = HotCache.build(w.up_Wq, w.up_scale, w.down_T_Wq, w.down_T_scale, hot)
        y_c, idx_c, mc = dip.cached_dip_mlp(w, cache, x, k)
        assert torch.equal(idx_c, idx)
        assert torch.equal(y_c, y_res), f"cache-aware DIP differs (C={C}, misses={mc})"


def test_cached_dip_from_pinned_host_matches(ops):
    from soinfer.offload.hot_cache import HotCache
    from soinfer.runtime import dip

    w = _layer(seed=3)
    k = 3072
    x = torch.randn(2048, generator=torch.Generator().manual_seed(5)).half().cuda()
    y_ref, _ = dip.dip_mlp(w, x, k)
    up_host = w.up_Wq.cpu().pin_memory()
    down_host = w.down_T_Wq.cpu().pin_memory()
    hot = list(range(0, 6144, 5))
    cache = HotCache.from_host(up_host, w.up_scale, down_host, w.down_T_scale, hot)
    staging = torch.empty(k * 1024, dtype=torch.uint8).pin_memory()
    y, _, mc = dip.cached_dip_mlp(w, cache, x, k, host_up=up_host, host_down_T=down_host, staging=staging)
    assert mc > 0
    assert torch.equal(y, y_ref)


# ---------------------------------------------------------------------------
# hot-cache GEMVs reading the misses in place (no descriptors / staging)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("C", [0, 1229, 6144])
@pytest.mark.parametrize("source", ["cuda", "pinned", "pinned_arena_view"])
def test_cached_direct_equals_staged_and_resident(ops, C, source):
    """soi_gemv_dip_cached_up / _up_silu / _down: bit-identical to the descriptor + staging kernels and to the
    index-driven resident kernels on the same selection, with the full matrices on the device, in pinned host
    memory, or as views at an offset inside one pinned arena."""
    from soinfer import _C
    from soinfer.offload.hot_cache import HotCache
    from soinfer.runtime import dip

    w = _layer(seed=5)
    k, H, gs = 3072, 2048, 128
    x = torch.randn(H, generator=torch.Generator().manual_seed(9)).half().cuda()
    gate, idx = dip.select_channels(w, x, k)
    hot = sorted(np.random.default_rng(C).choice(6144, C, replace=False).tolist())
    cache = HotCache.build(w.up_Wq, w.up_scale, w.down_T_Wq, w.down_T_scale, hot)
    if source == "cuda":
        full_up, full_dn = w.up_Wq, w.down_T_Wq
    elif source == "pinned":
        full_up, full_dn = w.up_Wq.cpu().pin_memory(), w.down_T_Wq.cpu().pin_memory()
    else:
        rows, rb = w.up_Wq.shape
        arena = torch.empty(4096 + 2 * rows * rb, dtype=torch.uint8).pin_memory()
        full_up = arena[4096:4096 + rows * rb].view(rows, rb)
        full_dn = arena[4096 + rows * rb:].view(rows, rb)
        full_up.copy_(w.up_Wq.cpu())
        full_dn.copy_(w.down_T_Wq.cpu())
    # staged reference: descriptors, device gathers of the misses, descriptor kernels
    desc, miss, mcnt = ops.build_dip_descriptors(idx, cache.slot_of)
    mc = int(mcnt.item())
    ml = miss[:mc].long()
    up_st = w.up_Wq.index_select(0, ml).contiguous()
    dn_st = w.down_T_Wq.index_select(0, ml).contiguous()
    u_ref = ops.gemv_dip_fused_up(cache.up_Wq, cache.up_scale, up_st, w.up_scale.index_select(0, ml), desc, x, H, gs)
    u = torch.empty(k, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, full_up, w.up_scale, cache.slot_of, idx, x, u, H, gs)
    assert torch.equal(u, u_ref), "cached up differs from the descriptor form"
    assert torch.equal(u, ops.gemv_w4a16_indexed(w.up_Wq, w.up_scale, idx, x, H, gs)), "cached up != resident"
    h_ref = torch.empty(k, dtype=torch.float16, device="cuda")
    _C.gemv_dip_fused_up_silu_into(cache.up_Wq, cache.up_scale, up_st, w.up_scale.index_select(0, ml), desc, idx,
                                   x, gate, h_ref, H, gs)
    h = torch.empty(k, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_up_silu_into(cache.up_Wq, cache.up_scale, full_up, w.up_scale, cache.slot_of, idx, x, gate,
                                    h, H, gs)
    assert torch.equal(h, h_ref), "cached up + SiLU differs from the descriptor form"
    y_ref = ops.gemv_dip_fused_down(cache.down_Wq, cache.down_scale, dn_st, w.down_T_scale.index_select(0, ml), desc,
                                    h, H, gs)
    ws = torch.zeros(_C.sparse_accumulate_workspace_bytes(H, k), dtype=torch.uint8, device="cuda")
    y = torch.empty(H, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, full_dn, w.down_T_scale, cache.slot_of, idx, h, y,
                                 H, gs, ws)
    assert torch.equal(y, y_ref), "cached down differs from the descriptor form"
    # the up GEMV copying the down^T miss rows to staging: same h; staging row j = down^T row sel[j] for every miss
    # (hit rows untouched); the down accumulate reading misses from that staging gives the same y
    stage = torch.full((k, w.down_T_Wq.shape[1]), 0xAB, dtype=torch.uint8, device="cuda")
    h2 = torch.empty(k, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_up_silu_into(cache.up_Wq, cache.up_scale, full_up, w.up_scale, cache.slot_of, idx, x, gate,
                                    h2, H, gs, full_dn, stage)
    assert torch.equal(h2, h_ref), "cached up + SiLU with the miss copy differs"
    is_miss = cache.slot_of[idx.long()] < 0
    assert int(is_miss.sum()) == mc
    assert torch.equal(stage[is_miss], w.down_T_Wq[idx.long()[is_miss]]), "staged miss rows differ"
    assert bool((stage[~is_miss] == 0xAB).all()), "hit rows of the staging buffer were written"
    y2 = torch.empty(H, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, full_dn, w.down_T_scale, cache.slot_of, idx, h, y2,
                                 H, gs, ws, stage)
    assert torch.equal(y2, y_ref), "cached down from the copied staging differs"
    # and the whole MLP equals resident DIP
    y_mlp, idx_mlp = dip.cached_dip_mlp_direct(w, cache, x, k, full_up, full_dn)
    y_res, idx_res = dip.dip_mlp(w, x, k)
    assert torch.equal(idx_mlp, idx_res) and torch.equal(y_mlp, y_res)
    sel = idx.long().cpu().numpy()
    assert_close(y, O.sparse_accumulate_f64(w.down_T_Wq.cpu().numpy()[sel], w.down_T_scale.cpu().numpy()[sel],
                                            h.cpu().numpy(), H, gs), f"cached down C={C}")


def test_cached_direct_edge_cases_and_rejections(ops):
    from soinfer import _C
    from soinfer.offload.hot_cache import HotCache

    w = _layer(seed=6)
    H, gs, I = 2048, 128, 6144
    x = torch.randn(H, generator=torch.Generator().manual_seed(1)).half().cuda()
    cache = HotCache.build(w.up_Wq, w.up_scale, w.down_T_Wq, w.down_T_scale, list(range(0, I, 3)))
    # out-of-range channels give NaN rows, never a read
    sel = torch.tensor([5, -1, I, 7], dtype=torch.int32, device="cuda")
    u = torch.zeros(4, dtype=torch.float16, device="cuda")
    _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, w.up_Wq, w.up_scale, cache.slot_of, sel, x, u, H, gs)
    assert not torch.isnan(u[0]) and torch.isnan(u[1]) and torch.isnan(u[2]) and not torch.isnan(u[3])
    # k = 0: the down accumulate writes zeros
    empty = torch.empty(0, dtype=torch.int32, device="cuda")
    y = torch.full((H,), 1.0, dtype=torch.float16, device="cuda")
    ws = torch.zeros(1, dtype=torch.uint8, device="cuda")
    _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, w.down_T_Wq, w.down_T_scale, cache.slot_of, empty,
                                 torch.empty(0, dtype=torch.float16, device="cuda"), y, H, gs, ws)
    assert int(y.count_nonzero()) == 0
    sel = torch.arange(8, dtype=torch.int32, device="cuda")
    u = torch.empty(8, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):  # full matrix in pageable host memory
        _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, w.up_Wq.cpu(), w.up_scale, cache.slot_of, sel, x, u,
                                   H, gs)
    with pytest.raises(RuntimeError):  # slot_of shorter than the channel count
        _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, w.up_Wq, w.up_scale, cache.slot_of[:100], sel, x, u,
                                   H, gs)
    with pytest.raises(RuntimeError):  # scale groups differ between cache and full matrix
        _C.gemv_dip_cached_up_into(cache.up_Wq, cache.up_scale, w.up_Wq, w.up_scale[:, :8].contiguous(),
                                   cache.slot_of, sel, x, u, H, gs)
    with pytest.raises(RuntimeError):  # copy destination without a source
        _C.gemv_dip_cached_up_silu_into(cache.up_Wq, cache.up_scale, w.up_Wq, w.up_scale, cache.slot_of, sel, x,
                                        torch.zeros(I, dtype=torch.float16, device="cuda"), u, H, gs, None,
                                        torch.empty(8, 1024, dtype=torch.uint8, device="cuda"))
    with pytest.raises(RuntimeError):  # staging narrower than a row
        _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, w.down_T_Wq, w.down_T_scale, cache.slot_of, sel,
                                     u, torch.empty(H, dtype=torch.float16, device="cuda"), H, gs,
                                     torch.zeros(1 << 16, dtype=torch.uint8, device="cuda"),
                                     torch.empty(8, 512, dtype=torch.uint8, device="cuda"))
    with pytest.raises(RuntimeError):  # workspace too small
        _C.gemv_dip_cached_down_into(cache.down_Wq, cache.down_scale, w.down_T_Wq, w.down_T_scale, cache.slot_of, sel,
                                     u, torch.empty(H, dtype=torch.float16, device="cuda"), H, gs, ws)
