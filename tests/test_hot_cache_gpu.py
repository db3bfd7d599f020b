"""Hot-channel cache, calibration counts and miss accounting on the GPU.

Counterparts of the reference's tests:
  * tests/test_m8_hot_cache_gpu.py:107-166: HotCache.build maps every channel to its slot (hot set given in
    any order) or -1, accepts an empty hot set, and holds exactly the packed bytes and scales of an
    INDEPENDENT quantization of the raw weights (the oracle's quantizer and packer, not soinfer.quant);
  * tests/test_m8_calibration.py:86-120: per-layer selection counts sum to tokens * k, no channel is counted
    more than once per token, and two runs on identically built weights give equal counts;
  * tests/test_m8_cached_dip_pipeline.py:141-179: miss bytes are zero with a full cache and k rows of up plus
    k rows of down^T with an empty one;
  * tests/test_m7_dip_pipeline.py:95-139: DIP with k = I selects every channel and agrees with the dense MLP
    (whose down_proj is quantized along the other axis) in direction, and exactly with the oracle's sum over
    all down^T rows.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu

H, I, GS = 2048, 6144, 128


@pytest.fixture(scope="module")
def raw(cuda):
    """Raw fp32 up [I, H] and down [H, I] weights, and both packed forms from soinfer.quant on the device."""
    from soinfer.quant import formats, pack

    g = torch.Generator().manual_seed(21)
    up = torch.randn(I, H, generator=g) * 0.02
    down = torch.randn(H, I, generator=g) * 0.02

    def q(w):
        qt = formats.quantize(w.cuda(), formats.QuantConfig(bits=4, granularity="group", group_size=GS))
        Wq, _ = pack.pack_int4(qt.qweight)
        return Wq.contiguous(), qt.scale.contiguous()

    return {"up": up, "down": down, "up_q": q(up), "down_T_q": q(down.t().contiguous())}


def test_hot_cache_slot_of_for_unsorted_hot_set(raw):
    from soinfer.offload.hot_cache import HotCache

    (uW, uS), (dW, dS) = raw["up_q"], raw["down_T_q"]
    given = [90, 3, 41, 8, 15, 7, 40, 6143]
    cache = HotCache.build(uW, uS, dW, dS, given)
    want = sorted(given)
    assert cache.cache_size == len(given)
    assert torch.equal(cache.hot_indices.cpu(), torch.tensor(want, dtype=torch.int64))
    slot_of = cache.slot_of.cpu().numpy()
    expect = np.full(I, -1, np.int32)
    expect[want] = np.arange(len(want), dtype=np.int32)
    assert slot_of.dtype == np.int32 and np.array_equal(slot_of, expect)


def test_hot_cache_empty_hot_set(raw):
    from soinfer.offload.hot_cache import HotCache

    (uW, uS), (dW, dS) = raw["up_q"], raw["down_T_q"]
    for cache in (HotCache.build(uW, uS, dW, dS, []),
                  HotCache.from_host(uW.cpu().pin_memory(), uS, dW.cpu().pin_memory(), dS, [])):
        assert cache.cache_size == 0
        assert cache.up_Wq.shape == (0, uW.shape[1]) and cache.down_Wq.shape == (0, dW.shape[1])
        assert cache.up_scale.shape[0] == 0 and cache.down_scale.shape[0] == 0
        assert bool((cache.slot_of == -1).all()) and cache.slot_of.numel() == I


@pytest.mark.parametrize("source", ["device", "pinned_host"])
def test_hot_cache_holds_independently_quantized_rows(raw, source):
    from soinfer.offload.hot_cache import HotCache

    (uW, uS), (dW, dS) = raw["up_q"], raw["down_T_q"]
    hot = sorted(torch.randperm(I, generator=torch.Generator().manual_seed(4))[: I // 3].tolist())
    if source == "device":
        cache = HotCache.build(uW, uS, dW, dS, hot)
    else:
        cache = HotCache.from_host(uW.cpu().pin_memory(), uS, dW.cpu().pin_memory(), dS, hot)
    # ground truth from the raw weights through the oracle's own quantizer and AWQ packer
    q_up, s_up = O.quantize_group(raw["up"].numpy(), GS)
    q_dn, s_dn = O.quantize_group(raw["down"].t().contiguous().numpy(), GS)
    Wup, Wdn = O.pack_int4(q_up), O.pack_int4(q_dn)
    assert np.array_equal(cache.up_Wq.cpu().numpy(), Wup[hot])
    assert np.array_equal(cache.up_scale.cpu().numpy(), s_up[hot])
    assert np.array_equal(cache.down_Wq.cpu().numpy(), Wdn[hot])
    assert np.array_equal(cache.down_scale.cpu().numpy(), s_dn[hot])
    # the cached rows dequantize to within half a quantization step of the raw weights
    deq = O.dequant_int4(cache.up_Wq.cpu().numpy(), cache.up_scale.cpu().numpy(), H, GS)
    step = np.repeat(cache.up_scale.cpu().numpy(), GS, axis=1)[:, :H]
    assert np.all(np.abs(deq - raw["up"].numpy()[hot]) <= 0.5 * step * (1 + 1e-6))


def _dip_weights(raw, seed=5):
    from helpers import int4_problem
    from soinfer.runtime.dip import DipMLPWeights

    gate = int4_problem(I, H, GS, seed=seed)
    (uW, uS), (dW, dS) = raw["up_q"], raw["down_T_q"]
    return DipMLPWeights(gate["Wq_d"], gate["s_d"], uW, uS, dW, dS, hidden_size=H, group_size=GS)


@pytest.mark.parametrize("k", [768, 3072])
def test_cached_dip_miss_bytes_full_and_empty_cache(raw, k):
    from soinfer.offload.hot_cache import HotCache
    from soinfer.runtime import dip

    w = _dip_weights(raw)
    x = torch.randn(H, generator=torch.Generator().manual_seed(9)).half().cuda()
    y_ref, idx_ref = dip.dip_mlp(w, x, k)
    full = HotCache.build(w.up_Wq, w.up_scale, w.down_T_Wq, w.down_T_scale, list(range(I)))
    empty = HotCache.build(w.up_Wq, w.up_scale, w.down_T_Wq, w.down_T_scale, [])
    miss_bytes = []
    y_full, idx_full, mc_full = dip.cached_dip_mlp(w, full, x, k, miss_bytes=miss_bytes)
    y_empty, idx_empty, mc_empty = dip.cached_dip_mlp(w, empty, x, k, miss_bytes=miss_bytes)
    assert mc_full == 0 and miss_bytes[0] == 0
    assert mc_empty == k and miss_bytes[1] == k * (w.up_Wq.shape[1] + w.down_T_Wq.shape[1]) == k * 2048
    for y, idx in ((y_full, idx_full), (y_empty, idx_empty)):
        assert torch.equal(idx, idx_ref) and torch.equal(y, y_ref)


def test_dip_at_full_k_matches_dense_mlp(raw):
    """k = I: every channel is selected (ascending), the sparse down over all rows of down^T equals the oracle's
    binary64 sum, and the dense MLP (down_proj [H, I] quantized along I) points the same way (its quantization
    groups run along the other axis, so the two differ by quantization noise only)."""
    from soinfer import ops
    from soinfer.quant import formats, pack
    from soinfer.runtime import dip

    w = _dip_weights(raw)
    x = torch.randn(H, generator=torch.Generator().manual_seed(13)).half().cuda()
    y_dip, idx = dip.dip_mlp(w, x, I)
    assert torch.equal(idx.cpu(), torch.arange(I, dtype=torch.int32))
    gate = ops.gemv_w4a16_group_lop3(w.gate_Wq, w.gate_scale, x, H, GS)
    up = ops.gemv_w4a16_group_lop3(w.up_Wq, w.up_scale, x, H, GS)
    h = dip.silu_gate(gate, idx, up)
    assert torch.equal(h, (torch.nn.functional.silu(gate.float()) * up.float()).half())
    ref = O.sparse_accumulate_f64(w.down_T_Wq.cpu().numpy(), w.down_T_scale.cpu().numpy(), h.cpu().numpy(), H, GS)
    assert_close(y_dip, ref, "DIP k=I")
    qt = formats.quantize(raw["down"].cuda(), formats.QuantConfig(bits=4, granularity="group", group_size=GS))
    dW, _ = pack.pack_int4(qt.qweight)
    y_dense = ops.gemv_w4a16_group_lop3(dW.contiguous(), qt.scale.contiguous(), h, I, GS)
    cos = torch.nn.functional.cosine_similarity(y_dip.float()[None], y_dense.float()[None]).item()
    assert cos > 0.99, f"DIP (k=I) and dense MLP outputs differ in direction: cosine {cos:.4f}"
    assert_close(y_dense, O.gemv_w4_f64(dW.cpu().numpy(), qt.scale.cpu().numpy(), h.cpu().numpy(), I, GS),
                 "dense down", floor=5e-5)  # K = 6144 through v_dot2 chains (tests/helpers.py)


TINY = dict(hidden=256, layers=3, q_heads=4, kv_heads=2, head_dim=64, intermediate=512, vocab=1000,
            group_size=128, max_seq=64)


def test_calibration_counts_consistent_and_deterministic(cuda):
    from soinfer.runtime import decoder as D
    from soinfer.runtime import dip

    cfg = D.DecoderConfig(**TINY)
    tokens = [1, 5, 2, 8, 3, 7, 4, 9]
    k = 64
    counts_a = D.calibrate_channel_counts(D.random_decoder(cfg, seed=9, linear_std=0.05), k, tokens)
    counts_b = D.calibrate_channel_counts(D.random_decoder(cfg, seed=9, linear_std=0.05), k, tokens)
    assert len(counts_a) == cfg.layers
    for ca, cb in zip(counts_a, counts_b):
        assert ca.shape == (cfg.intermediate,) and ca.dtype == torch.int64
        assert int(ca.sum()) == len(tokens) * k
        assert int(ca.min()) >= 0 and int(ca.max()) <= len(tokens)
        assert torch.equal(ca, cb)
    # one layer's MLP alone (dip.calibrate_channel_frequencies): same invariants
    from helpers import int4_problem
    from soinfer.runtime.dip import DipMLPWeights

    mats = [int4_problem(512, 256, 128, seed=40 + i) for i in range(3)]
    wl = DipMLPWeights(*(t for m in mats for t in (m["Wq_d"], m["s_d"])), hidden_size=256, group_size=128)
    xs = torch.randn(10, 256, generator=torch.Generator().manual_seed(2)).half().cuda()
    c1 = dip.calibrate_channel_frequencies(wl, xs, 100)
    c2 = dip.calibrate_channel_frequencies(wl, xs, 100)
    assert int(c1.sum()) == 10 * 100 and int(c1.max()) <= 10 and torch.equal(c1, c2)
