"""Pins the CPU oracle (oracle/soi_oracle.c) before it is trusted as the checker.

Each oracle function is checked against a golden vector from the reference's
own tests, a closed form, or an independent computation (numpy / torch CPU),
chosen so that a plausible mistake (wrong nibble order, dropped scale,
transposed index, off-by-one tie rule) fails:

  f16 conversion       numpy's IEEE binary16 conversion, exhaustive over all 65536 codes
  quantize_group       torch CPU restatement in soinfer.quant (independent code) + closed-form cases
  pack/unpack_int4     AWQ known-answer bytes (tests/test_quant_roundtrip.py:41-59) + round trips
  gemv_w4/w8           numpy float64 matmul of independently unpacked weights; basis vectors
  topk_rule_a          tau by the v_(k) closed form (golden cases), torch.topk set on distinct data
  topk_rule_b          brute-force sort
  gather_rows          numpy fancy indexing
  sparse_accumulate    numpy h @ W; one-hot rows
  build_dip_desc.      hand cases of tests/test_m8_fused_gemv.py:87-130
  decode_attention     numpy softmax attention written independently (GQA mapping by repeat)
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from soinfer.quant import formats, pack

GOLDEN = Path(__file__).resolve().parent / "golden"


def _rng(seed):
    return np.random.default_rng(seed)


def test_f16_conversion_exhaustive():
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = O.f16_bits_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    assert np.array_equal(f[finite], ref[finite])
    assert np.all(np.isnan(f[np.isnan(ref)]))
    back = O.f32_to_f16_bits(f[finite])
    assert np.array_equal(back, codes[finite])


def test_f32_to_f16_rounding_matches_numpy():
    r = _rng(0)
    vals = np.concatenate([
        r.standard_normal(200000).astype(np.float32) * np.float32(10) ** r.integers(-9, 6, 200000).astype(np.float32),
        np.array([65504, 65519.99, 65520, 1e-8, 2.98e-8, 5.96e-8, 6.1e-5, -0.0, 0.0], np.float32),
    ]).astype(np.float32)
    got = O.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f64_to_f16_is_correctly_rounded():
    r = _rng(1)
    d = r.standard_normal(100000) * 3.0
    got = O.f64_to_f16(d).astype(np.float64)
    # correct rounding: no binary16 value is strictly closer than the one returned
    up = np.nextafter(got.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    dn = np.nextafter(got.astype(np.float16), np.float16(-np.inf)).astype(np.float64)
    err = np.abs(got - d)
    assert np.all(err <= np.abs(up - d)) and np.all(err <= np.abs(dn - d))


# ---------------------------------------------------------------------------
# quantizer + packing
# ---------------------------------------------------------------------------

def test_awq_pack_known_answer():
    kat = json.loads((GOLDEN / "awq_pack_kat.json").read_text())
    q = np.array([kat["values"]], np.int8)
    assert O.pack_int4(q)[0].tolist() == kat["bytes"]
    packed, _ = pack.pack_int4(torch.tensor(kat["values"], dtype=torch.int8))
    assert packed.tolist() == kat["bytes"]
    ragged = O.pack_int4(np.zeros((2, kat["ragged"]["K"]), np.int8))
    assert ragged.shape == (2, kat["ragged"]["packed_bytes_per_row"])


@pytest.mark.parametrize("shape", [(1, 1), (3, 7), (4, 8), (5, 9), (2, 17), (6, 2048)])
def test_pack_unpack_roundtrip_oracle_vs_torch(shape):
    r = _rng(sum(shape))
    q = r.integers(-8, 8, shape).astype(np.int8)
    po = O.pack_int4(q)
    pt, k = pack.pack_int4(torch.from_numpy(q))
    assert k == shape[1]
    assert np.array_equal(po, pt.numpy())
    assert np.array_equal(O.unpack_int4(po, shape[1]), q)
    assert torch.equal(pack.unpack_int4(pt, k), torch.from_numpy(q))


@pytest.mark.parametrize("N,K,gs", [(16, 256, 128), (33, 300, 128), (8, 4099, 128), (5, 65, 32), (64, 2048, 128)])
def test_quantize_group_oracle_matches_torch_restatement(N, K, gs):
    g = torch.Generator().manual_seed(N * 1000 + K)
    w = torch.randn(N, K, generator=g) * 0.02
    w[0, : min(K, 5)] = 0.0
    qo, so = O.quantize_group(w.numpy(), gs)
    qt = formats.quantize(w, formats.QuantConfig(bits=4, granularity="group", group_size=gs))
    assert np.array_equal(qo, qt.qweight.numpy())
    assert np.array_equal(so, qt.scale.numpy())
    assert np.abs(qo).max() <= 7


def test_quantize_group_closed_form_cases():
    # one group of 8: amax 7 -> scale exactly 1, codes are the values rounded half to even
    w = np.array([[7.0, -3.5, 2.5, 0.5, -0.5, 1.5, 6.49, -7.0]], np.float32)
    q, s = O.quantize_group(w, 8)
    assert s.tolist() == [[1.0]]
    assert q.tolist() == [[7, -4, 2, 0, 0, 2, 6, -7]]
    # all-zero group: scale floored at FLT_MIN, codes 0
    q, s = O.quantize_group(np.zeros((1, 16), np.float32), 8)
    assert np.all(q == 0) and np.all(s == np.finfo(np.float32).tiny)
    # INT8: amax 127 -> scale 1
    q, s = O.quantize_group(np.array([[127.0, -1.5, 2.5, 64.0]], np.float32), 4, bits=8)
    assert s.tolist() == [[1.0]] and q.tolist() == [[127, -2, 2, 64]]


def test_quantize_simple_matches_torch():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(12, 40, generator=g)
    for gran in ("per_tensor", "per_channel"):
        qo, so = O.quantize_simple(w.numpy(), gran, bits=8)
        qt = formats.quantize(w, formats.QuantConfig(bits=8, granularity=gran))
        assert np.array_equal(qo, qt.qweight.numpy()) and np.array_equal(so, qt.scale.numpy())


# ---------------------------------------------------------------------------
# GEMVs
# ---------------------------------------------------------------------------

def _int4_problem(N, K, gs, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    q, s = O.quantize_group(w.numpy(), gs)
    Kp = q.shape[1]
    Wq = O.pack_int4(q)
    x = (torch.randn(Kp, generator=g)).half().numpy()
    return Wq, s, x, Kp, q


@pytest.mark.parametrize("N,K,gs", [(16, 256, 128), (7, 4099, 128), (9, 64, 32), (4, 200, 8)])
def test_gemv_w4_f64_matches_numpy(N, K, gs):
    Wq, s, x, Kp, q = _int4_problem(N, K, gs, 11)
    y = O.gemv_w4_f64(Wq, s, x, Kp, gs)
    W = q.astype(np.float64) * np.repeat(s.astype(np.float64), gs, axis=1)[:, :Kp]
    ref = W @ x.astype(np.float64)
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-14)
    y32 = O.gemv_w4_f32(Wq, s, x, Kp, gs)
    assert np.max(np.abs(y32 - ref)) <= 1e-5 * np.max(np.abs(ref)) + 1e-9


def test_gemv_w4_basis_vectors_give_dequant_columns():
    Wq, s, _, Kp, q = _int4_problem(8, 256, 128, 3)
    Wd = O.dequant_int4(Wq, s, Kp, 128)
    assert np.array_equal(Wd, (q.astype(np.float32) * np.repeat(s, 128, axis=1)))
    for k in (0, 1, 7, 8, 127, 128, 255):
        e = np.zeros(Kp, np.float16)
        e[k] = 1.0
        exact = q[:, k].astype(np.float64) * s[:, k // 128].astype(np.float64)
        assert np.array_equal(O.gemv_w4_f64(Wq, s, e, Kp, 128), exact)


@pytest.mark.parametrize("gran", ["per_tensor", "per_channel", "group"])
def test_gemv_w8_f64_matches_numpy(gran):
    g = torch.Generator().manual_seed(7)
    w = torch.randn(10, 96, generator=g)
    if gran == "group":
        q, s = O.quantize_group(w.numpy(), 32, bits=8)
        gs = 32
    else:
        q, s = O.quantize_simple(w.numpy(), gran, bits=8)
        gs = 96
    x = torch.randn(96, generator=g).half().numpy()
    y = O.gemv_w8_f64(q, s, x, gs)
    srep = np.broadcast_to(np.repeat(s.astype(np.float64), gs, axis=1)[:, :96], (10, 96))
    assert np.allclose(y, (q.astype(np.float64) * srep) @ x.astype(np.float64), rtol=1e-12, atol=1e-14)


# ---------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------

def test_topk_golden_cases():
    for c in json.loads((GOLDEN / "topk_rule_a_cases.json").read_text()):
        v = np.array(c["v"], np.float32)
        assert float(O.topk_tau_rule_a(v, c["k"])) == c["tau"], c["why"]
        assert O.topk_rule_a(v, c["k"]).tolist() == c["rule_a"], c["why"]
        assert O.topk_rule_b(v, c["k"]).tolist() == c["rule_b"], c["why"]


def _tau_from_vk(v, k):
    f = np.float32
    vk = np.sort(v)[::-1][k - 1]
    lo, hi = f(0), f(max(f(0), v.max()) + f(1e-3))
    for _ in range(24):
        mid = f(f(0.5) * f(lo + hi))
        lo, hi = (mid, hi) if mid <= vk else (lo, mid)
    return lo


@pytest.mark.parametrize("n,k", [(6144, 768), (6144, 1536), (6144, 3072), (1024, 1), (1024, 1024), (11008, 5504)])
def test_topk_rule_a_random(n, k):
    r = _rng(n + k)
    v = (r.random(n) * 10).astype(np.float32)
    tau = O.topk_tau_rule_a(v, k)
    assert tau == _tau_from_vk(v, k)
    idx = O.topk_rule_a(v, k)
    assert idx.size == k and np.all(np.diff(idx) > 0)
    # distinct continuous data: the selected set is the exact top-k (tests/test_m7_kernels.py:23-54)
    assert set(idx.tolist()) == set(torch.topk(torch.from_numpy(v), k).indices.tolist())
    assert np.array_equal(np.sort(O.topk_rule_b(v, k)), np.sort(idx))


@pytest.mark.parametrize("seed", range(6))
def test_binary16_threshold_shortcut_selects_the_same_values(seed):
    """The selection kernels skip the 24-step replay for binary16 values when v_(k) is a normal binary16 with
    v_(k) >= (max + 1e-3) * 2^-11 and use v_(k) itself as the threshold: after the replay lo <= v_(k) and
    v_(k) - lo <= 3 * hi0 * 2^-24, while the binary16 values below v_(k) are at least v_(k) * 2^-11 away, so no
    binary16 value lies in [lo, v_(k)). Checked here against the oracle's tau (the reference's 24 steps) over gates
    spanning many magnitudes, k from 1 to n, and every finite binary16 value as a candidate."""
    r = _rng(100 + seed)
    every_f16 = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    taken = 0
    for trial in range(300):
        scale = 10.0 ** r.uniform(-6, 4)
        n = int(r.integers(1, 200))
        v = np.abs((r.standard_normal(n) * scale).astype(np.float16)).astype(np.float32)
        if trial % 5 == 0:
            v = np.round(v * 4) / 4  # ties
            v = v.astype(np.float16).astype(np.float32)
        k = int(r.integers(1, n + 1))
        vk = np.sort(v)[::-1][k - 1]
        hi0 = np.float32(np.float32(v.max()) + np.float32(1e-3))
        if not (vk >= np.float32(2.0 ** -14) and vk >= np.float32(hi0 * np.float32(2.0 ** -11))):
            continue
        taken += 1
        tau = O.topk_tau_rule_a(v, k)
        assert tau <= vk
        assert not np.any((every_f16 >= tau) & (every_f16 < vk)), (trial, float(tau), float(vk))
        assert np.array_equal(v >= tau, v >= vk)
    assert taken > 100


def test_topk_rule_a_fp16_gates_ties():
    # |fp16 gate| values tie often; rule A must still return k ascending indices with v >= tau
    r = _rng(9)
    v = np.abs(r.standard_normal(6144).astype(np.float16)).astype(np.float32)
    for k in (768, 1536, 3072):
        tau = O.topk_tau_rule_a(v, k)
        idx = O.topk_rule_a(v, k)
        assert tau == _tau_from_vk(v, k)
        assert idx.size == k and np.all(np.diff(idx) > 0) and np.all(v[idx] >= tau)
        first = np.flatnonzero(v >= tau)[:k]
        assert np.array_equal(idx, first)


# ---------------------------------------------------------------------------
# gather, sparse accumulate, descriptors
# ---------------------------------------------------------------------------

def test_gather_rows_matches_numpy():
    r = _rng(2)
    m = r.integers(0, 256, (300, 24), dtype=np.uint8)
    idx = r.permutation(300)[:37].astype(np.int64)
    assert np.array_equal(O.gather_rows(m, idx), m[idx])


def test_sparse_accumulate_f64_matches_numpy_and_one_hot():
    Wq, s, _, H, q = _int4_problem(20, 256, 64, 4)
    h = (torch.randn(20, generator=torch.Generator().manual_seed(1))).half().numpy()
    y = O.sparse_accumulate_f64(Wq, s, h, H, 64)
    Wd = q.astype(np.float64) * np.repeat(s.astype(np.float64), 64, axis=1)
    assert np.allclose(y, h.astype(np.float64) @ Wd, rtol=1e-12, atol=1e-14)
    for i0 in (0, 5, 19):
        oh = np.zeros(20, np.float16)
        oh[i0] = 1.0
        assert np.array_equal(O.sparse_accumulate_f64(Wq, s, oh, H, 64), Wd[i0])


def test_sparse_accumulate_descriptors_equal_gathered():
    Wq, s, _, H, _ = _int4_problem(24, 128, 32, 5)
    h = np.linspace(-1, 1, 24).astype(np.float16)
    r = _rng(3)
    perm = r.permutation(24)
    cache_rows, stage_rows = sorted(perm[:12].tolist()), perm[12:].tolist()
    desc = np.empty(24, np.int32)
    for slot, j in enumerate(cache_rows):
        desc[j] = slot
    for pos, j in enumerate(stage_rows):
        desc[j] = np.int32(pos - (1 << 31)) | np.int32(0)
        desc[j] = np.array([pos | 0x80000000], dtype=np.uint32).view(np.int32)[0]
    y_desc = O.sparse_accumulate_f64(Wq[cache_rows], s[cache_rows], h, H, 32, Wq[stage_rows], s[stage_rows], desc)
    assert np.array_equal(y_desc, O.sparse_accumulate_f64(Wq, s, h, H, 32))
    x = np.linspace(-2, 2, 128).astype(np.float16)
    up = O.fused_up_f64(Wq[cache_rows], s[cache_rows], Wq[stage_rows], s[stage_rows], desc, x, 128, 32)
    assert np.array_equal(up, O.gemv_w4_f64(Wq, s, x, 128, 32))


def test_build_dip_descriptors_golden_cases():
    for c in json.loads((GOLDEN / "dip_descriptor_cases.json").read_text()):
        slot_of = np.full(c["num_channels"], -1, np.int32)
        for slot, ch in enumerate(c["cached"]):
            slot_of[ch] = slot
        desc, miss, mc = O.build_dip_descriptors(np.array(c["selected"], np.int32), slot_of)
        assert mc == c["expect_miss_count"], c["name"]
        assert miss[:mc].tolist() == c["expect_miss_channels"], c["name"]
        got = [[bool(d & 0x80000000), int(d & 0x7FFFFFFF)] for d in desc.view(np.uint32).tolist()]
        assert got == c["expect_desc"], c["name"]


# ---------------------------------------------------------------------------
# decode attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("NQ,NKV,hd,S,L", [(16, 8, 128, 64, 1), (16, 8, 128, 64, 37), (4, 2, 16, 8, 5),
                                          (6, 3, 24, 10, 10)])
def test_decode_attention_f64_matches_numpy(NQ, NKV, hd, S, L):
    r = _rng(NQ * 7 + L)
    q = r.standard_normal((NQ, hd)).astype(np.float16)
    kc = r.standard_normal((NKV, S, hd)).astype(np.float16)
    vc = r.standard_normal((NKV, S, hd)).astype(np.float16)
    got = O.decode_attention_f64(q, kc, vc, L)
    Kr = np.repeat(kc[:, :L].astype(np.float64), NQ // NKV, axis=0)  # [NQ, L, hd], head h -> kv h // rep
    Vr = np.repeat(vc[:, :L].astype(np.float64), NQ // NKV, axis=0)
    sc = np.einsum("hd,htd->ht", q.astype(np.float64), Kr) / np.sqrt(hd)
    p = np.exp(sc - sc.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    ref = np.einsum("ht,htd->hd", p, Vr)
    assert np.allclose(got, ref, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# decode-step oracle (oracle/decoder.py): closed forms and invariants
# ---------------------------------------------------------------------------

def test_decoder_oracle_rmsnorm_closed_form():
    from oracle import decoder as OD

    for a in (0.5, 3.0, -7.25):
        x = np.full(64, a, np.float16)
        w = np.linspace(0.5, 1.5, 64).astype(np.float16)
        want = (a / np.sqrt(a * a + 1e-6)) * w.astype(np.float64)
        assert np.array_equal(OD.rmsnorm(x, w, 1e-6), OD.f16(want))
    x = (np.random.default_rng(0).standard_normal((3, 256)) * 4).astype(np.float16)
    w = np.ones(256, np.float16)
    # mean (not sum) of squares, per row: eps = 0 makes the result scale-free, exactly for a power of two
    assert np.array_equal(OD.rmsnorm(x, w, 0.0), OD.rmsnorm((x.astype(np.float64) * 2).astype(np.float16), w, 0.0))
    r = OD.rmsnorm(x, w, 0.0).astype(np.float64)
    assert np.allclose(np.mean(r * r, axis=1), 1.0, rtol=2e-3)


def test_decoder_oracle_rope_closed_form():
    from oracle import decoder as OD

    x = np.array([[1.0, 0.0]], np.float16)  # head_dim 2: one pair, inv_freq 1, angle = pos radians
    for pos in (0, 1, 2, 5):
        out = OD.rope(x, 2, 10000.0, pos).astype(np.float64)
        assert np.array_equal(out, OD.f16([[np.cos(pos), np.sin(pos)]]).astype(np.float64))
    y = (np.random.default_rng(1).standard_normal((4, 128))).astype(np.float16)
    assert np.array_equal(OD.rope(y, 128, 1e6, 0), y), "position 0 is the identity"
    r = OD.rope(y, 128, 1e6, 1234).astype(np.float64)
    n0 = y[:, :64].astype(np.float64) ** 2 + y[:, 64:].astype(np.float64) ** 2
    n1 = r[:, :64] ** 2 + r[:, 64:] ** 2
    assert np.allclose(n0, n1, rtol=3e-3, atol=1e-6), "each (i, i + hd/2) pair is rotated"
    ang = OD.rope_angles(128, 1e6, 77)
    assert ang[0] == np.float32(77.0) and ang.dtype == np.float32


def test_decoder_oracle_silu_argmax_add():
    from oracle import decoder as OD

    t = np.linspace(-8, 8, 101)
    assert np.allclose(OD.silu(t) - OD.silu(-t), t, atol=1e-12)
    assert OD.silu(np.array([0.0]))[0] == 0.0
    assert OD.argmax_first(np.array([1, 3, 3, 2], np.float16)) == 1
    assert OD.argmax_first(np.array([1, np.nan, 5, np.nan], np.float16)) == 1
    a = np.random.default_rng(2).standard_normal(1000).astype(np.float16)
    b = np.random.default_rng(3).standard_normal(1000).astype(np.float16)
    assert np.array_equal(OD.residual_add(a, b), (a.astype(np.float32) + b.astype(np.float32)).astype(np.float16))


def test_decoder_oracle_gemv_f16():
    from oracle import decoder as OD

    W = (np.random.default_rng(4).standard_normal((64, 96)) * 0.1).astype(np.float16)
    e = np.zeros(96, np.float16)
    e[17] = 1.0
    assert np.array_equal(OD.gemv_f16(W, e), W[:, 17])
    x = np.random.default_rng(5).standard_normal(96).astype(np.float16)
    ref = W.astype(np.float64) @ x.astype(np.float64)
    assert np.allclose(OD.gemv_f16(W, x).astype(np.float64), ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max())


def test_decoder_oracle_swiglu_gate_up():
    from oracle import decoder as OD

    rng = np.random.default_rng(6)
    Wg = (rng.standard_normal((48, 64)) * 2).astype(np.float16)
    Wu = rng.standard_normal((48, 64)).astype(np.float16)
    # a unit x picks column j of both matrices: silu applies to the gate column only, times the up column
    e = np.zeros(64, np.float16)
    e[5] = 1.0
    assert np.array_equal(OD.swiglu_gate_up(Wg, Wu, e), OD.silu_mul(Wg[:, 5], Wu[:, 5]))
    assert not np.array_equal(OD.swiglu_gate_up(Wu, Wg, e), OD.swiglu_gate_up(Wg, Wu, e))
    # closed forms at the ends of silu: gate sum 0 -> 0, a gate of +30 passes u * 30 (1 + e^-30 = 1 in binary64
    # to 1e-13), a gate of -30 leaves |h| < 30 e^-30 |u|
    Wg2 = np.zeros((3, 64), np.float16)
    Wg2[1, 5], Wg2[2, 5] = 30.0, -30.0
    Wu2 = np.zeros((3, 64), np.float16)
    Wu2[:, 5] = 0.5
    h = OD.swiglu_gate_up(Wg2, Wu2, e).astype(np.float64)
    assert h[0] == 0.0 and h[1] == 15.0 and abs(h[2]) < 1e-11
    # binary64 sums of the full product: against a float64 matmul within the one final fp16 rounding
    x = rng.standard_normal(64).astype(np.float16)
    g = Wg.astype(np.float64) @ x.astype(np.float64)
    u = Wu.astype(np.float64) @ x.astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.allclose(OD.swiglu_gate_up(Wg, Wu, x).astype(np.float64), ref, rtol=2 ** -11, atol=2 ** -24)


def test_threaded_gemv_equals_single_thread():
    """The row-split form used for the multi-core CPU baseline gives the single-thread result exactly (each row is
    still summed by one thread in ascending k), including more threads than rows."""
    r = np.random.default_rng(12)
    for N, K, threads in ((37, 96, 8), (3, 256, 8), (1000, 2048, 5)):
        q = r.integers(-8, 8, (N, K)).astype(np.int8)
        Wq = O.pack_int4(q)
        s = r.random((N, -(-K // 32)), dtype=np.float32)
        x = r.standard_normal(K).astype(np.float16)
        assert np.array_equal(O.gemv_w4_f64(Wq, s, x, K, 32, threads=threads), O.gemv_w4_f64(Wq, s, x, K, 32))


# ---------------------------------------------------------------------------
# the reference's CPU GEMV path (oracle/cpu_path.py), the CPU baseline of bench.py
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K,gs", [(16, 256, 128), (9, 4099, 128), (7, 200, 8), (64, 2048, 128)])
def test_cpu_path_dequantize_equals_c_oracle(N, K, gs):
    """dequantize_group is fl(q*s) per element, exactly the C oracle's soi_ref_dequant_int4 on the packed bytes."""
    from oracle import cpu_path

    w = (torch.randn(N, K, generator=torch.Generator().manual_seed(N + K)) * 0.02).numpy()
    q, s = O.quantize_group(w, gs)
    Wd = cpu_path.dequantize_group(torch.from_numpy(q), torch.from_numpy(s), K, gs)
    ref = O.dequant_int4(O.pack_int4(q), s, q.shape[1], gs)[:, :K]
    assert Wd.shape == (N, K) and np.array_equal(Wd.numpy(), ref)


@pytest.mark.parametrize("N,K,gs", [(33, 4099, 128), (6144, 2048, 128), (5, 64, 32)])
def test_cpu_path_gemv_within_f16_rounding_of_oracle(N, K, gs):
    from oracle import cpu_path

    g = torch.Generator().manual_seed(3 + N)
    w = (torch.randn(N, K, generator=g) * 0.02).numpy()
    q, s = O.quantize_group(w, gs)
    x = torch.randn(q.shape[1], generator=g).half()
    y = cpu_path.gemv_dequant_mv(torch.from_numpy(q), torch.from_numpy(s), x, K, gs)
    ref = O.gemv_w4_f64(O.pack_int4(q), s, x.numpy(), q.shape[1], gs)
    err = np.abs(y.double().numpy() - ref)
    assert err.max() <= 1e-3 * np.abs(ref).max()
    Wd = cpu_path.dequantize_group(torch.from_numpy(q), torch.from_numpy(s), K, gs)
    assert torch.equal(cpu_path.gemv_mv_predequantized(Wd, x), y)


def test_cpu_path_basis_vector_gives_f16_column():
    from oracle import cpu_path

    w = (torch.randn(8, 256, generator=torch.Generator().manual_seed(1)) * 3.0).numpy()
    q, s = O.quantize_group(w, 128)
    Wd = O.dequant_int4(O.pack_int4(q), s, 256, 128)
    for k in (0, 77, 255):
        e = torch.zeros(256, dtype=torch.float16)
        e[k] = 1.0
        y = cpu_path.gemv_dequant_mv(torch.from_numpy(q), torch.from_numpy(s), e, 256, 128)
        assert np.array_equal(y.numpy(), Wd[:, k].astype(np.float16))


def test_cpu_path_topk_is_rule_a_on_distinct_values():
    """torch.topk (the reference test's top-k oracle) picks the rule-A set when the values are distinct."""
    from oracle import cpu_path

    r = _rng(31)
    v = (r.random(6144) * 10).astype(np.float32)
    for k in (1, 768, 3072, 6144):
        got = set(cpu_path.topk_indices(torch.from_numpy(v), k).tolist())
        assert got == set(O.topk_rule_a(v, k).tolist())


def test_cpu_path_gather_equals_numpy_indexing():
    from oracle import cpu_path

    r = _rng(32)
    m = r.integers(0, 256, (500, 64), dtype=np.uint8)
    idx = np.sort(r.permutation(500)[:123]).astype(np.int64)
    got = cpu_path.gather_rows(torch.from_numpy(m), torch.from_numpy(idx)).numpy()
    assert np.array_equal(got, O.gather_rows(m, idx)) and np.array_equal(got, m[idx])


def test_cpu_path_sparse_accumulate_within_f16_rounding_of_oracle():
    from oracle import cpu_path

    g = torch.Generator().manual_seed(33)
    k, H, gs = 300, 2048, 128
    w = (torch.randn(k, H, generator=g) * 0.02).numpy()
    q, s = O.quantize_group(w, gs)
    h = torch.randn(k, generator=g).half()
    Wd = cpu_path.dequantize_group(torch.from_numpy(q), torch.from_numpy(s), H, gs)
    y = cpu_path.sparse_accumulate_ref(h, Wd)
    ref = O.sparse_accumulate_f64(O.pack_int4(q), s, h.numpy(), H, gs)
    assert np.abs(y.double().numpy() - ref).max() <= 1e-3 * np.abs(ref).max()


@pytest.mark.parametrize("L", [1, 17, 300])
def test_cpu_path_attention_within_tolerance_of_oracle(L):
    from oracle import cpu_path

    g = torch.Generator().manual_seed(34 + L)
    q = torch.randn(16, 128, generator=g).half()
    kc = torch.randn(8, 320, 128, generator=g).half()
    vc = torch.randn(8, 320, 128, generator=g).half()
    out = cpu_path.decode_attention_ref(q, kc, vc, L)
    ref = O.decode_attention_f64(q.numpy(), kc.numpy(), vc.numpy(), L)
    assert np.abs(out.double().numpy() - ref).max() <= 1e-3 * np.abs(ref).max()
