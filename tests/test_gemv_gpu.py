"""INT4 / INT8 dequant-GEMV parity on the GPU (counterpart of the reference's tests/test_m4_kernels.py).

HIP kernels vs. the CPU oracle's binary64 GEMV on identical packed bytes:
  * basis vectors x = e_k give the binary16 rounding of the binary32 dequantized column, bit-exact;
  * seeded random problems within the tolerance rule of tests/helpers.py (1e-3);
  * gemv_w4a16_group (scalar nibble dequant) == gemv_w4a16_group_lop3 (bitfield dequant), bit-exact;
  * unaligned / ragged shapes take the dword path and agree bit-exactly with the 16-byte path;
  * the reference's argument checks raise RuntimeError.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import oracle as O

pytestmark = pytest.mark.gpu

W4_FNS = ["gemv_w4a16_group", "gemv_w4a16_group_lop3"]


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


@pytest.mark.parametrize("fn", W4_FNS)
@pytest.mark.parametrize("K", [256, 4096])
def test_w4_basis_vectors_exact(ops, fn, K):
    p = int4_problem(16, K, 128, seed=2, std=3.0)
    Wd = O.dequant_int4(p["Wq"], p["s"], p["K"], 128)  # binary32 fl(q*s)
    expect = torch.from_numpy(Wd.astype(np.float16))
    eye = torch.eye(K, dtype=torch.float16, device="cuda")
    for k in range(0, K, 41):
        y = getattr(ops, fn)(p["Wq_d"], p["s_d"], eye[k].contiguous(), K, 128)
        assert torch.equal(y.cpu(), expect[:, k]), f"{fn} K={K} column {k}"


SHAPES = [
    (512, 4096, 128), (512, 4099, 128),  # reference test shapes (4099 pads to 4224)
    (6144, 2048, 128), (2048, 6144, 128), (2048, 2048, 128), (1024, 2048, 128),  # Qwen3-1.7B
    (2049, 6144, 128), (1000, 5120, 128),  # multi-pass tiles with a ragged last tile / a pass count of 2.5
    (2560, 9728, 128), (4096, 12288, 64),  # 4-row multi-pass tiles (Qwen3-4B / 8B down), two load batches
    (37, 512, 32), (64, 256, 64), (33, 200, 8), (17, 1000, 40),  # non-32-multiple groups
    (1, 8, 8), (3, 100, 16),  # tiny / unaligned rows
]


@pytest.mark.parametrize("N,K,gs", SHAPES)
def test_w4_matches_oracle(ops, N, K, gs):
    p = int4_problem(N, K, gs, seed=N + K + gs)
    ref = O.gemv_w4_f64(p["Wq"], p["s"], p["x"], p["K"], gs)
    a = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)
    b = ops.gemv_w4a16_group(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs)
    assert_close(a, ref, f"int4 {N}x{K} gs{gs}")
    assert torch.equal(a, b), "scalar and bitfield dequant must agree bit for bit"


def test_w4_unaligned_path_bit_identical(ops):
    p = int4_problem(96, 2048, 128, seed=5)
    y_vec = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], 128)
    # same bytes at a 4-byte (not 16-byte) aligned address, x likewise misaligned
    wbuf = torch.empty(p["Wq_d"].numel() + 4, dtype=torch.uint8, device="cuda")
    wv = wbuf[4:].view(96, -1)
    wv.copy_(p["Wq_d"])
    xbuf = torch.empty(p["K"] + 2, dtype=torch.float16, device="cuda")
    xv = xbuf[2:]
    xv.copy_(p["x_d"])
    y_dw = ops.gemv_w4a16_group_lop3(wv, p["s_d"], xv, p["K"], 128)
    assert torch.equal(y_vec, y_dw)


def test_w4_deterministic(ops):
    p = int4_problem(6144, 2048, 128, seed=8)
    first = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], 128)
    for _ in range(5):
        assert torch.equal(first, ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], 128))


@pytest.mark.parametrize("fn", W4_FNS)
def test_w4_rejects_bad_arguments(ops, fn):
    p = int4_problem(4, 64, 32, seed=1)
    f = getattr(ops, fn)
    with pytest.raises(RuntimeError):
        f(p["Wq_d"], p["s_d"], p["x_d"], 64, 7)  # group_size not a multiple of 8
    with pytest.raises(RuntimeError):
        f(p["Wq_d"], p["s_d"][:, :1].contiguous(), p["x_d"], 64, 32)  # too few groups
    with pytest.raises(RuntimeError):
        f(p["Wq_d"], p["s_d"], p["x_d"][:-8].contiguous(), 56, 32)  # Wq width != ceil(K/8)*4
    with pytest.raises(RuntimeError):
        f(p["Wq_d"].cpu(), p["s_d"], p["x_d"], 64, 32)  # not a device tensor
    q65 = int4_problem(4, 65, 32, seed=2)  # ragged: 65 -> 96 padded, 3 groups
    with pytest.raises(RuntimeError):
        f(q65["Wq_d"], q65["s_d"][:, :2].contiguous(), q65["x_d"], q65["K"], 32)


# ---------------------------------------------------------------------------
# INT8
# ---------------------------------------------------------------------------

def _int8_problem(N, K, gran, gs, seed, std=1.0):
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(N, K, generator=g) * std).numpy()
    if gran == "group":
        q, s = O.quantize_group(w, gs, bits=8)
        q = q[:, :K].copy()  # K is a multiple of gs in these cases
    else:
        q, s = O.quantize_simple(w, gran, bits=8)
    x = torch.randn(K, generator=g).half()
    return q, s, x


W8 = [("per_tensor", None), ("per_channel", None), ("group", 128)]


@pytest.mark.parametrize("gran,gs", W8)
def test_w8_basis_vectors_exact(ops, gran, gs):
    K = 256
    q, s, _ = _int8_problem(16, K, gran, gs or K, seed=0, std=3.0)
    gsize = gs or K
    srep = np.broadcast_to(np.repeat(s, gsize, axis=1)[:, :K], (16, K)) if s.shape[1] > 1 else np.broadcast_to(s, (16, K))
    expect = (q.astype(np.float32) * srep.astype(np.float32)).astype(np.float16)
    Wq, sd = torch.from_numpy(q).cuda(), torch.from_numpy(np.ascontiguousarray(s)).cuda()
    eye = torch.eye(K, dtype=torch.float16, device="cuda")
    for k in range(0, K, 37):
        y = ops.gemv_w8a16(Wq, sd, eye[k].contiguous(), gsize)
        assert torch.equal(y.cpu(), torch.from_numpy(expect[:, k].copy())), f"{gran} column {k}"


# tiles: (512, 4096) 1 row x 4 passes; (6144, 2048) 4 x 2; (2048, 6144) 2 x 3; (2048, 2048) and (1024, 2048) x 2
# passes (the q/o and k/v projections) -- all full;
# (4097, 3072) 2 x 3 with a partial last tile; (8200, 1040) 4 x 2 with idle lanes; (2049, 100) and (7, 96) ragged;
# group sizes only where they divide K
@pytest.mark.parametrize("gran,gs,N,K", [(g, gs, N, K) for g, gs in W8 + [("group", 32), ("group", 4), ("group", 12)]
                                         for N, K in [(512, 4096), (6144, 2048), (2048, 6144), (2048, 2048),
                                                      (1024, 2048), (7, 96), (4097, 3072), (8200, 1040), (2049, 100)]
                                         if not (gs and K % gs)])
def test_w8_matches_oracle(ops, gran, gs, N, K):
    q, s, x = _int8_problem(N, K, gran, gs or K, seed=N + K)
    ref = O.gemv_w8_f64(q, s, x.numpy(), gs or K)
    y = ops.gemv_w8a16(torch.from_numpy(q).cuda(), torch.from_numpy(np.ascontiguousarray(s)).cuda(), x.cuda(), gs or K)
    assert_close(y, ref, f"int8 {gran} {N}x{K}")


def test_w8_ragged_k_path(ops):
    q, s, x = _int8_problem(9, 101, "per_channel", 101, seed=3)
    ref = O.gemv_w8_f64(q, s, x.numpy(), 101)
    y = ops.gemv_w8a16(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), x.cuda(), 101)
    assert_close(y, ref, "int8 ragged")


def test_w8_rejects_bad_arguments(ops):
    g = torch.Generator().manual_seed(0)
    w = torch.randn(4, 64, generator=g).numpy()
    q, s = O.quantize_group(w, 16, bits=8)
    Wq, sd = torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda()
    x = torch.randn(64, generator=g).half().cuda()
    with pytest.raises(RuntimeError):
        ops.gemv_w8a16(Wq, sd[:, :3].contiguous(), x, 16)  # too few groups
    q3, s3 = O.quantize_group(w, 3, bits=8)  # num_groups > 1 with gs not a multiple of 4
    with pytest.raises(RuntimeError):
        ops.gemv_w8a16(torch.from_numpy(q3[:, :64].copy()).cuda(), torch.from_numpy(s3[:, :22].copy()).cuda(), x, 3)


# ---------------------------------------------------------------------------
# batched (one launch, many problems)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("N,K,P", [(6144, 2048, 5), (1024, 2048, 9), (2048, 6144, 3), (33, 96, 4), (7, 200, 3)])
def test_batched_bit_identical_to_single(ops, N, K, P):
    probs = [int4_problem(N, K, 8 if K % 32 else 32 if K == 96 else 128, seed=100 + i) for i in range(P)]
    gs = probs[0]["gs"]
    ys = ops.gemv_w4a16_batched([p["Wq_d"] for p in probs], [p["s_d"] for p in probs], [p["x_d"] for p in probs],
                                probs[0]["K"], gs)
    for p, y in zip(probs, ys):
        assert torch.equal(y, ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs))
    assert_close(ys[0], O.gemv_w4_f64(probs[0]["Wq"], probs[0]["s"], probs[0]["x"], probs[0]["K"], gs), "batched")


def test_batched_rejects_mismatched_shapes(ops):
    a = int4_problem(64, 256, 128, seed=1)
    b = int4_problem(32, 256, 128, seed=2)
    with pytest.raises(RuntimeError):
        ops.gemv_w4a16_batched([a["Wq_d"], b["Wq_d"]], [a["s_d"], b["s_d"]], [a["x_d"], b["x_d"]], 256, 128)


# ---------------------------------------------------------------------------
# grouped (one launch, several shapes)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("gs,shapes", [
    (128, [(6144, 2048, 2), (2048, 6144, 2), (2048, 2048, 3), (1024, 2048, 3)]),  # Qwen3-1.7B classes (FULL path)
    (32, [(37, 512, 2), (64, 256, 3), (7, 96, 2)]),  # ragged N, short rows
    (8, [(33, 200, 2), (5, 8, 1), (17, 1000, 2)]),  # K not a multiple of 32 (dword path)
])
def test_grouped_bit_identical_to_single(ops, gs, shapes):
    probs = []
    for i, (N, K, P) in enumerate(shapes):
        for j in range(P):
            probs.append(int4_problem(N, K, gs, seed=1000 + 17 * i + j))
    # interleave shapes so the grouping has to reorder
    probs = probs[::2] + probs[1::2]
    grp = ops.GemvGroup([(p["Wq_d"], p["s_d"], p["x_d"], p["K"]) for p in probs], gs)
    ys = grp.run()
    for p, y in zip(probs, ys):
        assert torch.equal(y, ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], gs))
    assert_close(ys[0], O.gemv_w4_f64(probs[0]["Wq"], probs[0]["s"], probs[0]["x"], probs[0]["K"], gs), "grouped")
    again = [y.clone() for y in ys]
    grp.run()
    assert all(torch.equal(a, b) for a, b in zip(again, grp.ys))


def test_grouped_rejects_bad_arguments(ops):
    a = int4_problem(64, 256, 128, seed=1)
    with pytest.raises(RuntimeError):
        ops.GemvGroup([(a["Wq_d"], a["s_d"], a["x_d"], 512)], 128)  # K does not match the packed width
    many = [int4_problem(8 * (i + 1), 64, 32, seed=i) for i in range(9)]
    with pytest.raises(RuntimeError):
        ops.GemvGroup([(p["Wq_d"], p["s_d"], p["x_d"], 64) for p in many], 32)  # 9 distinct shapes


# ---------------------------------------------------------------------------
# misaligned operands of the batched / grouped forms
# ---------------------------------------------------------------------------

def _offset_view(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of t starting 2 bytes past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 8, dtype=t.dtype, device=t.device)
    v = buf[1:1 + t.numel()].view(t.shape)
    v.copy_(t)
    assert v.is_contiguous() and v.data_ptr() % 16 == 2
    return v


def test_batched_and_grouped_reject_misaligned_views(ops):
    p = int4_problem(1024, 2048, 128, seed=7)
    xo = _offset_view(p["x_d"])
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ops.GemvBatch([p["Wq_d"]], [p["s_d"]], [xo], 2048, 128)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ops.GemvGroup([(p["Wq_d"], p["s_d"], xo, 2048)], 128)
    # K % 32 != 0 takes the dword path, where any 2-byte aligned x is fine
    r = int4_problem(33, 200, 8, seed=8)
    xr = _offset_view(r["x_d"])
    ys = ops.GemvGroup([(r["Wq_d"], r["s_d"], xr, r["K"])], 8).run()
    assert torch.equal(ys[0], ops.gemv_w4a16_group_lop3(r["Wq_d"], r["s_d"], r["x_d"], r["K"], 8))


def test_batched_table_with_misaligned_x_writes_nan_rows(ops):
    """Through the raw pointer tables (no host check) a misaligned problem comes back as NaN rows, never as
    unwritten memory; the aligned problem in the same launch is unaffected."""
    from soinfer import _C

    a = int4_problem(1024, 2048, 128, seed=9)
    b = int4_problem(1024, 2048, 128, seed=10)
    xb = _offset_view(b["x_d"])
    ys = [torch.zeros(1024, dtype=torch.float16, device="cuda") for _ in range(2)]

    def table(ts):
        return torch.tensor([t.data_ptr() for t in ts], dtype=torch.int64, device="cuda")

    _C.gemv_w4a16_batched(table([a["Wq_d"], b["Wq_d"]]), table([a["s_d"], b["s_d"]]), table([a["x_d"], xb]),
                          table(ys), 1024, 2048, 128)
    assert torch.equal(ys[0], ops.gemv_w4a16_group_lop3(a["Wq_d"], a["s_d"], a["x_d"], 2048, 128))
    assert torch.isnan(ys[1]).all()
    yg = [torch.zeros(1024, dtype=torch.float16, device="cuda") for _ in range(2)]
    _C.gemv_w4a16_grouped(table([a["Wq_d"], b["Wq_d"]]), table([a["s_d"], b["s_d"]]), table([a["x_d"], xb]),
                          table(yg), [2], [1024], [2048], 128)
    assert torch.equal(yg[0], ys[0])
    assert torch.isnan(yg[1]).all()


def test_grouped_large_table_with_null_and_misaligned_problems(ops):
    """A grouped launch of the Qwen3 classes through the raw pointer tables (4992 8-row tiles): a problem whose
    y pointer is null is skipped and leaves the other outputs alone, a misaligned x gives NaN rows, and every
    other problem, the K = 6144 ones (three passes per row) included, equals the single GEMV bit for bit."""
    from soinfer import _C

    shapes = [(6144, 2048)] * 5 + [(2048, 6144)] * 3 + [(1024, 2048)] * 3
    probs = [int4_problem(N, K, 128, seed=300 + i) for i, (N, K) in enumerate(shapes)]
    xs = [p["x_d"] for p in probs]
    xs[9] = _offset_view(probs[9]["x_d"])  # misaligned x: NaN rows
    ys = [torch.full((N,), 7.0, dtype=torch.float16, device="cuda") for N, _ in shapes]

    def table(ts):
        return torch.tensor([t.data_ptr() if t is not None else 0 for t in ts], dtype=torch.int64, device="cuda")

    yt = [y if i != 6 else None for i, y in enumerate(ys)]  # problem 6: null y, skipped
    # classes in table order: 5 x (6144, 2048), 3 x (2048, 6144), 3 x (1024, 2048)
    _C.gemv_w4a16_grouped(table([p["Wq_d"] for p in probs]), table([p["s_d"] for p in probs]), table(xs), table(yt),
                          [5, 3, 3], [6144, 2048, 1024], [2048, 6144, 2048], 128)
    for i, p in enumerate(probs):
        if i == 6:
            assert (ys[i] == 7.0).all()
        elif i == 9:
            assert torch.isnan(ys[i]).all()
        else:
            assert torch.equal(ys[i], ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], p["x_d"], p["K"], 128)), i


@pytest.mark.parametrize("xkind", ["normal", "swiglu", "positive"])
def test_int4_gemv_accumulation_error_bound(ops, xkind):
    """The fp32 accumulation error of the INT4 GEMV over K = 6144 (the down projection), separated from the
    binary16 output rounding: max over outputs of |y - ref| - ulp16(ref)/2 stays below 3e-5 * max|ref|. The
    kernel's v_dot2_f32_f16 chains do not round to nearest even, which makes this ~30x the error of an fp32
    matmul of the dequantized weights (checked alongside: torch.mv stays below 1e-6 * max|ref|), and still
    ~30x inside the 1e-3 parity bound. With x = ones the dot products sum small integers exactly and the
    error drops to the round-to-nearest scale FMAs."""
    N, K, gs = 2048, 6144, 128
    p = int4_problem(N, K, gs, seed=21)
    g = torch.Generator().manual_seed(13)
    if xkind == "normal":
        x = torch.randn(K, generator=g)
    elif xkind == "swiglu":
        x = torch.nn.functional.silu(torch.randn(K, generator=g) * 0.9) * torch.randn(K, generator=g) * 0.9
    else:
        x = torch.randn(K, generator=g).abs()
    x = x.half()
    ref = O.gemv_w4_f64(p["Wq"], p["s"], x.numpy(), K, gs)
    scale = np.abs(ref).max()
    y = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], x.cuda(), K, gs).double().cpu().numpy()
    half_ulp = 0.5 * np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    excess = (np.abs(y - ref) - half_ulp).max()
    assert excess <= 3e-5 * scale, f"{xkind}: accumulation error {excess / scale:.2e} of max|ref|"
    Wd = torch.from_numpy(O.dequant_int4(p["Wq"], p["s"], K, gs)).cuda()
    yt = torch.mv(Wd, x.cuda().float()).double().cpu().numpy()
    assert np.abs(yt - ref).max() <= 1e-6 * scale
    ones = torch.ones(K, dtype=torch.float16)
    y1 = ops.gemv_w4a16_group_lop3(p["Wq_d"], p["s_d"], ones.cuda(), K, gs).double().cpu().numpy()
    r1 = O.gemv_w4_f64(p["Wq"], p["s"], ones.numpy(), K, gs)
    # integer dot products: only the (round-to-nearest) scale FMAs and the lane reduction round
    assert (np.abs(y1 - r1) - 0.5 * np.spacing(np.abs(r1).astype(np.float16)).astype(np.float64)).max() <= \
        2e-7 * np.abs(r1).max()


@pytest.mark.parametrize("gran,gs,N,K,P", [(g, gs, N, K, P) for g, gs in W8 + [("group", 32), ("group", 12)]
                                           for N, K, P in [(6144, 2048, 3), (2048, 6144, 2), (1024, 2048, 5),
                                                           (4097, 3072, 2), (7, 96, 4), (2049, 100, 3)]
                                           if not (gs and K % gs)])
def test_w8_batched_equals_single(ops, gran, gs, N, K, P):
    """Int8Batch: P same-shape INT8 GEMVs in one launch, each bit-identical to the single launch (vector and
    ragged-K tiles, per-tensor / per-channel / group scales, partial last tiles), and within the oracle's tolerance
    (group sizes only where they divide K)."""
    probs = [_int8_problem(N, K, gran, gs or K, seed=17 * p + N + K) for p in range(P)]
    Ws = [torch.from_numpy(q).cuda() for q, _, _ in probs]
    Ss = [torch.from_numpy(np.ascontiguousarray(s)).cuda() for _, s, _ in probs]
    xs = [x.cuda() for _, _, x in probs]
    ys = ops.Int8Batch(Ws, Ss, xs, gs or K).run()
    for p in range(P):
        assert torch.equal(ys[p], ops.gemv_w8a16(Ws[p], Ss[p], xs[p], gs or K)), f"problem {p}"
    q, s, x = probs[-1]
    assert_close(ys[-1], O.gemv_w8_f64(q, s, x.numpy(), gs or K), f"int8 batched {gran} {N}x{K}")


def test_w8_batched_rejects_mixed_shapes(ops):
    a = _int8_problem(64, 128, "per_channel", 128, seed=1)
    b = _int8_problem(32, 128, "per_channel", 128, seed=2)
    with pytest.raises(RuntimeError, match="Int8Batch"):
        ops.Int8Batch([torch.from_numpy(a[0]).cuda(), torch.from_numpy(b[0]).cuda()],
                      [torch.from_numpy(a[1]).cuda(), torch.from_numpy(b[1]).cuda()], [a[2].cuda(), b[2].cuda()], 128)
