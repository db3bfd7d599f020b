"""topk_threshold_select parity on the GPU (counterpart of the reference's tests/test_m7_kernels.py).

The HIP kernel must return exactly the oracle's rule-A indices (the reference
semantics of csrc/kernels/topk_select.cu:10-96) on identical fp32 inputs:
same set, same ascending order, same count -- including heavy ties and the
|fp16 gate| inputs DIP actually feeds it.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def C(cuda):
    from soinfer import _C

    return _C


def _check(C, v: np.ndarray, k: int, label: str):
    vd = torch.from_numpy(v).cuda()
    idx, cnt = C.topk_threshold_select(vd, k)
    ref = O.topk_rule_a(v, k)
    assert int(cnt.item()) == ref.size, f"{label}: count {int(cnt.item())} != {ref.size}"
    assert np.array_equal(idx.cpu().numpy()[: ref.size], ref), f"{label}: indices differ from rule A"
    return idx


def test_golden_cases(C):
    for c in json.loads((GOLDEN / "topk_rule_a_cases.json").read_text()):
        idx = _check(C, np.array(c["v"], np.float32), c["k"], c["why"])
        assert idx.tolist() == c["rule_a"], c["why"]


@pytest.mark.parametrize("n,k", [(11008, 5504), (17408, 8704), (1024, 1), (1024, 1024), (4096, 1), (6144, 3072),
                                 (1, 1), (100, 37), (1025, 513), (40000, 20000), (70000, 1234)])
def test_matches_rule_a_and_torch_topk_on_distinct_values(C, n, k):
    g = torch.Generator().manual_seed(n + k)
    v = (torch.rand(n, generator=g) * 10.0).numpy()
    idx = _check(C, v, k, f"n={n} k={k}")
    assert set(idx.tolist()) == set(torch.topk(torch.from_numpy(v), k).indices.tolist())


@pytest.mark.parametrize("k", [768, 1536, 3072])
@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_fp16_gate_magnitudes_with_ties(C, k, seed):
    # |gate| of a Qwen3-1.7B-shaped gate_proj: fp16-rounded values, boundary ties are common
    g = torch.Generator().manual_seed(100 + seed)
    gate = (torch.randn(6144, generator=g) * 0.9).half()
    v = gate.float().abs().numpy()
    _check(C, v, k, f"fp16 gates seed={seed} k={k}")


def _special(n: int, seed: int, kind: str) -> np.ndarray:
    g = np.random.default_rng(seed)
    v = g.uniform(0.0, 5.0, n).astype(np.float32)
    if kind == "nan":
        v[g.choice(n, n // 10, replace=False)] = np.nan
    elif kind == "mostly_nan":  # fewer valid values than k: every bisection decision is "no", tau = 0
        v[g.choice(n, n - n // 20, replace=False)] = np.nan
    elif kind == "signed":  # negatives, -0.0 and +0.0 next to positives (abs_g is unchecked in the reference)
        v = g.uniform(-5.0, 5.0, n).astype(np.float32)
        v[g.choice(n, 64, replace=False)] = -0.0
        v[g.choice(n, 64, replace=False)] = 0.0
    elif kind == "inf":
        v[g.choice(n, 40, replace=False)] = np.inf
        v[g.choice(n, 40, replace=False)] = -np.inf
    elif kind == "tiny":  # zeros and subnormals only
        v = (g.integers(0, 50, n) * np.float32(1e-45)).astype(np.float32)
    elif kind == "equal":
        v[:] = np.float32(0.3)
    return v


@pytest.mark.parametrize("kind", ["nan", "mostly_nan", "signed", "inf", "tiny", "equal"])
@pytest.mark.parametrize("n,k", [(6144, 3072), (6144, 1), (6144, 6144), (16384, 777), (300, 30), (20000, 30)])
def test_special_values_match_rule_a(C, kind, n, k):
    """NaN (never counted), negatives and signed zeros, infinities, subnormals and all-equal inputs: the indices
    and count equal the rule-A oracle's on the same fp32 array (n up to 16384 takes the radix-select kernel,
    20000 the bisection-histogram kernel)."""
    _check(C, _special(n, n + k, kind), k, f"{kind} n={n} k={k}")


@pytest.mark.parametrize("kind", ["nan", "mostly_nan", "inf", "tiny", "equal"])
@pytest.mark.parametrize("k", [1, 768, 3072, 6144])
def test_f16abs_special_values_equal_fp32_abs(C, kind, k):
    """The binary16-gate form (two radix passes) equals the fp32 form on gate.float().abs() for the same gates."""
    v = _special(6144, k, kind)
    sign = np.where(np.random.default_rng(k).random(6144) < 0.5, -1.0, 1.0).astype(np.float32)
    gate = torch.from_numpy(v * sign).half().cuda()
    idx_ref, cnt_ref = C.topk_threshold_select(gate.float().abs(), k)
    idx = torch.zeros(k, dtype=torch.int32, device="cuda")
    cnt = torch.zeros(1, dtype=torch.int32, device="cuda")
    C.topk_threshold_select_f16abs_into(gate, k, idx, cnt)
    n = int(cnt_ref.item())
    assert int(cnt.item()) == n
    assert torch.equal(idx[:n], idx_ref[:n])
    _check(C, gate.float().abs().cpu().numpy(), k, f"f16 {kind} k={k}")


def test_heavy_ties(C):
    g = torch.Generator().manual_seed(1)
    v = torch.randint(0, 10, (8192,), generator=g).float().numpy()
    idx = _check(C, v, 2048, "10 distinct values")
    assert len(set(idx.tolist())) == 2048


def test_bit_identical_across_repeated_calls(C):
    g = torch.Generator().manual_seed(4)
    v = (torch.rand(6144, generator=g) * 10).cuda()
    first = C.topk_threshold_select(v, 3072)[0]
    for _ in range(9):
        assert torch.equal(first, C.topk_threshold_select(v, 3072)[0])


def test_ops_wrapper_returns_indices_only(cuda):
    import soinfer.ops as ops

    v = torch.rand(1000, device="cuda")
    idx = ops.topk_threshold_select(v, 10)
    assert idx.shape == (10,) and idx.dtype == torch.int32


def test_rejects_bad_arguments(cuda):
    import soinfer.ops as ops

    v = torch.rand(1024, device="cuda")
    with pytest.raises(RuntimeError):
        ops.topk_threshold_select(v, 0)
    with pytest.raises(RuntimeError):
        ops.topk_threshold_select(v, 1025)
    with pytest.raises(RuntimeError):
        ops.topk_threshold_select(torch.rand(4, 256, device="cuda"), 10)
    with pytest.raises(RuntimeError):
        ops.topk_threshold_select(v.double(), 10)
