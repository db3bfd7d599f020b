"""Shared helpers for the parity tests: seeded problem builders and the tolerance rule.

Tolerance for floating-point outputs (GEMV, sparse accumulate, attention): the
HIP output (binary16) is compared with the oracle's binary64 result `ref`:
  normalized:  max|out - ref| <= 1e-3 * max|ref|
  per element: |out - ref|   <= 1e-3 * |ref| + 1e-5 * max|ref|
Binary16 rounding alone contributes <= 2^-11 |ref| (4.9e-4). The INT4 GEMVs
accumulate with v_dot2_f32_f16, whose rounding is not round-to-nearest-even:
over K = 6144 their fp32 error reaches ~2e-5 * max|ref| at cancelling outputs
(tests/test_gemv_gpu.py::test_int4_gemv_accumulation_error_bound measures it),
so comparisons of long-K dense GEMVs pass floor=5e-5; elsewhere the 1e-5 floor
holds. Index, byte and descriptor outputs are compared exactly.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as O

TOL = 1e-3
FLOOR = 1e-5


def assert_close(out: torch.Tensor, ref: np.ndarray, label: str = "", tol: float = TOL, floor: float = FLOOR) -> None:
    a = out.detach().float().cpu().numpy().astype(np.float64).reshape(ref.shape)
    assert np.all(np.isfinite(a)), f"{label}: non-finite output"
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = np.abs(a - ref)
    if ref.size == 0:
        return
    assert err.max() <= tol * scale + 1e-30, f"{label}: normalized error {err.max() / max(scale, 1e-30):.3e} > {tol}"
    bound = tol * np.abs(ref) + floor * scale
    bad = np.flatnonzero(err > bound)
    assert bad.size == 0, (f"{label}: {bad.size} elements beyond tolerance, first at {bad[0]}: "
                           f"out={a.flat[bad[0]]} ref={ref.flat[bad[0]]}")


def int4_problem(N: int, K: int, gs: int, seed: int, std: float = 0.02, device="cuda"):
    """W ~ N(0, std) quantized by the oracle (symmetric group INT4), x ~ N(0,1) fp16 of the padded K.
    Returns dict with numpy and device tensors."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * std
    q, s = O.quantize_group(w.numpy(), gs)
    Kp = q.shape[1]
    Wq = O.pack_int4(q)
    x = torch.randn(Kp, generator=g).half()
    return {
        "Wq": Wq, "s": s, "x": x.numpy(), "K": Kp, "q": q, "gs": gs,
        "Wq_d": torch.from_numpy(Wq).to(device), "s_d": torch.from_numpy(s).to(device), "x_d": x.to(device),
    }


def f16(t) -> np.ndarray:
    return np.asarray(t, dtype=np.float16)
