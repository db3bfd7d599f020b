"""Writes the golden fixtures in this directory.

The fixtures are the known-answer cases the reference's own tests hold for
the hot path, restated as data (inputs and expected outputs):
  awq_pack_kat.json          tests/test_quant_roundtrip.py:41-59 (byte layout of
                             csrc/include/layout.h:31-34 for v = [1,-2,3,-4,5,-6,7,-7])
  dip_descriptor_cases.json  tests/test_m8_fused_gemv.py:87-130 (hit/miss cases)
  static_policy_cases.json   tests/test_hot_cache.py:16-37 (hot-set choice, hit counts)
  topk_rule_a_cases.json     small top-k cases whose rule-A answers follow from the
                             threshold rule of csrc/kernels/topk_select.cu:19-95 by
                             hand (see the `why` field of each case)
Expected outputs are computed here from the closed forms, not by running the
reference. Run: python tests/golden/make_golden.py
"""
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def tau_closed_form(v, k):
    f = np.float32
    vs = sorted((f(x) for x in v), reverse=True)
    vk = vs[k - 1]
    lo, hi = f(0.0), f(max(f(0.0), vs[0]) + f(1e-3))
    for _ in range(24):
        mid = f(f(0.5) * f(lo + hi))
        if mid <= vk:
            lo = mid
        else:
            hi = mid
    return lo


def awq_bytes(v):
    n = [x & 0xF for x in v]
    return [n[0] | n[2] << 4, n[4] | n[6] << 4, n[1] | n[3] << 4, n[5] | n[7] << 4]


def main():
    v = [1, -2, 3, -4, 5, -6, 7, -7]
    (HERE / "awq_pack_kat.json").write_text(json.dumps({
        "values": v, "bytes": awq_bytes(v),
        "ragged": {"K": 17, "packed_bytes_per_row": 12},
    }, indent=1))

    desc_cases = [
        {"name": "hits_and_misses", "num_channels": 32, "cached": [3, 7, 15],
         "selected": [1, 3, 5, 7, 9, 15],
         "expect_miss_count": 3, "expect_miss_channels": [1, 5, 9],
         "expect_desc": [[True, 0], [False, 0], [True, 1], [False, 1], [True, 2], [False, 2]]},
        {"name": "all_hits", "num_channels": 16, "cached": list(range(16)), "selected": [2, 5, 9],
         "expect_miss_count": 0, "expect_miss_channels": [],
         "expect_desc": [[False, 2], [False, 5], [False, 9]]},
        {"name": "all_misses", "num_channels": 16, "cached": [], "selected": [0, 4, 8, 12],
         "expect_miss_count": 4, "expect_miss_channels": [0, 4, 8, 12],
         "expect_desc": [[True, 0], [True, 1], [True, 2], [True, 3]]},
    ]
    (HERE / "dip_descriptor_cases.json").write_text(json.dumps(desc_cases, indent=1))

    policy_cases = [
        {"frequencies": [5, 5, 5, 1], "cache_size": 2, "hot_set": [0, 1],
         "trace": [[0], [1], [2], [3], [0, 1, 2]], "hits": 4, "total": 7},
        {"frequencies": [3, 1], "cache_size": 10, "hot_set": [0, 1], "effective_cache_size": 2,
         "trace": [], "hits": 0, "total": 0},
    ]
    (HERE / "static_policy_cases.json").write_text(json.dumps(policy_cases, indent=1))

    # Rule A answers are computed from the closed form of the bisection: the
    # reference's step test count(v >= mid) >= k holds exactly when
    # mid <= v_(k) (the k-th largest value), so tau is obtained by replaying
    # the 24 binary32 steps against v_(k) alone -- no counting.
    topk_cases = []
    for v, k, why in [
        ([0.0, 3.0, 1.0, 2.0], 2, "distinct values"),
        ([1.0, 1.0, 1.0, 1.0, 0.5], 2, "4-way tie at the k-th value: first tied indices in ascending order"),
        ([0.99999994, 1.0, 3.0], 2, "v_(2)=1.0 but tau lands one ulp below it, so 0.99999994 passes and the "
                                    "ascending scan stops before the maximum 3.0 (rule A != exact top-k)"),
        ([0.99999994, 1.0, 2.0], 2, "same shape with max 2.0: tau lands exactly on 1.0"),
        ([0.0, 0.0, 0.0], 1, "all zero: tau = 0 and every index qualifies"),
    ]:
        tau = tau_closed_form(v, k)
        rule_a = [i for i, x in enumerate(np.float32(v)) if x >= tau][:k]
        order = sorted(range(len(v)), key=lambda i: (-np.float32(v[i]), i))[:k]
        topk_cases.append({"v": v, "k": k, "tau": float(tau), "rule_a": rule_a, "rule_b": sorted(order),
                           "why": why})
    (HERE / "topk_rule_a_cases.json").write_text(json.dumps(topk_cases, indent=1))


if __name__ == "__main__":
    main()
