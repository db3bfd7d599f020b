"""The allocation-free sparse accumulate (soi_gemv_w4a16_sparse_accumulate_noalloc), called through the C ABI.

Its workspace is a fixed per-GPU device array, so consecutive calls share it: each call must equal the
workspace form (soi_gemv_w4a16_sparse_accumulate, through soinfer.ops) bit for bit, whatever the previous call
left behind -- a large call, then a smaller one (smaller H and k), then the large one again, then another
shape; k = 0 gives zeros; sizes beyond the array are rejected before any launch; and the call replays from a
HIP graph with eager work between replays.
"""
import ctypes as C
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_close, int4_problem
from oracle import oracle as O

pytestmark = pytest.mark.gpu
LIB = Path(__file__).resolve().parent.parent / "sparse-offload-infer_amd" / "soinfer" / "libsoinfer_hip.so"


@pytest.fixture(scope="module")
def lib(cuda):
    import soinfer.ops  # noqa: F401  (loads the same library through the extension)

    L = C.CDLL(str(LIB))
    f = L.soi_gemv_w4a16_sparse_accumulate_noalloc
    f.argtypes = [C.c_void_p] * 4 + [C.c_int64] * 4 + [C.c_void_p]
    f.restype = C.c_int
    L.soi_last_error.restype = C.c_char_p
    L.soi_sparse_accumulate_noalloc_max_scratch_bytes.restype = C.c_size_t
    return L


def _call(lib, W, S, h, y, H, k, gs):
    return lib.soi_gemv_w4a16_sparse_accumulate_noalloc(W.data_ptr(), S.data_ptr(), h.data_ptr(), y.data_ptr(), H, k,
                                                        gs, S.shape[1], torch.cuda.current_stream().cuda_stream)


def _problem(H, k, gs, seed):
    p = int4_problem(k, H, gs, seed=seed)  # k selected rows of down^T, H columns
    h = torch.randn(k, generator=torch.Generator().manual_seed(seed + 100)).half().cuda()
    return p, h


def test_noalloc_equals_workspace_form_on_consecutive_calls(lib):
    import soinfer.ops as ops

    assert lib.soi_sparse_accumulate_noalloc_max_scratch_bytes() == 2 << 20
    # large, then smaller (fewer column slices and rows), then large again, then the 14B shape
    for H, k, gs, seed in [(2048, 3072, 128, 1), (1024, 100, 64, 2), (2048, 3072, 128, 3), (5120, 8704, 128, 4),
                           (256, 40, 32, 5)]:
        p, h = _problem(H, k, gs, seed)
        y = torch.full((H,), float("nan"), dtype=torch.float16, device="cuda")
        assert _call(lib, p["Wq_d"], p["s_d"], h, y, H, k, gs) == 0, lib.soi_last_error()
        want = ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, H, gs)
        assert torch.equal(y, want), f"H={H} k={k}: differs from the workspace form"
        if seed in (2, 5):
            assert_close(y, O.sparse_accumulate_f64(p["Wq"], p["s"], h.cpu().numpy(), H, gs), f"H={H} k={k}")


def test_noalloc_empty_selection_and_size_limit(lib):
    p, h = _problem(2048, 64, 128, 6)
    y = torch.full((2048,), float("nan"), dtype=torch.float16, device="cuda")
    assert _call(lib, p["Wq_d"], p["s_d"], h, y, 2048, 0, 128) == 0
    assert torch.equal(y, torch.zeros_like(y))
    # 60000 rows at H = 2048 need ~313 chunks x 8 KB of partial rows: beyond the 2 MiB array, rejected
    y.fill_(1.0)
    rc = _call(lib, p["Wq_d"], p["s_d"], h, y, 2048, 60000, 128)
    assert rc == 1 and b"scratch" in lib.soi_last_error()
    torch.cuda.synchronize()
    assert bool((y == 1.0).all()), "a rejected call must not launch"


def test_noalloc_replays_from_a_graph(lib):
    import soinfer.ops as ops

    H, k, gs = 2048, 1536, 128
    p, h = _problem(H, k, gs, 7)
    y = torch.zeros(H, dtype=torch.float16, device="cuda")
    assert _call(lib, p["Wq_d"], p["s_d"], h, y, H, k, gs) == 0  # eager first
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert _call(lib, p["Wq_d"], p["s_d"], h, y, H, k, gs) == 0
    torch.cuda.synchronize()
    want = ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, H, gs)
    q, h2 = _problem(1024, 77, 64, 8)
    y2 = torch.zeros(1024, dtype=torch.float16, device="cuda")
    for i in range(3):
        y.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {i}"
        # other eager work, including an eager call that shares the scratch array
        _ = torch.zeros(1 << 20, device="cuda").sum()
        assert _call(lib, q["Wq_d"], q["s_d"], h2, y2, 1024, 77, 64) == 0
        torch.cuda.synchronize()
        assert torch.equal(y2, ops.gemv_w4a16_sparse_accumulate(q["Wq_d"], q["s_d"], h2, 1024, 64))


_FIRST_CALL_UNDER_CAPTURE = r'''
import ctypes as C, sys
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2], sys.argv[3]]
import soinfer.ops as ops
from helpers import int4_problem
L = C.CDLL(sys.argv[4])
f = L.soi_gemv_w4a16_sparse_accumulate_noalloc
f.argtypes = [C.c_void_p] * 4 + [C.c_int64] * 4 + [C.c_void_p]
f.restype = C.c_int
L.soi_last_error.restype = C.c_char_p
H, k, gs = 2048, 1536, 128
p = int4_problem(k, H, gs, seed=9)
h = torch.randn(k, generator=torch.Generator().manual_seed(109)).half().cuda()
y = torch.zeros(H, dtype=torch.float16, device="cuda")
want = ops.gemv_w4a16_sparse_accumulate(p["Wq_d"], p["s_d"], h, H, gs)
torch.cuda.synchronize()
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g, stream=s):
    rc = f(p["Wq_d"].data_ptr(), p["s_d"].data_ptr(), h.data_ptr(), y.data_ptr(), H, k, gs, p["s_d"].shape[1],
           torch.cuda.current_stream().cuda_stream)
if rc != 0:
    print("FIRST CALL FAILED", L.soi_last_error(), flush=True)
    sys.exit(3)
for i in range(3):
    y.zero_()
    g.replay()
    torch.cuda.synchronize()
    if not torch.equal(y, want):
        print("REPLAY DIFFERS", i, flush=True)
        sys.exit(4)
    _ = torch.zeros(1 << 20, device="cuda").sum()
    torch.cuda.synchronize()
print("FIRST-CALL-UNDER-CAPTURE OK", flush=True)
'''


def test_noalloc_first_call_under_capture(lib, tmp_path):
    """In a fresh process the first call on the device (symbol lookup + the counter-clearing kernel) is made
    inside a graph capture; every replay equals the workspace form."""
    import subprocess
    import sys

    root = Path(__file__).resolve().parent.parent
    script = tmp_path / "first_call_under_capture.py"
    script.write_text(_FIRST_CALL_UNDER_CAPTURE)
    print("running the first-call-under-capture child", flush=True)
    r = subprocess.run([sys.executable, str(script), str(root / "sparse-offload-infer_amd"), str(root),
                        str(root / "tests"), str(LIB)], capture_output=True, text=True, timeout=100)
    assert r.returncode == 0 and "FIRST-CALL-UNDER-CAPTURE OK" in r.stdout, (r.returncode, r.stdout[-2000:],
                                                                          r.stderr[-2000:])
