"""The grid-barrier measurement kernel (csrc/grid_sync.hip): every round's exchange reads the other workgroups'
words of that round (no mismatch), no bounded wait gives up, stamps are written, for small and ragged grids
(P not a multiple of the 8 counters) up to 1024 workgroups, fenced and coherent forms; repeated calls on one
workspace continue its generation count; a grid larger than the GPU holds at once is rejected before launch."""
import pytest
import torch

pytestmark = pytest.mark.gpu
SYNC_BYTES = 4608


@pytest.fixture(scope="module")
def C(cuda):
    from soinfer import _C

    return _C


def _run(C, fenced, P, rounds, ws=None):
    if ws is None:
        ws = torch.zeros(C.grid_barrier_bench_workspace_bytes(P), dtype=torch.uint8, device="cuda")
    print(f"grid barrier: fenced={fenced} P={P} rounds={rounds}", flush=True)
    C.grid_barrier_bench(fenced, P, rounds, ws)
    torch.cuda.synchronize()
    err = ws[:SYNC_BYTES].view(torch.int32)[1088:1090].tolist()
    stamps = ws[SYNC_BYTES:SYNC_BYTES + 16 * P].view(torch.int64).view(P, 2)
    return ws, err, stamps


@pytest.mark.parametrize("fenced", [False, True])
@pytest.mark.parametrize("P", [1, 7, 8, 13, 256, 1024])
def test_grid_barrier_exchanges_and_drains(C, fenced, P):
    assert C.grid_barrier_max_workgroups() >= 1024
    ws, err, stamps = _run(C, fenced, P, 50)
    assert err == [0, 0], f"timeout flag / mismatched words: {err}"
    assert bool((stamps[:, 1] >= stamps[:, 0]).all()) and bool((stamps[:, 0] > 0).all())
    # the same workspace again: the counters and generation continue from where the last call left them
    ws, err, _ = _run(C, fenced, P, 33, ws)
    assert err == [0, 0]


def test_grid_barrier_rejections(C):
    big = C.grid_barrier_max_workgroups() + 1
    ws = torch.zeros(C.grid_barrier_bench_workspace_bytes(big), dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="at most"):
        C.grid_barrier_bench(False, big, 10, ws)
    small = torch.zeros(100, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        C.grid_barrier_bench(False, 256, 10, small)
    with pytest.raises(RuntimeError, match="rounds"):
        C.grid_barrier_bench(False, 256, 0, torch.zeros(C.grid_barrier_bench_workspace_bytes(256),
                                                        dtype=torch.uint8, device="cuda"))
