"""Decode attention parity on the GPU (counterpart of tests/test_m5_kernels.py:157-213 in the reference).

HIP split-KV attention vs the oracle's binary64 softmax attention on the same
fp16 q / K / V, within the tolerance rule of tests/helpers.py.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close
from oracle import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(cuda):
    import soinfer.ops as ops

    return ops


def _qkv(NQ, NKV, hd, S, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(NQ, hd, generator=g).half()
    k = torch.randn(NKV, S, hd, generator=g).half()
    v = torch.randn(NKV, S, hd, generator=g).half()
    return q, k, v


@pytest.mark.parametrize("L", [1, 2, 17, 63, 64, 65, 300, 1000, 1024, 1025, 2047, 2048])
def test_qwen_shape_matches_oracle(ops, L):
    q, k, v = _qkv(16, 8, 128, 2048, seed=L)
    ref = O.decode_attention_f64(q.numpy(), k.numpy(), v.numpy(), L)
    out = ops.decode_attention(q.cuda(), k.cuda(), v.cuda(), L)
    assert_close(out, ref, f"attention L={L}")


@pytest.mark.parametrize("NQ,NKV,hd,S,L", [(4, 2, 16, 8, 5), (8, 8, 64, 100, 77), (32, 4, 128, 512, 300),
                                          (16, 16, 256, 64, 64), (6, 3, 24, 40, 33), (2, 1, 100, 20, 20),
                                          (12, 1, 128, 256, 200)])
def test_other_shapes_match_oracle(ops, NQ, NKV, hd, S, L):
    q, k, v = _qkv(NQ, NKV, hd, S, seed=NQ + hd + L)
    ref = O.decode_attention_f64(q.numpy(), k.numpy(), v.numpy(), L)
    out = ops.decode_attention(q.cuda(), k.cuda(), v.cuda(), L)
    assert_close(out, ref, f"attention {NQ}/{NKV}/{hd} L={L}")


@pytest.mark.parametrize("L", [4096, 8191, 16384])
def test_long_context_matches_oracle(ops, L):
    """Past the BASELINE context (2048): more than 8192 timestep rows per launch switch the split target, and
    each split then spans several 8-pass load batches. The host-length form against the binary64 oracle, and
    the device-position form (length read from pos on the device, the engine's form) bit for bit against it."""
    from soinfer import _C

    S = 16384
    q, k, v = _qkv(16, 8, 128, S, seed=L)
    ref = O.decode_attention_f64(q.numpy(), k.numpy(), v.numpy(), L)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    out = ops.decode_attention(qd, kd, vd, L)
    assert_close(out, ref, f"attention L={L}")
    ws = torch.zeros(_C.decode_attention_workspace_bytes(16, 8, 128, S), dtype=torch.uint8, device="cuda")
    pos = torch.tensor([L - 1], dtype=torch.int32, device="cuda")
    at = torch.empty_like(out)
    _C.decode_attention_at(qd, kd, vd, pos, at, ws)
    assert torch.equal(at, out), f"device-position form differs at L={L}"


def test_caller_buffers_form_equals_allocating_form(ops):
    """decode_attention_into (caller out and workspace, reused across calls) == decode_attention, bit for bit, on
    both sides of the split boundary (a split host length combines in a second launch) and for one KV head."""
    from soinfer import _C

    for NQ, NKV, hd, S in ((16, 8, 128, 2048), (8, 1, 128, 4096)):
        q, k, v = _qkv(NQ, NKV, hd, S, seed=S + NKV)
        q, k, v = q.cuda(), k.cuda(), v.cuda()
        ws = torch.full((_C.decode_attention_workspace_bytes(NQ, NKV, hd, S),), 255, dtype=torch.uint8,
                        device="cuda")
        out = torch.empty(NQ, hd, dtype=torch.float16, device="cuda")
        for L in (1, 256, 257, 1000, S // 2 + 1, S):
            _C.decode_attention_into(q, k, v, L, out, ws)
            assert torch.equal(out, ops.decode_attention(q, k, v, L)), f"NQ={NQ} NKV={NKV} L={L}"


def test_large_scores_stable(ops):
    q, k, v = _qkv(16, 8, 128, 256, seed=3)
    q = (q.float() * 8).half()
    ref = O.decode_attention_f64(q.numpy(), k.numpy(), v.numpy(), 256)
    out = ops.decode_attention(q.cuda(), k.cuda(), v.cuda(), 256)
    assert_close(out, ref, "attention large scores")


def test_deterministic(ops):
    q, k, v = _qkv(16, 8, 128, 2048, seed=4)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    first = ops.decode_attention(qd, kd, vd, 2048)
    for _ in range(5):
        assert torch.equal(first, ops.decode_attention(qd, kd, vd, 2048))


def test_rejections(ops):
    q = torch.randn(15, 128, device="cuda").half()
    k = torch.randn(8, 64, 128, device="cuda").half()
    with pytest.raises(RuntimeError):
        ops.decode_attention(q, k, k, 1)  # 15 query heads over 8 KV heads
    q16 = torch.randn(16, 128, device="cuda").half()
    with pytest.raises(RuntimeError):
        ops.decode_attention(q16, k, k, 0)
    with pytest.raises(RuntimeError):
        ops.decode_attention(q16, k, k, 65)
