"""INT4 / INT8 packing -- the byte layout every INT4 kernel reads.

INT4: eight signed 4-bit values v0..v7 (consecutive along K) share one
little-endian 32-bit word in AWQ order: nibble i holds v[AWQ_ORDER[i]] with
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7), i.e.

    byte0 = v0 | v2<<4   byte1 = v4 | v6<<4   byte2 = v1 | v3<<4   byte3 = v5 | v7<<4

(reference csrc/include/layout.h:19-45, python/soinfer/quant/pack.py:14-69).
A row of K values occupies ceil(K/8)*4 bytes; a ragged tail is zero-padded.
INT8 is stored unpacked (one signed byte per value).
"""
from __future__ import annotations

import torch

GROUP = 8
AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)
# logical position j of a word -> (byte, shift) holding it
_BYTE_OF = tuple(AWQ_ORDER.index(j) // 2 for j in range(GROUP))
_SHIFT_OF = tuple(4 * (AWQ_ORDER.index(j) % 2) for j in range(GROUP))


def pack_int8(q: torch.Tensor) -> tuple[torch.Tensor, int]:
    if q.dtype != torch.int8:
        raise ValueError(f"pack_int8 expects int8, got {q.dtype}")
    return q.clone(), q.shape[-1]


def unpack_int8(packed: torch.Tensor, orig_k: int) -> torch.Tensor:
    if packed.dtype != torch.int8:
        raise ValueError(f"unpack_int8 expects int8, got {packed.dtype}")
    return packed[..., :orig_k].clone()


def pack_int4(q: torch.Tensor) -> tuple[torch.Tensor, int]:
    """q: int8 in [-8, 7], shape [..., K] -> (uint8 [..., ceil(K/8)*4], K)."""
    if q.dtype != torch.int8:
        raise ValueError(f"pack_int4 expects int8, got {q.dtype}")
    K = q.shape[-1]
    words = -(-K // GROUP)
    if words * GROUP != K:
        q = torch.nn.functional.pad(q, (0, words * GROUP - K))
    nib = (q.to(torch.int32) & 0xF).reshape(*q.shape[:-1], words, GROUP)
    out = torch.zeros(*q.shape[:-1], words, 4, dtype=torch.int32, device=q.device)
    for j in range(GROUP):
        out[..., _BYTE_OF[j]] |= nib[..., j] << _SHIFT_OF[j]
    return out.to(torch.uint8).reshape(*q.shape[:-1], words * 4), K


def unpack_int4(packed: torch.Tensor, orig_k: int) -> torch.Tensor:
    """Inverse of pack_int4: uint8 [..., ceil(K/8)*4] -> int8 [..., orig_k], sign-extended."""
    if packed.dtype != torch.uint8:
        raise ValueError(f"unpack_int4 expects uint8, got {packed.dtype}")
    words = packed.shape[-1] // 4
    b = packed.to(torch.int32).reshape(*packed.shape[:-1], words, 4)
    vals = torch.stack([(b[..., _BYTE_OF[j]] >> _SHIFT_OF[j]) & 0xF for j in range(GROUP)], dim=-1)
    vals = vals - ((vals & 0x8) << 1)  # two's complement sign extension of a nibble
    return vals.reshape(*packed.shape[:-1], words * GROUP)[..., :orig_k].to(torch.int8)
