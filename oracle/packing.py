"""Oracle: exact LSB-first bit packing (numpy) -- test infrastructure only.

Follows ``turboquant_kv/packing.py:14-17`` (layout: LSB-first within an index,
indices in order along the last axis, an index may straddle a byte) and
``packing.py:24-34`` (supported widths, bytes per vector).  The implementation is
independent of the reference's: it goes through ``numpy.packbits`` with
``bitorder="little"`` instead of an int16 weighted sum.

Pinned by: hand-built known-answer vectors (3-bit and 6-bit straddles, nibble
order), ``packed_bytes`` KATs from ``test_packing.py:43-44``, the round trip of
``test_packing.py:20-40``, and brute force over every value of tiny vectors
(``tests/test_oracle_packing.py``).
"""
from __future__ import annotations

import numpy as np

SUPPORTED = (2, 3, 4, 5, 6, 8)          # packing.py:24


def packed_bytes(head_dim: int, bit_width: int) -> int:
    """Bytes for one ``head_dim`` vector of ``bit_width``-bit indices (packing.py:27-34)."""
    total = head_dim * bit_width
    if total % 8:
        raise ValueError(f"head_dim*bit_width must be a multiple of 8, got {head_dim}*{bit_width}={total}")
    return total // 8


def pack(idx: np.ndarray, bit_width: int) -> np.ndarray:
    """(..., D) uint8 codes -> (..., D*bw/8) uint8, LSB-first (packing.py:37-64)."""
    idx = np.asarray(idx, dtype=np.uint8)
    D = idx.shape[-1]
    nb = packed_bytes(D, bit_width)
    if bit_width == 8:
        return idx.copy()
    flat = idx.reshape(-1, D)
    sh = np.arange(bit_width, dtype=np.uint8)
    bits = ((flat[:, :, None] >> sh) & 1).reshape(flat.shape[0], D * bit_width)
    out = np.packbits(bits, axis=-1, bitorder="little")
    assert out.shape[-1] == nb
    return out.reshape(*idx.shape[:-1], nb)


def unpack(packed: np.ndarray, bit_width: int, head_dim: int) -> np.ndarray:
    """(..., NB) uint8 -> (..., D) uint8 codes (packing.py:67-89)."""
    packed = np.asarray(packed, dtype=np.uint8)
    if bit_width == 8:
        return packed.copy()
    nb = packed.shape[-1]
    flat = packed.reshape(-1, nb)
    bits = np.unpackbits(flat, axis=-1, bitorder="little")[:, :head_dim * bit_width]
    bits = bits.reshape(-1, head_dim, bit_width).astype(np.uint16)
    w = (1 << np.arange(bit_width, dtype=np.uint16))
    out = (bits * w).sum(-1).astype(np.uint8)
    return out.reshape(*packed.shape[:-1], head_dim)
