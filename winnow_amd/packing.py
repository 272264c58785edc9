"""Exact bit packing of TurboQuant codes, run on the GPU.

Same names, layout and errors as ``turboquant_kv/packing.py``: LSB-first within
a code, codes in order along the last axis, a code may straddle a byte
(``packing.py:14-17``); ``SUPPORTED = (2, 3, 4, 5, 6, 8)``; ``packed_bytes``
raises ``ValueError`` when ``head_dim * bit_width`` is not a multiple of 8.
``pack``/``unpack`` run the ``wn_pack``/``wn_unpack`` HIP kernels; tensors that
are not on a HIP device are rejected (there is no host implementation).
"""
from __future__ import annotations

import torch

from winnow_amd import _lib

SUPPORTED = (2, 3, 4, 5, 6, 8)


class UnsupportedDevice(RuntimeError):
    """The operand is not on a HIP device; this package has no host fallback."""


def packed_bytes(head_dim: int, bit_width: int) -> int:
    """Bytes for one ``head_dim`` vector of ``bit_width``-bit codes (packing.py:27-34)."""
    total_bits = head_dim * bit_width
    if total_bits % 8 != 0:
        raise ValueError(f"head_dim*bit_width must be a multiple of 8, got "
                         f"{head_dim}*{bit_width}={total_bits}")
    return total_bits // 8


def _require_hip(t: torch.Tensor, what: str) -> None:
    if not _lib.is_hip(t):
        raise UnsupportedDevice(f"{what}: tensor on {t.device}, a HIP device is required")


@torch.no_grad()
def pack(idx: torch.Tensor, bit_width: int) -> torch.Tensor:
    """(..., D) uint8 codes -> (..., D*bit_width/8) uint8 (packing.py:37-64)."""
    _require_hip(idx, "pack")
    if idx.dtype != torch.uint8:
        raise TypeError(f"pack: codes must be uint8, got {idx.dtype}")
    if bit_width not in SUPPORTED:
        raise ValueError(f"bit_width {bit_width} not in {SUPPORTED}")
    D = idx.shape[-1]
    nb = packed_bytes(D, bit_width)
    if bit_width == 8:
        return idx.contiguous()
    src = idx.contiguous()
    out = torch.empty(*idx.shape[:-1], nb, dtype=torch.uint8, device=idx.device)
    rows = src.numel() // D if D else 0
    with torch.cuda.device(idx.device):
        _lib.call("wn_pack", _lib.ptr(src), rows, D, bit_width, _lib.ptr(out), _lib.stream_of(idx.device))
    return out


@torch.no_grad()
def unpack(packed: torch.Tensor, bit_width: int, head_dim: int) -> torch.Tensor:
    """(..., D*bit_width/8) uint8 -> (..., D) uint8 codes (packing.py:67-89)."""
    _require_hip(packed, "unpack")
    if bit_width == 8:
        return packed
    nb = packed_bytes(head_dim, bit_width)
    if packed.shape[-1] != nb:
        raise ValueError(f"unpack: last dim {packed.shape[-1]} != {nb} bytes for D={head_dim}, bw={bit_width}")
    src = packed.contiguous()
    out = torch.empty(*packed.shape[:-1], head_dim, dtype=torch.uint8, device=packed.device)
    rows = src.numel() // nb if nb else 0
    with torch.cuda.device(packed.device):
        _lib.call("wn_unpack", _lib.ptr(src), rows, head_dim, bit_width, _lib.ptr(out),
                  _lib.stream_of(packed.device))
    return out
