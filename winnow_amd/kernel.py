"""Fused TurboQuant dequantization: a drop-in for ``turboquant_kv/kernel.py``'s ``tq_dequant``
(``kernel.py:78-115``) and the CUDA extension's ``tq_dequant_cuda`` (``csrc/tq_dequant.cu:186-215``).

``tq_dequant(packed, norms, centroids, Pi, bit_width, head_dim)`` unpacks the codes,
gathers their centroids, applies the inverse rotation ``y @ Pi`` and the norm, and
writes the result once in ``out``'s dtype (bf16 by default) -- one HIP kernel
(``wn_tq_dequant``) on the matrix cores. Like the reference it reads a
``(..., MAXLEN, NB)`` cache buffer sliced to its first ``L`` positions in place
(``kernel.py:46-51``). ``allow_tf32`` keeps its meaning: False (the default) runs the
rotation at near-fp32 accuracy, True trades it for speed (one fp16 product per term,
2^-11 relative, the class of tf32). The other schedule keywords (``block_n``,
``num_warps``, ``num_stages``) are accepted and ignored.
"""
from __future__ import annotations

import torch

from winnow_amd import _lib
from winnow_amd.packing import SUPPORTED, UnsupportedDevice, packed_bytes


def _plane_rows(t: torch.Tensor, L: int) -> int:
    """Rows between consecutive (..., L) planes of a (..., rows, cols) view whose leading dims collapse."""
    if t.dim() < 3:
        return L
    step = t.stride(-3) // t.stride(-2)
    lead = t.shape[:-2]
    # the leading dims must form one evenly strided sequence of planes
    expect = t.stride(-3)
    for i in range(len(lead) - 2, -1, -1):
        expect *= t.shape[i + 1]
        if t.shape[i] > 1 and t.stride(i) != expect:
            raise ValueError("tq_dequant: leading dims of the cache view are not evenly strided")
    return step


@torch.no_grad()
def tq_dequant(packed: torch.Tensor, norms: torch.Tensor, centroids: torch.Tensor, Pi: torch.Tensor,
               bit_width: int, head_dim: int, out: torch.Tensor | None = None, block_n: int = 64,
               allow_tf32: bool = False, num_warps: int = 4, num_stages: int = 2) -> torch.Tensor:
    """``packed`` (..., NB) uint8 and ``norms`` (...) -> (..., head_dim) in ``out``'s dtype (kernel.py:78-115)."""
    del block_n, num_warps, num_stages  # schedule keywords of the Triton kernel
    if not _lib.is_hip(packed):
        raise UnsupportedDevice(f"tq_dequant: tensor on {packed.device}, a HIP device is required")
    if bit_width not in SUPPORTED:
        raise ValueError(f"bit_width {bit_width} not in {SUPPORTED}")
    NB = packed_bytes(head_dim, bit_width)
    if packed.dtype != torch.uint8 or packed.shape[-1] != NB:
        raise ValueError(f"tq_dequant: packed must be uint8 (..., {NB}), got {tuple(packed.shape)} {packed.dtype}")
    if tuple(norms.shape) != tuple(packed.shape[:-1]):
        raise ValueError(f"tq_dequant: norms {tuple(norms.shape)} do not match packed {tuple(packed.shape)}")
    if centroids.dtype != torch.float32 or Pi.dtype != torch.float32:
        raise ValueError("tq_dequant: centroids and Pi must be fp32")
    if centroids.numel() != 2 ** bit_width or tuple(Pi.shape) != (head_dim, head_dim):
        raise ValueError("tq_dequant: centroids must have 2**bit_width entries and Pi (head_dim, head_dim)")
    lead = tuple(packed.shape[:-1])
    if out is None:
        out = torch.empty(*lead, head_dim, dtype=torch.bfloat16, device=packed.device)
    if tuple(out.shape) != lead + (head_dim,):
        raise ValueError(f"tq_dequant: out {tuple(out.shape)} != {lead + (head_dim,)}")
    N = 1
    for s in lead:
        N *= s
    if N == 0:
        return out
    if packed.dim() == 1:
        packed, norms = packed[None], norms[None]
    L = packed.shape[-2]
    if packed.stride(-1) != 1 or packed.stride(-2) != NB:
        packed = packed.contiguous()
    if norms.half().dtype != norms.dtype or norms.stride(-1) != 1:
        norms = norms.half().contiguous()
    prow = _plane_rows(packed, L)
    if norms.dim() >= 2 and norms.shape[-2] > 1 and norms.stride(-2) != prow:
        norms = norms.contiguous()
        if prow != L:  # the norms must follow the packed rows' plane stride
            packed = packed.contiguous()
            prow = L
    dst = out if (out.is_contiguous() and out.dtype in _lib.DTYPE_CODE) else \
        torch.empty(out.shape, dtype=torch.float32, device=out.device)
    with torch.cuda.device(packed.device):
        _lib.call("wn_tq_dequant", _lib.ptr(packed), _lib.ptr(norms), N // L, L, prow,
                  _lib.ptr(centroids.contiguous()), _lib.ptr(Pi.contiguous()), bit_width, head_dim,
                  _lib.ptr(dst), _lib.DTYPE_CODE[dst.dtype], 1 if allow_tf32 else 0, _lib.stream_of(packed.device))
    if dst is not out:
        out.copy_(dst)
    return out
