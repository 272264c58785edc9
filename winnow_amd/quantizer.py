"""TurboQuant MSE quantizer: seeded rotation + per-coordinate Lloyd-Max codebook.

Drop-in for ``TurboQuantMSE`` / ``_get_quantizer`` of ``turboquant_kv/cache.py``
(lines 62-148). The constants are built on the host exactly as the reference
builds them -- ``torch.randn`` on a CPU generator seeded with
``rotation_seed``, ``torch.linalg.qr`` and a sign fix for ``Pi`` (cache.py:92-97);
a float64 Lloyd-Max iteration with ``scipy.stats.norm`` for the codebook
(cache.py:62-82, 98-103) -- and then live on the device. ``quantize`` and
``dequantize_into`` run the ``wn_quantize`` / ``wn_dequantize`` HIP kernels.
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch
from scipy.stats import norm as _norm

from winnow_amd import _lib
from winnow_amd.packing import SUPPORTED, UnsupportedDevice


def lloyd_max_gaussian(levels: int, sigma: float = 1.0, iters: int = 200, tol: float = 1e-12):
    """Centroids and (+-inf terminated) boundaries of the Lloyd-Max quantizer of N(0, sigma^2).

    Start from ``linspace(-3 sigma, 3 sigma)``; each step moves every centroid to
    the conditional mean of its cell; stop after ``iters`` steps or once no
    centroid moves by ``tol`` (cache.py:62-82).
    """
    c = np.linspace(-3 * sigma, 3 * sigma, levels)
    for _ in range(iters):
        edges = np.concatenate(([-np.inf], (c[:-1] + c[1:]) / 2.0, [np.inf]))
        nxt = np.empty_like(c)
        for i in range(levels):
            lo, hi = edges[i] / sigma, edges[i + 1] / sigma
            mass = _norm.cdf(hi) - _norm.cdf(lo)
            nxt[i] = c[i] if mass < 1e-300 else sigma * (_norm.pdf(lo) - _norm.pdf(hi)) / mass
        moved = np.max(np.abs(nxt - c))
        c = nxt
        if moved < tol:
            break
    return c, np.concatenate(([-np.inf], (c[:-1] + c[1:]) / 2.0, [np.inf]))


_CANONICAL = Path(__file__).resolve().parent / "rotations_d128.npz"


def seeded_rotation(head_dim: int, seed: int) -> torch.Tensor:
    """Q of the QR factorisation of a seeded Gaussian matrix, columns signed so R has a
    positive diagonal (cache.py:92-97). Built on the host, fp32.

    The fp32 QR's bits depend on the host's CPU and on how many threads LAPACK splits
    it over (the reference leaves both free), and every code depends on them. The
    standard rotations, head_dim 128 at seeds 42 and 43 (``quantizers_for``'s and the
    reference tests'), are therefore the reference's own single-threaded bits, shipped
    in ``rotations_d128.npz``: every host encodes and decodes with the same Pi. Other
    shapes run the QR here on one thread.
    """
    if head_dim == 128 and seed in (42, 43):
        with np.load(_CANONICAL) as f:
            return torch.from_numpy(np.array(f[f"pi_{seed}"], dtype=np.float32)).contiguous()
    gen = torch.Generator(device="cpu").manual_seed(seed)
    g = torch.randn(head_dim, head_dim, generator=gen, dtype=torch.float32)
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        q, r = torch.linalg.qr(g)
    finally:
        torch.set_num_threads(threads)
    signs = torch.sign(torch.diag(r))
    signs[signs == 0] = 1.0
    return (q * signs.unsqueeze(0)).contiguous()


class TurboQuantMSE:
    """Fixed random rotation + per-coordinate Lloyd-Max scalar quantizer (cache.py:85-131)."""

    def __init__(self, bit_width: int, head_dim: int, device="cuda", rotation_seed: int = 42):
        if bit_width not in SUPPORTED:
            raise ValueError(f"bit_width {bit_width} not in {SUPPORTED}")
        device = torch.device(device)
        self.Pi = seeded_rotation(head_dim, rotation_seed).to(device).contiguous()
        c, b = lloyd_max_gaussian(2 ** bit_width, sigma=1.0 / math.sqrt(head_dim))
        self.centroids = torch.tensor(c, dtype=torch.float32, device=device).contiguous()
        self.boundaries = torch.tensor(b[1:-1], dtype=torch.float32, device=device).contiguous()
        self.bit_width = bit_width
        self.head_dim = head_dim
        self.device = device
        self.rotation_seed = rotation_seed

    def _require(self, t: torch.Tensor, what: str) -> None:
        if not _lib.is_hip(t):
            raise UnsupportedDevice(f"{what}: tensor on {t.device}, a HIP device is required")
        if t.device != self.Pi.device:
            raise ValueError(f"{what}: tensor on {t.device}, quantizer on {self.Pi.device}")

    @torch.no_grad()
    def quantize(self, x: torch.Tensor):
        """(..., D) -> (uint8 codes (..., D), fp32 norms (...)) (cache.py:108-115)."""
        self._require(x, "quantize")
        D = self.head_dim
        if x.shape[-1] != D:
            raise ValueError(f"quantize: last dim {x.shape[-1]} != head_dim {D}")
        if x.dtype not in _lib.DTYPE_CODE:
            x = x.float()
        flat = x.reshape(-1, D)
        if flat.stride(-1) != 1:
            flat = flat.contiguous()
        rows = flat.shape[0]
        idx = torch.empty(rows, D, dtype=torch.uint8, device=x.device)
        norms = torch.empty(rows, dtype=torch.float32, device=x.device)
        with torch.cuda.device(x.device):
            _lib.call("wn_quantize", _lib.ptr(flat), _lib.DTYPE_CODE[flat.dtype], rows,
                      flat.stride(0) if rows else D, _lib.ptr(self.Pi), _lib.ptr(self.boundaries),
                      self.bit_width, D, _lib.ptr(idx), _lib.ptr(norms), _lib.stream_of(x.device))
        return idx.view(x.shape), norms.view(x.shape[:-1])

    @torch.no_grad()
    def dequantize_into(self, idx: torch.Tensor, norms: torch.Tensor, out: torch.Tensor) -> None:
        """out <- (centroids[idx] Pi) * norms, with fp16 norms (cache.py:117-131)."""
        self._require(idx, "dequantize_into")
        D = self.head_dim
        codes = idx.reshape(-1, D).contiguous()
        nrm = norms.reshape(-1).to(torch.float16).contiguous()
        rows = codes.shape[0]
        if out.dtype in _lib.DTYPE_CODE and out.is_contiguous():
            dst = out
        else:
            dst = torch.empty(out.shape, dtype=torch.float32, device=out.device)
        with torch.cuda.device(idx.device):
            _lib.call("wn_dequantize", _lib.ptr(codes), _lib.ptr(nrm), rows, _lib.ptr(self.Pi),
                      _lib.ptr(self.centroids), self.bit_width, D, _lib.ptr(dst),
                      _lib.DTYPE_CODE[dst.dtype], _lib.stream_of(idx.device))
        if dst is not out:
            out.copy_(dst)


_QUANTIZER_CACHE: dict = {}


def get_quantizer(bw: int, dim: int, dev, seed: int = 42) -> TurboQuantMSE:
    """Build once per (bit_width, dim, device, seed) (cache.py:137-148)."""
    key = (bw, dim, str(torch.device(dev)), seed)
    q = _QUANTIZER_CACHE.get(key)
    if q is None:
        q = _QUANTIZER_CACHE[key] = TurboQuantMSE(bw, dim, dev, rotation_seed=seed)
    return q


_get_quantizer = get_quantizer
