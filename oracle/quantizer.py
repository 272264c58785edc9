"""Oracle: TurboQuant MSE quantizer on the CPU -- test infrastructure only.

Restates ``turboquant_kv/cache.py:62-131`` with the same library calls
(numpy float64 Lloyd-Max iteration with ``scipy.stats.norm``; ``torch.randn`` on
a seeded CPU generator followed by ``torch.linalg.qr`` and a sign fix; torch CPU
fp32 ``norm`` / matmul / ``bucketize``), so on one image it reproduces the
reference's constants and codes bit for bit.

Pinned by (``tests/test_oracle_quantizer.py``):

* ``lloyd_max_gaussian``: the Lloyd-Max optimality conditions (every centroid
  is the conditional mean of its cell, computed independently by quadrature;
  every boundary is the midpoint of its neighbours), symmetry
  ``c_i = -c_{L-1-i}``, and the Gaussian relative-L2 distortions the reference
  records per width (``results/bitwidth_sweep.json``: 0.1838 / 0.0963 / 0.0496 /
  0.0262 / 0.0070 for 3 / 4 / 5 / 6 / 8 bits).
* ``rotation``: orthogonality and the uniqueness of a QR factorisation with a
  positive-diagonal R (``Pi^T G`` must be upper triangular with a positive
  diagonal, where ``G`` is the seeded Gaussian draw).
* ``quantize``: bucketize semantics on hand-built vectors that sit exactly on,
  just below and just above fp32 boundaries; zero vectors (norm clamps to
  1e-10, every code equals ``#{b < 0}``); the norm against a float64 norm.
* The exact fp32 bits of ``Pi`` (seeds 42 and 43) and of every codebook
  (2-8 bits): ``tests/golden/reference_constants.json``, written in the build
  container by the reference's own ``TurboQuantMSE`` (``cache.py:84-106``),
  checked by ``tests/test_golden.py``.

The fp32 QR's bits depend on the host's CPU and on LAPACK's thread count, so the
standard rotations (head_dim 128, seeds 42 and 43) are not rebuilt: ``rotation``
loads the reference's single-threaded bits from ``winnow_amd/rotations_d128.npz``
(data the same script writes; the product loads them too), and every host
quantizes with the same ``Pi``. ``qr_rotation`` is the restated construction; on
the build container it reproduces those bits exactly (``tests/test_golden.py``).
"""
from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch
from scipy.stats import norm as _norm


def lloyd_max_gaussian(levels: int, sigma: float = 1.0, iters: int = 200, tol: float = 1e-12):
    """Lloyd-Max centroids and boundaries (with +-inf ends) for N(0, sigma^2).

    cache.py:62-82: linspace(-3s, 3s) start, conditional-mean update on
    standardised cell edges, stop at ``iters`` or when ``max|dc| < tol``.
    """
    c = np.linspace(-3 * sigma, 3 * sigma, levels)
    for _ in range(iters):
        b = np.concatenate(([-np.inf], (c[:-1] + c[1:]) / 2.0, [np.inf]))
        new_c = np.empty_like(c)
        for i in range(levels):
            lo, hi = b[i] / sigma, b[i + 1] / sigma
            p = _norm.cdf(hi) - _norm.cdf(lo)
            if p < 1e-300:
                new_c[i] = c[i]
                continue
            new_c[i] = sigma * (_norm.pdf(lo) - _norm.pdf(hi)) / p
        done = np.max(np.abs(new_c - c)) < tol
        c = new_c
        if done:
            break
    b = np.concatenate(([-np.inf], (c[:-1] + c[1:]) / 2.0, [np.inf]))
    return c, b


_CANONICAL = Path(__file__).resolve().parents[1] / "winnow_amd" / "rotations_d128.npz"


def rotation(head_dim: int, seed: int) -> torch.Tensor:
    """Seeded random orthogonal matrix (cache.py:92-97): the reference's single-threaded
    bits for head_dim 128 at seeds 42 and 43, else ``qr_rotation`` on this host."""
    if head_dim == 128 and seed in (42, 43):
        with np.load(_CANONICAL) as f:
            return torch.from_numpy(np.array(f[f"pi_{seed}"], dtype=np.float32)).contiguous()
    return qr_rotation(head_dim, seed)


def qr_rotation(head_dim: int, seed: int) -> torch.Tensor:
    """Q of QR(randn) times sign(diag R) (cache.py:92-97), the QR on one thread.

    Its fp32 rounding depends on the host's CPU and thread count; one thread gives
    the same bits on every host of one CPU model.
    """
    gen = torch.Generator(device="cpu").manual_seed(seed)
    G = torch.randn(head_dim, head_dim, generator=gen, dtype=torch.float32)
    threads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        Q, R = torch.linalg.qr(G)
    finally:
        torch.set_num_threads(threads)
    ds = torch.sign(torch.diag(R))
    ds[ds == 0] = 1.0
    return (Q * ds.unsqueeze(0)).contiguous()


def gaussian_draw(head_dim: int, seed: int) -> torch.Tensor:
    """The matrix ``rotation`` factorises (exposed for the uniqueness check)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(head_dim, head_dim, generator=gen, dtype=torch.float32)


class OracleTQ:
    """CPU restatement of ``TurboQuantMSE`` (cache.py:85-131)."""

    def __init__(self, bit_width: int, head_dim: int, rotation_seed: int = 42):
        self.Pi = rotation(head_dim, rotation_seed)
        c, b = lloyd_max_gaussian(2 ** bit_width, sigma=1.0 / math.sqrt(head_dim))
        self.centroids = torch.tensor(c, dtype=torch.float32).contiguous()
        self.boundaries = torch.tensor(b[1:-1], dtype=torch.float32).contiguous()
        self.bit_width = bit_width
        self.head_dim = head_dim

    @torch.no_grad()
    def quantize(self, x: torch.Tensor):
        """(..., D) -> (uint8 codes (..., D), fp32 norms (...)) -- cache.py:108-115."""
        flat = x.float().reshape(-1, self.head_dim)
        norms = flat.norm(dim=-1, keepdim=True).clamp(min=1e-10)
        y = (flat / norms) @ self.Pi.T
        idx = torch.bucketize(y, self.boundaries).to(torch.uint8)
        return idx.view(x.shape), norms.squeeze(-1).view(x.shape[:-1])

    @torch.no_grad()
    def rotated(self, x: torch.Tensor) -> torch.Tensor:
        """float64 ``(x/n) Pi^T`` with the fp32 ``x/n`` of ``quantize`` (for adjudication)."""
        flat = x.float().reshape(-1, self.head_dim)
        norms = flat.norm(dim=-1, keepdim=True).clamp(min=1e-10)
        return ((flat / norms).double() @ self.Pi.double().T).view(x.shape)

    @torch.no_grad()
    def dequantize(self, idx: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        """``centroids[idx] @ Pi * n`` in fp32 (cache.py:117-131)."""
        D = self.head_dim
        y = self.centroids.index_select(0, idx.reshape(-1).to(torch.int32)).view(-1, D)
        return ((y @ self.Pi) * norms.reshape(-1, 1).float()).view(idx.shape)


_CACHE: dict = {}


def get_quantizer(bit_width: int, head_dim: int, seed: int = 42) -> OracleTQ:
    """Memoised like ``cache._get_quantizer`` (cache.py:137-148)."""
    key = (bit_width, head_dim, seed)
    q = _CACHE.get(key)
    if q is None:
        q = _CACHE[key] = OracleTQ(bit_width, head_dim, seed)
    return q
