"""Pins the oracle's TurboQuant quantizer (oracle/quantizer.py, restating cache.py:62-131).

* Lloyd-Max codebook (cache.py:62-82): replayed independently, with the cell
  conditional means computed by numerical quadrature of x*phi(x) and phi(x)
  instead of the closed form ``sigma*(pdf(lo)-pdf(hi))/(cdf(hi)-cdf(lo))``,
  from the same ``linspace(-3 sigma, 3 sigma)`` start under the same stopping
  rule (200 steps, or the first step moving no centroid by 1e-12); the fp32
  centroids and midpoint boundaries must come out identical. Symmetry
  ``c_i = -c_{L-1-i}`` and the Gaussian relative-L2 distortions the reference
  recorded per width (results/bitwidth_sweep.json, "rel_l2_gaussian") are
  checked on top.
* Rotation (cache.py:92-97): orthogonal, and ``Pi^T G`` upper triangular with a
  positive diagonal for the seeded Gaussian draw G -- the QR factor with a
  positive-diagonal R is unique, so this fixes Pi up to rounding.
* quantize (cache.py:108-115): ``#{boundary < y}`` (torch.bucketize right=False)
  on values placed exactly on boundaries; zero vectors (norm clamps to 1e-10);
  fp32 norms against float64.
* dequantize (cache.py:117-131): equals ``centroids[idx] @ Pi * n`` (test_cache.py:17-23)
  and the fp16-norm budget of test_cache.py:26-60.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
from scipy import integrate

from oracle import quantizer as oq

SIGMA_128 = 1.0 / math.sqrt(128)

# results/bitwidth_sweep.json rows[*].rel_l2_gaussian (mean over vectors of
# ||x_hat - x|| / ||x||, 10240 N(0,1) vectors of dim 128)
REL_L2_GAUSSIAN = {3: 0.18380960822105408, 4: 0.09626737982034683, 5: 0.04964372143149376,
                   6: 0.026249954476952553, 8: 0.006993969436734915}


def _lloyd_by_quadrature(levels, sigma, iters=200, tol=1e-12):
    """Lloyd-Max iteration with cell means from adaptive quadrature (independent of the closed form)."""
    def phi(x):
        return math.exp(-0.5 * (x / sigma) ** 2)

    c = np.array([-3 * sigma + 6 * sigma * i / (levels - 1) for i in range(levels)])
    for _ in range(iters):
        b = [-math.inf] + [(c[i] + c[i + 1]) / 2 for i in range(levels - 1)] + [math.inf]
        new = np.empty(levels)
        for i in range(levels):
            m0 = integrate.quad(phi, b[i], b[i + 1], epsabs=0, epsrel=1e-13, limit=200)[0]
            m1 = integrate.quad(lambda x: x * phi(x), b[i], b[i + 1], epsabs=0, epsrel=1e-13, limit=200)[0]
            new[i] = m1 / m0
        moved = np.max(np.abs(new - c))
        c = new
        if moved < tol:
            break
    return c


@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_lloyd_max_matches_independent_quadrature(bw):
    c_ref = _lloyd_by_quadrature(2 ** bw, SIGMA_128)
    tq = oq.OracleTQ(bw, 128, 42)
    assert tq.centroids.dtype == torch.float32 and tq.centroids.numel() == 2 ** bw
    assert np.array_equal(tq.centroids.numpy(), c_ref.astype(np.float32))
    mids = ((c_ref[:-1] + c_ref[1:]) / 2).astype(np.float32)
    got = tq.boundaries.numpy()
    # The middle boundary is zero up to float64 rounding of the closed-form cell
    # means (about 1e-17, sign set by the reference's call sequence, which the
    # oracle repeats); every other boundary is bit-identical.
    mid = len(mids) // 2
    assert abs(float(got[mid])) < 1e-15 and abs(float(mids[mid])) < 1e-15
    assert np.array_equal(np.delete(got, mid), np.delete(mids, mid))
    assert np.all(np.diff(got) > 0)


@pytest.mark.parametrize("bw", [2, 3, 4, 6, 8])
def test_codebook_symmetry(bw):
    c, b = oq.lloyd_max_gaussian(2 ** bw, SIGMA_128)
    assert np.allclose(c, -c[::-1], atol=1e-15)
    assert b[0] == -np.inf and b[-1] == np.inf


def test_planted_codebook_mistakes_fail_the_replay():
    """A wrong start (+-2 sigma), sigma = 1 / D, or one step fewer cap is caught."""
    good = _lloyd_by_quadrature(8, SIGMA_128).astype(np.float32)
    c_bad_sigma, _ = oq.lloyd_max_gaussian(8, sigma=1.0 / 128)
    assert not np.array_equal(c_bad_sigma.astype(np.float32), good)
    c2 = np.linspace(-2 * SIGMA_128, 2 * SIGMA_128, 16)
    ref16 = _lloyd_by_quadrature(16, SIGMA_128).astype(np.float32)
    # 16 levels stop on the step cap, so the start point still shows in the fp32 values
    c_wrong = c2.copy()
    for _ in range(200):
        b = np.concatenate(([-np.inf], (c_wrong[:-1] + c_wrong[1:]) / 2, [np.inf])) / SIGMA_128
        from scipy.stats import norm
        p = norm.cdf(b[1:]) - norm.cdf(b[:-1])
        c_wrong = SIGMA_128 * (norm.pdf(b[:-1]) - norm.pdf(b[1:])) / p
    assert not np.array_equal(c_wrong.astype(np.float32), ref16)
    c_short, _ = oq.lloyd_max_gaussian(16, SIGMA_128, iters=150)
    assert not np.array_equal(c_short.astype(np.float32), ref16)


@pytest.mark.parametrize("bw", [3, 4, 5, 6, 8])
def test_gaussian_distortion_matches_reference_record(bw):
    g = torch.Generator().manual_seed(1234)
    x = torch.randn(10240, 128, generator=g)
    tq = oq.get_quantizer(bw, 128, 42)
    idx, n = tq.quantize(x)
    rec = tq.dequantize(idx, n)
    rel = ((rec - x).norm(dim=-1) / x.norm(dim=-1)).mean().item()
    want = REL_L2_GAUSSIAN[bw]
    assert abs(rel - want) / want < 0.01, (bw, rel, want)


@pytest.mark.parametrize("seed", [42, 43])
@pytest.mark.parametrize("D", [64, 128])
def test_rotation_is_the_positive_diagonal_qr_factor(seed, D):
    Pi = oq.rotation(D, seed)
    G = oq.gaussian_draw(D, seed)
    eye = torch.eye(D, dtype=torch.float64)
    P64 = Pi.double()
    assert (P64.T @ P64 - eye).abs().max() < 1e-5
    R = P64.T @ G.double()
    assert R.tril(-1).abs().max() < 1e-4          # upper triangular
    assert (R.diagonal() > 0).all()               # positive diagonal
    assert torch.det(P64).abs().sub(1).abs() < 1e-4


def test_rotation_seeds_differ_and_are_not_symmetric():
    a, b = oq.rotation(128, 42), oq.rotation(128, 43)
    assert not torch.equal(a, b)
    assert not torch.allclose(a, a.T)


def test_bucketize_counts_boundaries_strictly_below():
    """With Pi = I and a norm of exactly 5, y = (3/5, 4/5, 0, ...) in fp32; boundaries placed
    exactly on those values are not counted (right=False)."""
    tq = oq.OracleTQ(4, 8, 42)
    tq.Pi = torch.eye(8)
    y0 = float(torch.tensor(3.0) / torch.tensor(5.0))
    y1 = float(torch.tensor(4.0) / torch.tensor(5.0))
    tq.boundaries = torch.tensor([-0.5, 0.0, y0, 0.7, y1, 0.9], dtype=torch.float32)
    x = torch.tensor([[3.0, 4.0, 0, 0, 0, 0, 0, 0]])
    idx, n = tq.quantize(x)
    assert float(n) == 5.0
    assert idx.tolist() == [[2, 4, 1, 1, 1, 1, 1, 1]]
    # just above a boundary counts it
    x2 = torch.tensor([[3.0 + 1e-5, 4.0, 0, 0, 0, 0, 0, 0]])
    assert tq.quantize(x2)[0][0, 0].item() == 3


def test_zero_and_tiny_vectors():
    tq = oq.get_quantizer(4, 128, 42)
    x = torch.zeros(3, 128)
    x[1, 7] = 1e-30
    idx, n = tq.quantize(x)
    assert n[0].item() == pytest.approx(1e-10, rel=1e-6)   # clamp(min=1e-10)
    zero_code = int((tq.boundaries < 0).sum())
    assert (idx[0] == zero_code).all()
    assert n.half()[0].item() == 0.0                       # 1e-10 underflows fp16


def test_norms_against_float64():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(512, 128, generator=g) * torch.logspace(-3, 3, 512)[:, None]
    _, n = oq.get_quantizer(6, 128, 42).quantize(x)
    n64 = x.double().norm(dim=-1)
    assert ((n.double() - n64).abs() / n64).max() < 2e-7


def test_codes_are_nearest_centroid_of_rotated_vector():
    """Lloyd boundaries are centroid midpoints, so each code is the nearest centroid to y."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(256, 128, generator=g)
    tq = oq.get_quantizer(4, 128, 42)
    idx, _ = tq.quantize(x)
    y = tq.rotated(x)
    nearest = (y[..., None] - tq.centroids.double()).abs().argmin(-1)
    agree = (nearest == idx.long()).float().mean().item()
    assert agree > 0.9999


@pytest.mark.parametrize("bw", [3, 4])
def test_dequantize_and_fp16_norm_budget(bw):
    """test_cache.py:26-60: dequantize == centroids[idx] @ Pi * n; fp16 norms cost < 1% of the
    quantization error."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 4, 64, 128, generator=g)
    tq = oq.get_quantizer(bw, 128, 42)
    idx, n = tq.quantize(x)
    ref = (tq.centroids[idx.long()].reshape(-1, 128) @ tq.Pi * n.reshape(-1, 1)).view(x.shape)
    assert torch.allclose(tq.dequantize(idx, n), ref, atol=1e-6)
    half = tq.dequantize(idx, n.half().float())
    assert (half - ref).abs().max() / (ref - x).abs().max() < 0.01
