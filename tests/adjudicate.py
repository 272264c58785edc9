"""Bit-exactness protocol for quantizer codes and fp16 norms.

Packing is exact on identical codes, so packed bytes must match byte for byte.
Codes come from ``bucketize(y)`` of an fp32 rotation whose summation order
differs between a CPU GEMM and the GPU kernel; a code may differ only where
that rounding can cross a boundary. A mismatch is accepted ("adjudicated") only
when all of the following hold, and is counted:

* the two codes are adjacent buckets;
* the boundary between them lies within the fp32 error bound of the exact
  (float64) rotation ``y64`` of the same fp32 ``x / n``:
  ``|y64 - b| <= (D + 4) * 2^-24 * (sum_d |xn_d Pi_jd| + |y64|)``
  (the classical dot-product bound plus the norm's own rounding);

fp16 norms may differ only by one fp16 ulp, and only when the two fp32 norms
straddle (or touch) the fp16 rounding midpoint between the two values.
Anything else is an unexplained mismatch and fails the test.
"""
from __future__ import annotations

import torch


def adjudicate_codes(x: torch.Tensor, codes_a: torch.Tensor, codes_b: torch.Tensor, tq) -> int:
    """Return the number of adjudicated code mismatches; raise AssertionError on any other."""
    D = tq.head_dim
    ca = codes_a.reshape(-1, D).cpu().long()
    cb = codes_b.reshape(-1, D).cpu().long()
    diff = (ca != cb).nonzero()
    if diff.numel() == 0:
        return 0
    flat = x.float().reshape(-1, D).cpu()
    n = flat.norm(dim=-1, keepdim=True).clamp(min=1e-10)
    xn = (flat / n).double()
    Pi = tq.Pi.cpu().double()
    bnd = tq.boundaries.cpu().double()
    for r, j in diff.tolist():
        a, b = int(ca[r, j]), int(cb[r, j])
        assert abs(a - b) == 1, f"row {r} dim {j}: codes {a} vs {b} are not adjacent"
        y = float(xn[r] @ Pi[j])
        mag = float((xn[r] * Pi[j]).abs().sum()) + abs(y)
        edge = float(bnd[min(a, b)])
        tol = (D + 4) * 2.0 ** -24 * mag
        assert abs(y - edge) <= tol, (
            f"row {r} dim {j}: codes {a}/{b} but y={y!r} is {abs(y - edge):.3e} from boundary "
            f"{edge!r} (bound {tol:.3e})")
    return int(diff.shape[0])


def adjudicate_fp16_norms(n32_a: torch.Tensor, n32_b: torch.Tensor, h_a: torch.Tensor, h_b: torch.Tensor) -> int:
    """fp16 norms h_a/h_b from fp32 norms n32_a/n32_b; return adjudicated flips, raise on others."""
    ha = h_a.reshape(-1).cpu()
    hb = h_b.reshape(-1).cpu()
    bad = (ha.view(torch.int16) != hb.view(torch.int16)).nonzero().flatten()
    na, nb = n32_a.reshape(-1).cpu().double(), n32_b.reshape(-1).cpu().double()
    for i in bad.tolist():
        ua = int(ha[i].view(torch.int16)) & 0xFFFF
        ub = int(hb[i].view(torch.int16)) & 0xFFFF
        assert abs(ua - ub) == 1, f"norm {i}: fp16 {ha[i]} vs {hb[i]} differ by more than one ulp"
        mid = (float(ha[i]) + float(hb[i])) / 2.0
        lo, hi = min(na[i], nb[i]), max(na[i], nb[i])
        slack = 4 * 2.0 ** -24 * hi
        assert lo - slack <= mid <= hi + slack, (
            f"norm {i}: fp32 norms {na[i]!r}/{nb[i]!r} do not straddle the fp16 midpoint {mid!r}")
    return int(bad.numel())
