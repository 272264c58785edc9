"""The reference's frozen kernel-screen cases for decode attention.

``turboquant_kv/tsc/validation.py:192-238`` (``attention_cases``, ``validate_attention``)
screens every decode schedule on four frozen cases before it may be used: an empty
sequence beside one-token, page-boundary and one-past-a-page sequences; a page-tail
batch; two long sequences; and scores forty times the usual size. Case ``i`` draws its
K, V and q from ``torch.Generator().manual_seed(1101 + i)`` (``VALIDATION_SEEDS[0] + i``,
``validation.py:42, 202``), quantizes K with rotation seed 42 and V with 43, and scatters
the pages in the generator's random order (``pages_from_dense``); a schedule passes when
its output is finite and within atol = rtol = 2e-3 of ``tiled_compressed_attention``
(``validation.py:209-238``). The reference screens at 28 query / 4 kv heads, head_dim
128, 16-token pages, 8-bit codes (``test_tsc_wrong_code.py:53-57``).

Here the same cases, drawn the same way, run through the HIP decode at 4, 6 and 8 bits,
at the reference's head family and at BASELINE's Llama-3 family (32 / 8), on the
default plan and two fixed split counts, against the oracle's restatement of
``tiled_compressed_attention``; the bar is the screen's and the north star's
(2e-3 absolute, 1e-3 relative). The matched unquantized decode runs the same K/V as
bf16 pages against the float64 dense oracle.
"""
from __future__ import annotations

import pytest
import torch

from cases import to_device
from oracle import attention as oa
from oracle.quantizer import get_quantizer as oracle_quantizer

pytestmark = pytest.mark.gpu

DEV = "cuda"
VALIDATION_SEED0 = 1101          # validation.py:42 VALIDATION_SEEDS[0]; case i uses 1101 + i
SCREEN_ATOL, SCREEN_RTOL = 2e-3, 2e-3     # validation.py:211
ATOL, RTOL = 2e-3, 1e-3                   # the north star's bar


def screen_specs(S):
    """(lens, q scale) of validation.py:196-197."""
    return [((0, 1, S, S + 1), 1.0), ((3 * S - 1, 70, 5), 1.0), ((1024, 517), 1.0), ((200, 33, 64, 9), 40.0)]


def screen_cases(hq, hkv, D, S, bw):
    """The frozen cases as validation.py:192-207 draws them: (name, q, k, v, oracle KV)."""
    for i, (lens, qs) in enumerate(screen_specs(S)):
        g = torch.Generator().manual_seed(VALIDATION_SEED0 + i)
        B, Lmax = len(lens), max(max(lens), 1)
        k = torch.randn(B, hkv, Lmax, D, generator=g)
        v = torch.randn(B, hkv, Lmax, D, generator=g)
        q = torch.randn(B, hq, 1, D, generator=g) * qs
        kv = oa.pages_from_dense(k, v, lens, oracle_quantizer(bw, D, 42), oracle_quantizer(bw, D, 43), S,
                                 generator=g)
        yield f"lens{lens}_q{qs}", q, k, v, kv


def _check(name, got, ref):
    assert torch.isfinite(got).all(), f"{name}: non-finite outputs"
    err = (got - ref).abs()
    assert torch.allclose(got, ref, atol=SCREEN_ATOL, rtol=SCREEN_RTOL), f"{name}: max abs err {float(err.max()):.3e}"
    bound = ATOL + RTOL * ref.abs()
    assert bool((err <= bound).all()), f"{name}: max abs err {float(err.max()):.3e} beyond 2e-3 + 1e-3|ref|"


@pytest.mark.parametrize("bw", [4, 6, 8])
@pytest.mark.parametrize("hq,hkv", [(28, 4), (32, 8)])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_packed_decode_passes_the_kernel_screen(bw, hq, hkv, splits):
    from winnow_amd import packed_attention as pa
    D, S = 128, 16
    scale = oa.default_scale(D)
    for name, q, _, _, kv in screen_cases(hq, hkv, D, S, bw):
        ref = oa.tiled_compressed_attention(q, kv, scale)
        got = pa.packed_decode_attention(q.to(DEV), to_device(kv, DEV), scale, num_splits=splits,
                                         out_dtype=torch.float32).cpu()
        _check(f"bw{bw} {hq}/{hkv} splits={splits} {name}", got, ref)


def _dense_pages(k, v, kv, dtype):
    """bf16/fp16 pages holding k, v at the screen case's page ids (the table of ``kv``)."""
    B, Hkv, _, D = k.shape
    P, S = kv.k_pages.shape[0], kv.k_pages.shape[2]
    kp = torch.zeros(P, Hkv, S, D, dtype=dtype)
    vp = torch.zeros(P, Hkv, S, D, dtype=dtype)
    for b, L in enumerate(kv.seq_lens.tolist()):
        for t in range((L + S - 1) // S):
            pid, lo, hi = int(kv.page_table[b, t]), t * S, min((t + 1) * S, L)
            kp[pid, :, :hi - lo] = k[b, :, lo:hi].to(dtype)
            vp[pid, :, :hi - lo] = v[b, :, lo:hi].to(dtype)
    return kp, vp


@pytest.mark.parametrize("hq,hkv", [(28, 4), (32, 8)])
@pytest.mark.parametrize("splits", [None, 1, 3])
def test_dense_decode_passes_the_kernel_screen(hq, hkv, splits):
    from winnow_amd import packed_attention as pa
    D, S = 128, 16
    scale = oa.default_scale(D)
    for name, q, k, v, kv in screen_cases(hq, hkv, D, S, 8):
        kp, vp = _dense_pages(k, v, kv, torch.bfloat16)
        ref = oa.dense_paged_attention_f64(q, kp, vp, kv.page_table, kv.seq_lens, scale).float()
        dkv = pa.DenseKV(kp.to(DEV), vp.to(DEV), kv.page_table.to(DEV), kv.seq_lens.to(DEV), D)
        got = pa.dense_decode_attention(q.to(DEV), dkv, scale, num_splits=splits, out_dtype=torch.float32).cpu()
        _check(f"dense {hq}/{hkv} splits={splits} {name}", got, ref)
