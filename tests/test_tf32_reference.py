"""Pins the float64 TF32-class reference (``tf32_reference.tf32_class_reference``) on the
CPU, so that the GPU test comparing the TF32-class scan against it compares with a
checked function:

- with its rounding switched off it is the float64 oracle decode
  (``reconstruct_attention_f64``) to float64 rounding;
- its rounding is fp16's (11 significant bits, ties to even), ties included;
- with the rounding on, at scores fifty times the usual size, it moves away from the
  fp32 oracle by more than the fp32 bar (the case it exists for), and at ordinary
  scales it stays within that bar of it.
"""
from __future__ import annotations

import torch

from cases import build
from oracle import attention as oa
from tf32_reference import round11, tf32_class_reference

LENS = (0, 1, 17, 130, 300)


def test_without_rounding_it_is_the_float64_oracle():
    for Hq, Hkv, seed in ((32, 8, 1), (8, 8, 2), (12, 4, 3)):
        q, kv = build(seed, len(LENS), Hq, Hkv, 128, LENS, 16, 4)
        scale = oa.default_scale(128)
        got = tf32_class_reference(q, kv, scale, rnd=lambda x: x.double())
        want = oa.reconstruct_attention_f64(q, kv, scale)
        assert (got - want).abs().max().item() < 1e-12


def test_rounding_is_fp16_rounding():
    """Over fp16's normal range (|x| >= 2^-14). Below it fp16 keeps fewer bits and
    round11 does not; in the scan those are query components 2^-29 below the largest,
    which the power-of-two scaling keeps out of the sums' significant bits."""
    g = torch.Generator().manual_seed(7)
    # fp32 inputs, as the scan's operands are: torch converts float64 to fp16 through
    # fp32 (two roundings), while round11 and the scan's fp32 -> fp16 round once
    x = torch.cat([torch.randn(10000, generator=g) * s for s in (1e-3, 1.0, 300.0)])
    x = x[x.abs() >= 2.0 ** -14]
    assert x.numel() > 25000
    assert torch.equal(round11(x.double()), x.half().double())
    one = torch.tensor([1.0], dtype=torch.float64)
    ulp = 2.0 ** -10
    # halfway cases go to the even significand, as fp16 conversion does
    assert round11(one + ulp / 2).item() == 1.0
    assert round11(one + 3 * ulp / 2).item() == 1.0 + 2 * ulp
    assert torch.equal(round11(torch.tensor([1.0 + ulp / 2, 1.0 + 3 * ulp / 2], dtype=torch.float64)),
                       torch.tensor([1.0 + ulp / 2, 1.0 + 3 * ulp / 2], dtype=torch.float64).half().double())


def test_rounding_matters_where_it_should():
    lens = (700, 300)
    scale = oa.default_scale(128)
    q, kv = build(11, len(lens), 32, 8, 128, lens, 16, 4, q_scale=50.0)
    big = (tf32_class_reference(q, kv, scale) - oa.reconstruct_attention_f64(q, kv, scale)).abs().max().item()
    assert big > 2e-3
    q, kv = build(12, len(lens), 32, 8, 128, lens, 16, 4)
    ordinary = (tf32_class_reference(q, kv, scale).float() - oa.tiled_compressed_attention(q, kv, scale))
    assert torch.allclose(ordinary, torch.zeros_like(ordinary), atol=2e-3)


def test_prefill_queries_follow_the_offset_causal_mask():
    """Q > 1: with the rounding off it is the oracle's fp32 reconstruct attention
    (offset causal mask, rows without a key = 0) to fp32 rounding, the queries of a
    sequence shorter than Q included; query i of one row, alone as a Q = 1 decode of
    the history cut at L - Q + i + 1, gives the same row."""
    lens = (0, 3, 17, 130, 300)
    Q = 5
    q, kv = build(21, len(lens), 12, 4, 128, lens, 16, 4)
    q = torch.randn(len(lens), 12, Q, 128, generator=torch.Generator().manual_seed(22))
    scale = oa.default_scale(128)
    got = tf32_class_reference(q, kv, scale, rnd=lambda x: x.double())
    want = oa.reconstruct_attention(q, kv, scale)
    assert (got.float() - want).abs().max().item() < 1e-5
    assert (got[1, :, :2] == 0).all()            # L = 3 < Q: queries 0 and 1 see no key
    b, i = 3, 2
    cut = oa.OracleKV(kv.k_pages, kv.k_norms, kv.v_pages, kv.v_norms, kv.page_table,
                      torch.tensor([lens[b] - Q + i + 1 if j == b else 0 for j in range(len(lens))],
                                   dtype=torch.int32), kv.k_quant, kv.v_quant, kv.head_dim)
    one = tf32_class_reference(q[:, :, i:i + 1], cut, scale, rnd=lambda x: x.double())
    assert (one[b, :, 0] - got[b, :, i]).abs().max().item() < 1e-12
