"""GPU parity of the TF32-class decode (``allow_tf32=True``, ``wn_decode_attention_tf32``)
against the CPU oracle.

The reference's kernel hands ``allow_tf32`` to both ``tl.dot`` products
(packed_attention_triton.py:113, 127): with it set, the products take operands of ten
stored mantissa bits and accumulate in fp32. The TF32-class row scan (4 or 6-bit K
and V, alike or mixed, up to eight query heads per kv head) rounds each operand
to fp16 (eleven significant bits) and accumulates in fp32. The bar is the north
star's: within 2e-3 max-abs and 1e-3 relative of the oracle's fp32 tiled path
(``tiled_compressed_attention``, packed_attention.py:260-311); rows of empty
sequences are exactly zero. Shapes the TF32-class scan does not cover run the
fp32-exact scan and give the default call's result bit for bit.
"""
from __future__ import annotations

import pytest
import torch

from cases import build, to_device
from oracle import attention as oa
from tf32_reference import tf32_class_reference

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3
DEV = "cuda"
RAGGED = (0, 1, 15, 16, 17, 333, 1024)
RAGGED_WITH_GAPS = (0, 130, 0, 0, 64, 1, 700, 0, 65, 2000, 0)


def _pa():
    from winnow_amd import packed_attention as pa
    return pa


def _check(got, ref, lens):
    got = got.float().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs().max().item()
    assert torch.allclose(got, ref, atol=ATOL, rtol=RTOL), f"max abs err {err:.3e}"
    for b, L in enumerate(lens):
        if L == 0:
            assert (got[b] == 0).all()
    return err


@pytest.mark.parametrize("bwk,bwv,Hq,Hkv", [
    (4, 4, 32, 8), (4, 4, 16, 8), (4, 4, 8, 8), (4, 4, 24, 8), (4, 4, 8, 2),
    (6, 6, 32, 8), (6, 6, 8, 8), (4, 6, 32, 8), (6, 4, 32, 8),
    (4, 4, 64, 8), (4, 6, 64, 8), (6, 6, 64, 8), (6, 4, 64, 8), (4, 6, 40, 8), (6, 6, 56, 8),
    (4, 4, 32, 2), (4, 6, 64, 4)])
def test_tf32_matches_oracle(bwk, bwv, Hq, Hkv):
    """4 and 6-bit K and V, alike and mixed: n_rep 4, 2, 1 and 3 (one head group,
    padded columns), n_rep 8, 5 and 7 (two groups), n_rep 16 (virtual kv heads of
    eight); ragged lengths with an empty sequence, library plan and two fixed splits."""
    print(f"tf32 {bwk}/{bwv} Hq={Hq} Hkv={Hkv}", flush=True)
    q, kv = build(700 + Hq + Hkv + 10 * bwk + bwv, len(RAGGED), Hq, Hkv, 128, RAGGED, 16, bwk, bw_v=bwv)
    scale = oa.default_scale(128)
    ref = oa.tiled_compressed_attention(q, kv, scale)
    dkv = to_device(kv, DEV)
    for splits in (None, 2):
        got = _pa().packed_decode_attention(q.to(DEV), dkv, scale, num_splits=splits, allow_tf32=True,
                                            out_dtype=torch.float32)
        _check(got, ref, RAGGED)


@pytest.mark.parametrize("waves,bwk,bwv,Hq", [(1, 4, 4, 32), (5, 4, 4, 32), (37, 4, 4, 32), (5, 6, 6, 32),
                                              (37, 4, 6, 64), (8, 4, 6, 64)])
def test_tf32_balanced_plan_with_few_waves(waves, bwk, bwv, Hq):
    """A balanced plan over a handful of waves: each wave scans runs of chunks, crosses
    (sequence, kv head) boundaries and skips zero-length sequences mid-share."""
    lens = RAGGED_WITH_GAPS
    print(f"tf32 balanced {waves} waves {bwk}/{bwv} Hq={Hq}", flush=True)
    q, kv = build(800 + waves + bwk + bwv, len(lens), Hq, 8, 128, lens, 16, bwk, bw_v=bwv)
    scale = oa.default_scale(128)
    ref = oa.tiled_compressed_attention(q, kv, scale)
    got = _pa().packed_decode_attention(q.to(DEV), to_device(kv, DEV), scale, plan=(0, waves), allow_tf32=True,
                                        out_dtype=torch.float32)
    _check(got, ref, lens)


@pytest.mark.parametrize("bwk,bwv,Hq", [(4, 4, 32), (6, 6, 32), (4, 6, 64)])
def test_tf32_large_scores_and_long_history(bwk, bwv, Hq):
    """Scores 50 times larger (the lazy maximum moves often) over 4,096 and 2,500 tokens,
    S=32. Here the TF32-class rounding itself moves scores of several hundred by tenths,
    beyond the fp32 bar, as the reference's allow_tf32 does; so the result is checked
    against the float64 decode of operands rounded the same way (tf32_class_reference),
    at the north-star tolerance. The default call stays within the bar of the fp32
    oracle, and the two results differ (the TF32-class scan ran)."""
    lens = (4096, 2500)
    print(f"tf32 large scores {bwk}/{bwv} Hq={Hq}", flush=True)
    q, kv = build(901 + bwk + bwv + Hq, len(lens), Hq, 8, 128, lens, 32, bwk, bw_v=bwv, q_scale=50.0)
    scale = oa.default_scale(128)
    dkv, qd = to_device(kv, DEV), q.to(DEV)
    tf = _pa().packed_decode_attention(qd, dkv, scale, allow_tf32=True, out_dtype=torch.float32)
    exact = _pa().packed_decode_attention(qd, dkv, scale, out_dtype=torch.float32)
    _check(tf, tf32_class_reference(q, kv, scale).float(), lens)
    _check(exact, oa.tiled_compressed_attention(q, kv, scale), lens)
    assert not torch.equal(tf, exact)


@pytest.mark.parametrize("bwk,bwv,Hq", [(4, 4, 32), (6, 6, 32), (4, 6, 64)])
def test_tf32_matches_the_rounded_operand_reference(bwk, bwv, Hq):
    """At ordinary scales the TF32-class result also sits within the bar of the decode of
    rounded operands (the check above, on the ragged batch)."""
    q, kv = build(902 + bwk + bwv + Hq, len(RAGGED), Hq, 8, 128, RAGGED, 16, bwk, bw_v=bwv)
    scale = oa.default_scale(128)
    tf = _pa().packed_decode_attention(q.to(DEV), to_device(kv, DEV), scale, allow_tf32=True,
                                       out_dtype=torch.float32)
    _check(tf, tf32_class_reference(q, kv, scale).float(), RAGGED)


@pytest.mark.parametrize("bwk,bwv,Hq,Hkv", [(2, 2, 16, 4), (5, 5, 32, 8), (3, 3, 64, 8), (4, 8, 32, 8)])
def test_tf32_other_shapes_run_the_exact_scan(bwk, bwv, Hq, Hkv):
    """Width pairs without a TF32-class scan (2, 3 and 5 bits, 8-bit values) give the
    default call's output bit for bit."""
    q, kv = build(950 + bwk + bwv, len(RAGGED), Hq, Hkv, 128, RAGGED, 16, bwk, bw_v=bwv)
    scale = oa.default_scale(128)
    dkv, qd = to_device(kv, DEV), q.to(DEV)
    tf = _pa().packed_decode_attention(qd, dkv, scale, allow_tf32=True, out_dtype=torch.float32)
    exact = _pa().packed_decode_attention(qd, dkv, scale, out_dtype=torch.float32)
    assert torch.equal(tf, exact)


def test_tf32_bf16_query_and_output():
    """bf16 query in, bf16 output out (the cast after the merge), as the default path."""
    q, kv = build(960, 2, 32, 8, 128, (300, 77), 16, 4)
    scale = oa.default_scale(128)
    got = _pa().packed_decode_attention(q.to(DEV, torch.bfloat16), to_device(kv, DEV), scale, allow_tf32=True)
    assert got.dtype == torch.bfloat16
    ref = oa.tiled_compressed_attention(q.bfloat16().float(), kv, scale)
    assert (got.float().cpu() - ref).abs().max() < 2e-2


def test_tf32_strided_pool_layer_view():
    """Pages handed over as one layer of a (layers, P, ...) pool tensor (a storage offset
    on every page and norm pointer)."""
    lens = (450, 200, 0)
    q, kv = build(961, len(lens), 32, 8, 128, lens, 16, 4)
    dkv = to_device(kv, DEV)

    def layer(t):
        return torch.stack([torch.zeros_like(t), t, torch.zeros_like(t)])[1]

    pa = _pa()
    kv2 = pa.PackedKV(layer(dkv.k_pages), layer(dkv.k_norms), layer(dkv.v_pages), layer(dkv.v_norms),
                      dkv.page_table, dkv.seq_lens, dkv.k_quant, dkv.v_quant, dkv.head_dim,
                      seq_lens_host=kv.seq_lens.clone(), page_table_host=kv.page_table.clone())
    assert kv2.k_pages.storage_offset() > 0
    scale = oa.default_scale(128)
    got = pa.packed_decode_attention(q.to(DEV), kv2, scale, allow_tf32=True, out_dtype=torch.float32)
    _check(got, oa.tiled_compressed_attention(q, kv, scale), lens)
