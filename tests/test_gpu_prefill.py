"""GPU parity of the fused prefill over packed pages (``packed_prefill_attention``,
``wn_prefill_attention``) against the CPU oracle.

The reference serves Q > 1 by dequantizing each history and calling SDPA with the
offset causal mask (packed_backend.py:211-226; the mask is packed_attention.py:198-206:
query i of a sequence of length L, which already counts the Q new tokens, sees keys
j <= L - Q + i; a query that sees none gives 0). Its own test of that semantics is
test_packed_attention.py:84-89 (causal Q > 1 against reconstruct_attention). The fused
scan reads the packed pages directly with single fp16 operands (11 significant bits)
and fp32 accumulation, so the bar is the TF32-class decode's: within 2e-3 max-abs and
1e-3 relative of the oracle's fp32 reconstruct_attention at ordinary scales, and of the
float64 decode of operands rounded the same way (tf32_class_reference) where scores
are large enough for the rounding itself to exceed that bar.
"""
from __future__ import annotations

import math

import pytest
import torch

from cases import build, to_device
from oracle import attention as oa
from tf32_reference import prefill_q_log2, tf32_class_reference

pytestmark = pytest.mark.gpu

ATOL = 2e-3
RTOL = 1e-3
DEV = "cuda"


def _pa():
    from winnow_amd import packed_attention as pa
    return pa


def _case(seed, lens, Hq, Hkv, Q, bwk, bwv, S=16, q_scale=1.0):
    """Pages of ``lens`` tokens (the oracle quantizes them) and a (B, Hq, Q, D) query."""
    _, kv = build(seed, len(lens), Hq, Hkv, 128, lens, S, bwk, bw_v=bwv)
    q = torch.randn(len(lens), Hq, Q, 128, generator=torch.Generator().manual_seed(seed + 1)) * q_scale
    return q, kv


def _check(got, ref, lens, Q):
    got = got.float().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref).abs().max().item()
    assert torch.allclose(got, ref, atol=ATOL, rtol=RTOL), f"max abs err {err:.3e}"
    for b, L in enumerate(lens):
        blind = max(0, min(Q, Q - L))  # queries i with L - Q + i < 0 see no key
        assert (got[b, :, :blind] == 0).all()
    return err


@pytest.mark.parametrize("bwk,bwv,Hq,Hkv,Q", [
    (4, 4, 32, 8, 16), (4, 4, 32, 8, 7), (4, 4, 8, 8, 40), (4, 4, 16, 8, 33), (4, 4, 12, 4, 5),
    (6, 6, 32, 8, 16), (6, 6, 8, 8, 3), (4, 6, 64, 8, 16), (6, 4, 32, 8, 9), (4, 6, 40, 8, 2),
    (4, 4, 64, 4, 24), (4, 4, 32, 8, 64), (6, 6, 32, 8, 100), (4, 6, 64, 8, 40), (6, 4, 16, 8, 70)])
def test_prefill_matches_the_oracle(bwk, bwv, Hq, Hkv, Q):
    """Widths 4/4, 6/6, 4/6 and 6/4; n_rep 1 to 16 (query blocks that cut through a
    query's heads); ragged lengths with an empty sequence, a sequence shorter than Q
    (its first queries see no key), one of exactly Q tokens and long ones; library
    split count and fixed counts of 1 and 5. Shapes of at least eight 32-row query
    blocks per kv head (n_rep Q >= 225) run the shared-tile scan, the 6/6 case with a
    last work-group of six blocks; the others the per-wave scan."""
    lens = (0, 3, Q, 17 + Q, 700, 1500)
    print(f"prefill {bwk}/{bwv} Hq={Hq} Hkv={Hkv} Q={Q}", flush=True)
    q, kv = _case(1000 + Hq + 7 * Q + 10 * bwk + bwv, lens, Hq, Hkv, Q, bwk, bwv)
    scale = oa.default_scale(128)
    ref = oa.reconstruct_attention(q, kv, scale)
    dkv = to_device(kv, DEV)
    for splits in (None, 1, 5):
        got = _pa().packed_prefill_attention(q.to(DEV), dkv, scale, num_splits=splits, out_dtype=torch.float32)
        _check(got, ref, lens, Q)


@pytest.mark.parametrize("S", [32, 64, 256])
def test_prefill_page_sizes(S):
    """Page sizes above 16: tiles of 16 tokens inside a page, chunks across pages."""
    lens = (333, 1024, 90)
    Q = 12
    print(f"prefill S={S}", flush=True)
    q, kv = _case(1100 + S, lens, 32, 8, Q, 4, 4, S=S)
    scale = oa.default_scale(128)
    got = _pa().packed_prefill_attention(q.to(DEV), to_device(kv, DEV), scale, out_dtype=torch.float32)
    _check(got, oa.reconstruct_attention(q, kv, scale), lens, Q)


@pytest.mark.parametrize("bwk,bwv,Hq,Q", [(4, 4, 32, 20), (6, 6, 32, 20), (4, 6, 64, 20), (4, 4, 32, 96),
                                          (4, 6, 64, 48)])
def test_prefill_large_scores_against_the_rounded_operand_reference(bwk, bwv, Hq, Q):
    """Scores 50 times larger (the lazy maximum moves often) over 2,500 and 4,096
    tokens: the TF32-class rounding itself moves scores of several hundred by tenths,
    so the result is held to the float64 attention of operands rounded the same way.
    Q = 96 and 48 run the shared-tile scan."""
    lens = (2500, 4096)
    Hkv = 8
    print(f"prefill large scores {bwk}/{bwv} Hq={Hq}", flush=True)
    q, kv = _case(1200 + bwk + bwv + Hq + Q, lens, Hq, Hkv, Q, bwk, bwv, S=32, q_scale=50.0)
    scale = oa.default_scale(128)
    pa = _pa()
    B = len(lens)
    ws = torch.empty(pa.prefill_workspace_bytes(B, Hq, Hkv, Q, 128, 3), dtype=torch.uint8, device=DEV)
    got = pa.packed_prefill_attention(q.to(DEV), to_device(kv, DEV), scale, num_splits=3, workspace=ws,
                                      out_dtype=torch.float32)
    # the scan's fp32 rotated queries: one ulp of a query component near a rounding
    # halfway point moves these outputs by ~5e-3, so the reference rounds the scan's
    # own values
    q_log2 = prefill_q_log2(ws, B, Hq, Hkv, Q)
    assert torch.allclose(q_log2.double(), (q.double() @ kv.k_quant.Pi.double().T) * scale / math.log(2.0),
                          rtol=1e-5, atol=1e-4)
    _check(got, tf32_class_reference(q, kv, scale, q_log2=q_log2).float(), lens, Q)


def test_prefill_bf16_query_is_closer_to_the_oracle_than_the_reconstruct_route():
    """A bf16 query and bf16 output, as a model runs it: the fused prefill (fp16
    operands) lands at least as close to the fp32 oracle as the reference's route,
    the history dequantized to bf16 and bf16 SDPA (the product's _reconstruct_sdpa)."""
    from winnow_amd import packed_backend as pb
    lens = (600, 257, 1200)
    Q = 16
    q, kv = _case(1300, lens, 32, 8, Q, 4, 4)
    scale = oa.default_scale(128)
    qb = q.bfloat16()
    ref = oa.reconstruct_attention(qb.float(), kv, scale)
    dkv = to_device(kv, DEV)
    fused = _pa().packed_prefill_attention(qb.to(DEV), dkv, scale)
    assert fused.dtype == torch.bfloat16
    recon = pb._reconstruct_sdpa(qb.to(DEV), dkv, scale)
    e_fused = (fused.float().cpu() - ref).abs().max().item()
    e_recon = (recon.float().cpu() - ref).abs().max().item()
    assert e_fused <= e_recon * 1.05 + 1e-6, (e_fused, e_recon)
    assert e_fused < 2e-2


def test_prefill_one_query_is_the_tf32_decode_class():
    """Q = 1 through the prefill is a decode step: within the bar of the oracle and of
    the TF32-class decode."""
    lens = (0, 1, 17, 1000)
    q, kv = _case(1400, lens, 32, 8, 1, 4, 4)
    scale = oa.default_scale(128)
    dkv = to_device(kv, DEV)
    got = _pa().packed_prefill_attention(q.to(DEV), dkv, scale, out_dtype=torch.float32)
    _check(got, oa.reconstruct_attention(q, kv, scale), lens, 1)
    dec = _pa().packed_decode_attention(q.to(DEV), dkv, scale, allow_tf32=True, out_dtype=torch.float32)
    assert torch.allclose(got, dec, atol=ATOL, rtol=RTOL)


def test_prefill_strided_pool_layer_view_and_strided_query():
    """Pages handed over as one layer of a (layers, P, ...) pool (a storage offset on
    every page and norm pointer) and a query in (B, Q, Hq, D) memory order, as the
    model's attention hands it over after its transpose."""
    lens = (450, 200, 0)
    Q = 9
    q, kv = _case(1500, lens, 32, 8, Q, 4, 6)
    dkv = to_device(kv, DEV)

    def layer(t):
        return torch.stack([torch.zeros_like(t), t, torch.zeros_like(t)])[1]

    pa = _pa()
    kv2 = pa.PackedKV(layer(dkv.k_pages), layer(dkv.k_norms), layer(dkv.v_pages), layer(dkv.v_norms),
                      dkv.page_table, dkv.seq_lens, dkv.k_quant, dkv.v_quant, dkv.head_dim,
                      seq_lens_host=kv.seq_lens.clone(), page_table_host=kv.page_table.clone())
    assert kv2.k_pages.storage_offset() > 0
    qt = q.transpose(1, 2).contiguous().to(DEV).transpose(1, 2)   # (B, Hq, Q, D) view of (B, Q, Hq, D)
    assert not qt.is_contiguous()
    scale = oa.default_scale(128)
    got = pa.packed_prefill_attention(qt, kv2, scale, out_dtype=torch.float32)
    _check(got, oa.reconstruct_attention(q, kv, scale), lens, Q)


def test_prefill_route_for_bf16_queries_and_fp32_queries():
    """winnow_packed_attention sends a bf16 Q > 1 step over packed pages to the fused
    prefill and an fp32 one to the fp32 reconstruct route (the reference's numerics for
    fp32), unless the handle allows TF32-class products."""
    from winnow_amd import packed_backend as pb
    lens = (100, 40)
    Q = 4
    q, kv = _case(1600, lens, 8, 2, Q, 4, 4)
    dkv = to_device(kv, DEV)
    pb.BACKEND_COUNTS.clear()
    out, _ = pb.winnow_packed_attention(None, q.to(DEV, torch.bfloat16), dkv, None, None, scaling=0.088)
    assert pb.BACKEND_COUNTS["prefill_hip_packed"] == 1 and out.shape == (2, Q, 8, 128)
    pb.winnow_packed_attention(None, q.to(DEV), dkv, None, None, scaling=0.088)
    assert pb.BACKEND_COUNTS["prefill_reconstruct_sdpa"] == 1
    dkv.allow_tf32 = True
    pb.winnow_packed_attention(None, q.to(DEV), dkv, None, None, scaling=0.088)
    assert pb.BACKEND_COUNTS["prefill_hip_packed"] == 2
    ref = oa.reconstruct_attention(q.bfloat16().float(), kv, 0.088).transpose(1, 2)
    assert (out.float().cpu() - ref).abs().max().item() < 2e-2


def test_prefill_rejects_what_it_does_not_compile():
    q, kv = _case(1700, (50,), 8, 8, 4, 2, 2)
    with pytest.raises(_pa().UnsupportedLayout):
        _pa().packed_prefill_attention(q.to(DEV), to_device(kv, DEV), 0.088)
