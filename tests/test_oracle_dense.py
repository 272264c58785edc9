"""Pins ``oracle.attention.dense_paged_attention_f64``, the reference for the dense
decode (packed_attention_triton.py:190-201, whose own test compares it with the page
gather + SDPA of packed_backend.py:229-246, test_packed_attention_triton.py:153-173).

The independent side is torch's scaled_dot_product_attention (float64) over the
contiguous K/V the pages were scattered from, so paging never enters it. Planted
mistakes (pages in the wrong order, a dropped tail page, the wrong GQA head map)
must miss by far more than the tolerance.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oa


def _case(seed, lens, Hq, Hkv, S, D=128, spare=3):
    g = torch.Generator().manual_seed(seed)
    B, Lmax = len(lens), max(max(lens), 1)
    k = torch.randn(B, Hkv, Lmax, D, generator=g, dtype=torch.float64)
    v = torch.randn(B, Hkv, Lmax, D, generator=g, dtype=torch.float64)
    need = [(L + S - 1) // S for L in lens]
    P = sum(need) + spare
    order = torch.randperm(P, generator=g).tolist()
    kp = torch.randn(P, Hkv, S, D, generator=g, dtype=torch.float64)  # unused pages hold noise
    vp = torch.randn(P, Hkv, S, D, generator=g, dtype=torch.float64)
    table = torch.full((B, max(max(need), 1)), -1, dtype=torch.int32)
    for b, L in enumerate(lens):
        for t in range(need[b]):
            pid = order.pop()
            table[b, t] = pid
            n = min(S, L - t * S)
            kp[pid, :, :n] = k[b, :, t * S:t * S + n]
            vp[pid, :, :n] = v[b, :, t * S:t * S + n]
    return k, v, kp, vp, table, torch.tensor(lens, dtype=torch.int32)


def _sdpa(q, k, v, lens, scale):
    """Contiguous reference: per sequence, SDPA over its first L keys with the offset causal mask."""
    B, Hq, Q, D = q.shape
    out = torch.zeros(B, Hq, Q, D, dtype=torch.float64)
    for b, L in enumerate(lens.tolist()):
        if L == 0:
            continue
        mask = torch.arange(L)[None, :] <= (L - Q + torch.arange(Q))[:, None]
        out[b] = F.scaled_dot_product_attention(q[b:b + 1].double(), k[b:b + 1, :, :L], v[b:b + 1, :, :L],
                                                attn_mask=mask, scale=scale,
                                                enable_gqa=Hq != k.shape[1])[0]
    return out


@pytest.mark.parametrize("lens,Hq,Hkv,S,Q", [((33, 0, 70), 28, 4, 16, 1), ((1, 17, 64), 8, 8, 16, 1),
                                             ((5, 100), 16, 2, 32, 3), ((129,), 32, 8, 64, 1)])
def test_dense_oracle_matches_contiguous_sdpa(lens, Hq, Hkv, S, Q):
    k, v, kp, vp, table, sl = _case(7 + Hq, lens, Hq, Hkv, S)
    q = torch.randn(len(lens), Hq, Q, 128, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    got = oa.dense_paged_attention_f64(q, kp, vp, table, sl, 0.09)
    ref = _sdpa(q, k, v, sl, 0.09)
    assert torch.allclose(got, ref, atol=1e-12, rtol=1e-12), (got - ref).abs().max()
    for b, L in enumerate(lens):
        if L == 0:
            assert bool((got[b] == 0).all())


def test_dense_oracle_catches_planted_paging_and_head_mistakes():
    lens = (45, 70)
    k, v, kp, vp, table, sl = _case(11, lens, 8, 2, 16)
    q = torch.randn(2, 8, 1, 128, generator=torch.Generator().manual_seed(4), dtype=torch.float64)
    ref = _sdpa(q, k, v, sl, 0.09)
    tol = 1e-6
    # pages of sequence 1 in reverse order
    bad = table.clone()
    bad[1, :5] = table[1, :5].flip(0)
    assert (oa.dense_paged_attention_f64(q, kp, vp, bad, sl, 0.09) - ref).abs().max() > 100 * tol
    # the partial tail page dropped (L rounded down to whole pages)
    short = torch.tensor([32, 64], dtype=torch.int32)
    assert (oa.dense_paged_attention_f64(q, kp, vp, table, short, 0.09) - ref).abs().max() > 100 * tol
    # query head h read from kv head h % Hkv instead of h // n_rep
    # (SDPA's GQA map is h // n_rep; reordering the query heads gives the h % Hkv map)
    wrong = _sdpa(q[:, [0, 2, 4, 6, 1, 3, 5, 7]], k, v, sl, 0.09)[:, [0, 4, 1, 5, 2, 6, 3, 7]]
    assert (oa.dense_paged_attention_f64(q, kp, vp, table, sl, 0.09) - wrong).abs().max() > 100 * tol
