"""GPU checks of the split merge for batches of many (kv head, sequence) pairs.

At head_dim 128, with 512 or more work-groups' worth of (query-head group of four, kv
head, sequence), the merge runs four heads per work-group (``merge4_kernel``), which
reads Pi_V a quarter as often; smaller batches keep one head per work-group
(``merge_kernel``). Both merge a (sequence, head)'s partials in the same order, so
the outputs must be the same bits. With fixed splits and equal lengths a sequence's
partials do not depend on the rest of the batch (``cdiv(max_pages, n)`` pages per
split, packed_attention_triton.py:211-216), so the first eight sequences of a
64-sequence batch (merge4_kernel) must equal, bit for bit, the same eight decoded
alone (merge_kernel); the large batch is also held to the oracle at the north-star
tolerance (2e-3 abs, 1e-3 rel).
"""
from __future__ import annotations

import pytest
import torch

from cases import build, to_device
from oracle import attention as oa

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL, RTOL = 2e-3, 1e-3


@pytest.mark.parametrize("Hq", [8, 24, 32, 40, 64])
def test_large_batch_merge_equals_the_per_head_merge(Hq):
    """n_rep 1, 3, 4, 5, 8 (groups of four heads with idle waves and padded columns)."""
    from winnow_amd import packed_attention as pa
    B, Hkv, L = 64, 8, 300
    lens = (L,) * B
    print(f"merge B={B} Hq={Hq}", flush=True)
    q, kv = build(1900 + Hq, B, Hq, Hkv, 128, lens, 16, 4)
    scale = oa.default_scale(128)
    dkv = to_device(kv, DEV)
    big = pa.packed_decode_attention(q.to(DEV), dkv, scale, num_splits=3, out_dtype=torch.float32)
    ref = oa.tiled_compressed_attention(q, kv, scale)
    assert torch.allclose(big.cpu(), ref, atol=ATOL, rtol=RTOL), (big.cpu() - ref).abs().max()
    n = 8
    small_kv = pa.PackedKV(dkv.k_pages, dkv.k_norms, dkv.v_pages, dkv.v_norms, dkv.page_table[:n].contiguous(),
                           dkv.seq_lens[:n].contiguous(), dkv.k_quant, dkv.v_quant, dkv.head_dim,
                           seq_lens_host=kv.seq_lens[:n].clone(), page_table_host=kv.page_table[:n].clone())
    small = pa.packed_decode_attention(q[:n].to(DEV), small_kv, scale, num_splits=3, out_dtype=torch.float32)
    assert torch.equal(big[:n], small)


def test_large_batch_dense_merge_equals_the_per_head_merge():
    """The dense decode's merge (no output rotation) at 64 sequences x 8 kv heads."""
    from winnow_amd import packed_attention as pa
    B, Hq, Hkv, L, S = 64, 32, 8, 200, 16
    g = torch.Generator().manual_seed(1950)
    need = (L + S - 1) // S
    kp = torch.randn(B * need, Hkv, S, 128, generator=g).bfloat16()
    vp = torch.randn(B * need, Hkv, S, 128, generator=g).bfloat16()
    table = torch.randperm(B * need, generator=g).to(torch.int32).reshape(B, need)
    sl = torch.full((B,), L, dtype=torch.int32)
    q = torch.randn(B, Hq, 1, 128, generator=g)
    scale = 0.09
    kv = pa.DenseKV(kp.to(DEV), vp.to(DEV), table.to(DEV), sl.to(DEV), 128)
    big = pa.dense_decode_attention(q.to(DEV), kv, scale, num_splits=2, out_dtype=torch.float32)
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
    assert torch.allclose(big.cpu().double(), ref, atol=ATOL, rtol=RTOL), (big.cpu().double() - ref).abs().max()
    n = 8
    kv8 = pa.DenseKV(kp.to(DEV), vp.to(DEV), table[:n].contiguous().to(DEV), sl[:n].to(DEV), 128)
    small = pa.dense_decode_attention(q[:n].to(DEV), kv8, scale, num_splits=2, out_dtype=torch.float32)
    assert torch.equal(big[:n], small)
