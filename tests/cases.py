"""Case builders shared by the parity tests.

Inputs are built the way the reference's tests build them
(``test_packed_attention_triton.py:30-39``, ``test_packed_attention.py:53-63``):
a seeded CPU generator draws K, V and q; the CPU oracle quantizes them into
randomly ordered pages (``pages_from_dense``); the same pages then go to the
device as the product's ``PackedKV``. The oracle is the checker here only.
"""
from __future__ import annotations

import torch

from oracle import attention as oa
from oracle.quantizer import get_quantizer as oracle_quantizer

# Frozen differential matrix of test_packed_attention_triton.py:51-68
# (name, B, Hq, Hkv, D, lens, S, bw, q_scale) with its fixed seeds.
CASES = [
    ("qwen7b_gqa_short", 3, 28, 4, 128, (1, 17, 64), 16, 8, 1.0),
    ("qwen7b_gqa_mixed", 4, 28, 4, 128, (0, 300, 31, 129), 32, 8, 1.0),
    ("mha_like", 2, 8, 8, 64, (40, 7), 16, 8, 1.0),
    ("gqa8_2", 3, 8, 2, 64, (16, 33, 1), 16, 8, 1.0),
    ("huge_scores", 2, 28, 4, 128, (90, 47), 16, 8, 50.0),
    ("four_bit", 2, 28, 4, 128, (77, 160), 16, 4, 1.0),
    ("three_bit", 2, 8, 2, 128, (50, 19), 16, 3, 1.0),
    ("long_4k", 2, 28, 4, 128, (4096, 2500), 32, 8, 1.0),
    ("batch32", 32, 28, 4, 128, tuple(range(5, 5 + 32 * 61, 61)), 16, 8, 1.0),
]
CASE_SEEDS = {"qwen7b_gqa_short": 101, "qwen7b_gqa_mixed": 102, "mha_like": 103, "gqa8_2": 104,
              "huge_scores": 105, "four_bit": 106, "three_bit": 107, "long_4k": 108, "batch32": 109}


def build(seed, B, Hq, Hkv, D, lens, S, bw, q_scale=1.0, distinct=True, bw_v=None, num_pages=None):
    """(q, oracle KV) on the CPU, quantized by the oracle, pages shuffled."""
    g = torch.Generator().manual_seed(seed)
    Lmax = max(max(lens), 1)
    k = torch.randn(B, Hkv, Lmax, D, generator=g)
    v = torch.randn(B, Hkv, Lmax, D, generator=g)
    q = torch.randn(B, Hq, 1, D, generator=g) * q_scale
    kq = oracle_quantizer(bw, D, 42)
    vq = oracle_quantizer(bw_v or bw, D, 43 if distinct else 42)
    kv = oa.pages_from_dense(k, v, lens, kq, vq, S, num_pages=num_pages, generator=g)
    return q, kv


def to_device(kv, dev):
    """The oracle's pages as the product's PackedKV on ``dev`` (host mirrors attached)."""
    from winnow_amd import packed_attention as pa
    return pa.PackedKV(kv.k_pages.to(dev), kv.k_norms.to(dev), kv.v_pages.to(dev), kv.v_norms.to(dev),
                       kv.page_table.to(dev), kv.seq_lens.to(dev),
                       pa.Quantizer(kv.k_quant.Pi.to(dev), kv.k_quant.centroids.to(dev), kv.k_quant.bit_width),
                       pa.Quantizer(kv.v_quant.Pi.to(dev), kv.v_quant.centroids.to(dev), kv.v_quant.bit_width),
                       kv.head_dim, seq_lens_host=kv.seq_lens.clone(), page_table_host=kv.page_table.clone())


def to_host(kv, seqs=None):
    """Device PackedKV -> oracle KV on the CPU, optionally restricted to sequences ``seqs``
    (their pages are renumbered compactly)."""
    table = kv.page_table_host if kv.page_table_host is not None else kv.page_table.cpu()
    lens = kv.seq_lens_host if kv.seq_lens_host is not None else kv.seq_lens.cpu()
    kq = oa.OracleQuant(kv.k_quant.Pi.cpu(), kv.k_quant.centroids.cpu(), kv.k_quant.bit_width)
    vq = oa.OracleQuant(kv.v_quant.Pi.cpu(), kv.v_quant.centroids.cpu(), kv.v_quant.bit_width)
    if seqs is None:
        return oa.OracleKV(kv.k_pages.cpu(), kv.k_norms.cpu(), kv.v_pages.cpu(), kv.v_norms.cpu(),
                           table.clone(), lens.clone().to(torch.int32), kq, vq, kv.head_dim)
    S = kv.page_size
    rows = []
    for b in seqs:
        n = (int(lens[b]) + S - 1) // S
        rows.append(table[b, :n].long())
    ids = torch.cat(rows) if rows else torch.zeros(0, dtype=torch.long)
    width = max(max((len(r) for r in rows), default=1), 1)
    new_table = torch.full((len(seqs), width), -1, dtype=torch.int32)
    off = 0
    for i, r in enumerate(rows):
        new_table[i, :len(r)] = torch.arange(off, off + len(r), dtype=torch.int32)
        off += len(r)
    dev_ids = ids.to(kv.k_pages.device)
    return oa.OracleKV(kv.k_pages[dev_ids].cpu(), kv.k_norms[dev_ids].cpu(), kv.v_pages[dev_ids].cpu(),
                       kv.v_norms[dev_ids].cpu(), new_table,
                       torch.tensor([int(lens[b]) for b in seqs], dtype=torch.int32), kq, vq, kv.head_dim)


def config1_inputs():
    """B1, 8 q = 8 kv heads, D128, 1024 tokens, fp32 K/V/q ~N(0,1) from seed 0
    (drawn K, then V, then q), 4-bit, 16-token pages in table order 0..63, quantizer seed 42 for
    K and V (the reference's default, packed_backend.py:298-303)."""
    g = torch.Generator().manual_seed(0)
    k = torch.randn(1, 8, 1024, 128, generator=g)
    v = torch.randn(1, 8, 1024, 128, generator=g)
    q = torch.randn(1, 8, 1, 128, generator=g)
    return q, k, v


def config1_kv():
    """The oracle's packed pages of config 1: contiguous table, K and V through oracle.append."""
    from oracle import append as oapp
    q, k, v = config1_inputs()
    tq = oracle_quantizer(4, 128, 42)
    P, S = 64, 16
    kp = torch.zeros(P, 8, S, 64, dtype=torch.uint8)
    vp = torch.zeros(P, 8, S, 64, dtype=torch.uint8)
    kn = torch.zeros(P, 8, S, dtype=torch.float16)
    vn = torch.zeros(P, 8, S, dtype=torch.float16)
    table = torch.arange(P, dtype=torch.int32)[None]
    oapp.append(k, tq, kp, kn, table, [0])
    oapp.append(v, tq, vp, vn, table, [0])
    quant = oa.OracleQuant.from_tq(tq)
    kv = oa.OracleKV(kp, kn, vp, vn, table, torch.tensor([1024], dtype=torch.int32), quant, quant, 128)
    return q, k, v, kv
