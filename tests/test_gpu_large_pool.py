"""Pools whose pages lie beyond 4 GiB of byte offset (one MI355X holds 288 GB of HBM).

The reference's pool is one tensor per side, ``(layers, P, Hkv, S, NB)``
(page_pool.py:73-78), and its kernels address a page as ``pid * page_stride``.
A pool of more than 2^32 bytes is ordinary at this memory size, so every product
kernel must form page addresses in 64 bits. Each test here places the pages of
a small batch on both sides of the 4 GiB offset of a ~4.3 GB pool and checks
that the result is bit-identical to the same pages in a compact pool, whose
parity with the oracle the other GPU tests establish. The decode is also held
to the north star's 2e-3 / 1e-3 against the CPU oracle directly.
"""
from __future__ import annotations

import pytest
import torch

from cases import build, to_device
from oracle import attention as oa

pytestmark = pytest.mark.gpu

DEV = "cuda"
FOUR_GIB = 1 << 32


def _first_high_page(page_bytes: int, n: int) -> int:
    """A base id so that ids [base, base + n) straddle byte offset 2^32."""
    return FOUR_GIB // page_bytes - n // 2


def _spread(pages: torch.Tensor, base: int, P: int) -> torch.Tensor:
    """A zeroed pool of P pages holding ``pages`` at ids base, base+1, ..."""
    big = torch.zeros((P,) + tuple(pages.shape[1:]), dtype=pages.dtype, device=DEV)
    big[base:base + pages.shape[0]] = pages
    return big


def _shift(table: torch.Tensor, base: int) -> torch.Tensor:
    return torch.where(table >= 0, table + base, table)


@pytest.mark.parametrize("bwk,bwv", [(4, 4), (4, 6)])
def test_packed_decode_reads_pages_beyond_4gib(bwk, bwv):
    from winnow_amd import packed_attention as pa
    lens = (300, 1000, 17)
    q, kv = build(4100 + bwv, 3, 32, 8, 128, lens, 16, bwk, bw_v=bwv)
    scale = oa.default_scale(128)
    small = to_device(kv, DEV)
    n = small.k_pages.shape[0]
    page_bytes = small.k_pages[0].numel()
    base = _first_high_page(page_bytes, n)
    P = base + n + 3
    assert (base + n) * page_bytes > FOUR_GIB > base * page_bytes
    print(f"packed decode bw {bwk}/{bwv}: {n} pages at ids {base}..{base + n - 1}, "
          f"pool {P * page_bytes / 2 ** 30:.2f} GiB per side", flush=True)
    table = _shift(kv.page_table, base)
    big = pa.PackedKV(_spread(small.k_pages, base, P), _spread(small.k_norms, base, P),
                      _spread(small.v_pages, base, P), _spread(small.v_norms, base, P),
                      table.to(DEV), small.seq_lens, small.k_quant, small.v_quant, 128,
                      seq_lens_host=kv.seq_lens.clone(), page_table_host=table.clone())
    for splits in (None, 1):
        want = pa.packed_decode_attention(q.to(DEV), small, scale, num_splits=splits, out_dtype=torch.float32)
        got = pa.packed_decode_attention(q.to(DEV), big, scale, num_splits=splits, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(got, want), splits
    ref = oa.tiled_compressed_attention(q, kv, scale)
    assert torch.allclose(got.cpu(), ref, atol=2e-3, rtol=1e-3)
    del big
    torch.cuda.empty_cache()


def test_append_and_history_dequant_beyond_4gib():
    """wn_append_kv scatters into pages past 4 GiB exactly as into a compact pool, and
    wn_dequantize_history reads them back identically."""
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    from winnow_amd.quantizer import get_quantizer
    B, Hkv, n_new, D, S, bw = 2, 8, 40, 128, 16, 4
    tq_k, tq_v = get_quantizer(bw, D, DEV, 42), get_quantizer(bw, D, DEV, 43)
    g = torch.Generator().manual_seed(77)
    k = torch.randn(B, Hkv, n_new, D, generator=g).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, Hkv, n_new, D, generator=g).to(torch.bfloat16).to(DEV)
    start = torch.tensor([5, 0], dtype=torch.int32, device=DEV)       # sequence 0 starts mid-page
    per_seq = 4                                                        # pages per sequence cover 5 + 40 tokens
    n = B * per_seq
    order = torch.randperm(n, generator=g).to(torch.int32).view(B, per_seq)
    NB = D * bw // 8
    page_bytes = Hkv * S * NB
    base = _first_high_page(page_bytes, n)
    P = base + n + 3
    assert (base + n) * page_bytes > FOUR_GIB > base * page_bytes
    print(f"append: {n} pages at ids {base}..{base + n - 1}, pool {P * page_bytes / 2 ** 30:.2f} GiB", flush=True)
    pools = {}
    for name, (npages, tab) in {"small": (n, order), "big": (P, order + base)}.items():
        kp = torch.zeros(npages, Hkv, S, NB, dtype=torch.uint8, device=DEV)
        vp = torch.zeros_like(kp)
        kn = torch.zeros(npages, Hkv, S, dtype=torch.float16, device=DEV)
        vn = torch.zeros_like(kn)
        table = tab.to(DEV)
        pb.append_kv(k, v, tq_k, tq_v, kp, vp, kn, vn, table, start)
        pools[name] = (kp, vp, kn, vn, tab)
    torch.cuda.synchronize()
    sk, sv, skn, svn, _ = pools["small"]
    bk, bv, bkn, bvn, _ = pools["big"]
    assert torch.equal(bk[base:base + n], sk) and torch.equal(bv[base:base + n], sv)
    assert torch.equal(bkn[base:base + n], skn) and torch.equal(bvn[base:base + n], svn)
    assert int(bk[:base].count_nonzero()) == 0 and int(bk[base + n:].count_nonzero()) == 0
    lens = (start.cpu() + n_new).to(torch.int32)
    hist = {}
    for name, (kp, vp, kn, vn, tab) in pools.items():
        kv = pa.PackedKV(kp, kn, vp, vn, tab.to(DEV), lens.to(DEV),
                         pa.Quantizer(tq_k.Pi, tq_k.centroids, bw), pa.Quantizer(tq_v.Pi, tq_v.centroids, bw), D,
                         seq_lens_host=lens.clone(), page_table_host=tab.clone())
        hist[name] = [pb.dequantize_history(kv, kv.v_pages, kv.v_norms, kv.v_quant, b, torch.float32)
                      for b in range(B)]
    for b in range(B):
        assert torch.equal(hist["big"][b], hist["small"][b]), b
    del pools
    torch.cuda.empty_cache()


def test_dense_decode_reads_pages_beyond_4gib():
    from winnow_amd import packed_attention as pa
    lens, Hkv, S, D = (200, 513), 8, 16, 128
    g = torch.Generator().manual_seed(4242)
    need = [(L + S - 1) // S for L in lens]
    n = sum(need)
    kp = torch.randn(n, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    vp = torch.randn(n, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV)
    order = torch.randperm(n, generator=g).tolist()
    table = torch.full((len(lens), max(need)), -1, dtype=torch.int32)
    for b, k in enumerate(need):
        for t in range(k):
            table[b, t] = order.pop()
    q = torch.randn(len(lens), 32, 1, D, generator=g).to(DEV)
    sl = torch.tensor(lens, dtype=torch.int32, device=DEV)
    page_bytes = kp[0].numel() * kp.element_size()
    base = _first_high_page(page_bytes, n)
    P = base + n + 3
    assert (base + n) * page_bytes > FOUR_GIB > base * page_bytes
    print(f"dense decode: {n} pages at ids {base}..{base + n - 1}, pool {P * page_bytes / 2 ** 30:.2f} GiB "
          f"per side", flush=True)
    small = pa.DenseKV(kp, vp, table.to(DEV), sl, D)
    big = pa.DenseKV(_spread(kp, base, P), _spread(vp, base, P), _shift(table, base).to(DEV), sl, D)
    want = pa.dense_decode_attention(q, small, 0.1, out_dtype=torch.float32)
    got = pa.dense_decode_attention(q, big, 0.1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    del big
    torch.cuda.empty_cache()
