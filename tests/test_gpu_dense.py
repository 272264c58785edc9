"""GPU parity of the dense (unquantized) paged decode, the matched baseline of the
packed decode (``dense_decode_attention``, packed_attention_triton.py:190-201).

Checked against the float64 oracle ``dense_paged_attention_f64`` (itself pinned to
SDPA over contiguous K/V) on the same bf16 / fp16 page values, at the tolerance of
the packed decode: fp32 output within 2e-3 abs / 1e-3 rel. The case matrix: the
reference's own test case (test_packed_attention_triton.py:153-173: B 3, Hq 28, Hkv
4, lengths 33 / 0 / 70, shuffled tables, splits 1, 2, 3), every n_rep class up to
16 and n_rep 17-96 as virtual kv heads, page sizes 16 / 32 / 64, ragged lengths
including 0, 1, 15, 16, 17, head_dim 64 and 128, fp16 and fp32 pages, bf16 output,
long contexts, and the rejections.
"""
from __future__ import annotations

import pytest
import torch

from oracle import attention as oa

DEV = "cuda"
ATOL, RTOL = 2e-3, 1e-3


def _pages(seed, lens, Hkv, S, dtype=torch.bfloat16, D=128, spare=2, width=None):
    g = torch.Generator().manual_seed(seed)
    need = [(L + S - 1) // S for L in lens]
    P = sum(need) + spare
    kp = torch.randn(P, Hkv, S, D, generator=g).to(dtype)
    vp = torch.randn(P, Hkv, S, D, generator=g).to(dtype)
    order = torch.randperm(P, generator=g).tolist()
    table = torch.full((len(lens), width or max(max(need), 1)), -1, dtype=torch.int32)
    for b, L in enumerate(lens):
        for t in range(need[b]):
            table[b, t] = order.pop()
    return kp, vp, table, torch.tensor(lens, dtype=torch.int32)


def _run(q, kp, vp, table, sl, scale, **kw):
    from winnow_amd import packed_attention as pa
    kv = pa.DenseKV(kp.to(DEV), vp.to(DEV), table.to(DEV), sl.to(DEV), kp.shape[-1])
    return pa.dense_decode_attention(q.to(DEV), kv, scale, **kw)


@pytest.mark.gpu
@pytest.mark.parametrize("splits", [None, 1, 2, 3])
def test_dense_matches_the_reference_case(splits):
    """test_packed_attention_triton.py:153-173 with bf16 pages."""
    kp, vp, table, sl = _pages(8, (33, 0, 70), 4, 16, width=5)
    q = torch.randn(3, 28, 1, 128, generator=torch.Generator().manual_seed(9))
    got = _run(q, kp, vp, table, sl, 0.09, num_splits=splits, out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, 0.09)
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()
    assert bool((got[1] == 0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 8), (32, 8), (28, 4), (64, 8), (16, 1)])
@pytest.mark.parametrize("S", [16, 64])
def test_dense_head_groups_and_page_sizes(Hq, Hkv, S):
    lens = (0, 1, 15, 16, 17, 333, 1024)
    kp, vp, table, sl = _pages(20 + Hq + S, lens, Hkv, S)
    q = torch.randn(len(lens), Hq, 1, 128, generator=torch.Generator().manual_seed(Hq))
    scale = 128 ** -0.5
    got = _run(q, kp, vp, table, sl, scale, out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv,S", [(8, 2, 16), (16, 1, 32), (14, 2, 64)])
def test_dense_head_dim_64(Hq, Hkv, S):
    lens = (0, 1, 17, 333, 1024)
    kp, vp, table, sl = _pages(80 + Hq + S, lens, Hkv, S, D=64)
    q = torch.randn(len(lens), Hq, 1, 64, generator=torch.Generator().manual_seed(Hq + S))
    scale = 64 ** -0.5
    got = _run(q, kp, vp, table, sl, scale, out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()
    for s in (1, 3):
        got_s = _run(q, kp, vp, table, sl, scale, num_splits=s, out_dtype=torch.float32).cpu()
        assert torch.allclose(got_s.double(), ref, atol=ATOL, rtol=RTOL)


@pytest.mark.gpu
def test_dense_fp16_pages_bf16_query_and_output():
    lens = (77, 500, 4)
    kp, vp, table, sl = _pages(31, lens, 4, 32, dtype=torch.float16)
    q = torch.randn(3, 16, 1, 128, generator=torch.Generator().manual_seed(5)).bfloat16()
    got = _run(q, kp, vp, table, sl, 0.1)
    assert got.dtype == torch.bfloat16
    ref = oa.dense_paged_attention_f64(q.float(), kp, vp, table, sl, 0.1)
    assert torch.allclose(got.cpu().double(), ref, atol=1e-2, rtol=1e-2)
    got32 = _run(q, kp, vp, table, sl, 0.1, out_dtype=torch.float32).cpu()
    assert torch.allclose(got32.double(), ref, atol=ATOL, rtol=RTOL), (got32.double() - ref).abs().max()


@pytest.mark.gpu
def test_dense_long_context_splits_agree():
    """16k and 40k tokens: the balanced plan and fixed splits give the same result."""
    lens = (16384, 40000)
    kp, vp, table, sl = _pages(41, lens, 8, 16)
    q = torch.randn(2, 32, 1, 128, generator=torch.Generator().manual_seed(6))
    scale = 128 ** -0.5
    a = _run(q, kp, vp, table, sl, scale, out_dtype=torch.float32).cpu()
    for s in (1, 7, 64):
        b = _run(q, kp, vp, table, sl, scale, num_splits=s, out_dtype=torch.float32).cpu()
        assert torch.allclose(a, b, atol=1e-5, rtol=1e-5), (s, (a - b).abs().max())
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
    assert torch.allclose(a.double(), ref, atol=ATOL, rtol=RTOL), (a.double() - ref).abs().max()


@pytest.mark.gpu
def test_dense_large_scores_stay_finite():
    kp, vp, table, sl = _pages(51, (300,), 2, 16)
    q = torch.randn(1, 4, 1, 128, generator=torch.Generator().manual_seed(7)) * 30
    got = _run(q, kp, vp, table, sl, 1.0, out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, 1.0)
    assert torch.isfinite(got).all()
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()


@pytest.mark.gpu
@pytest.mark.parametrize("D", [128, 64])
@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (28, 4), (32, 8), (16, 1)])
def test_dense_fp32_pages(D, Hq, Hkv):
    """fp32 pages (the reference's dense_decode_attention takes them,
    packed_attention_triton.py:190-201) on the vector-ALU scan, fixed splits: the
    library's plan, one and three splits, ragged lengths including 0."""
    lens = (0, 1, 17, 333, 1024)
    kp, vp, table, sl = _pages(80 + Hq + D, lens, Hkv, 16, dtype=torch.float32, D=D)
    q = torch.randn(len(lens), Hq, 1, D, generator=torch.Generator().manual_seed(81))
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, D ** -0.5)
    for splits in (None, 1, 3):
        print(f"fp32 pages D={D} Hq={Hq} Hkv={Hkv} splits={splits}", flush=True)
        got = _run(q, kp, vp, table, sl, D ** -0.5, num_splits=splits, out_dtype=torch.float32).cpu()
        assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()
        assert bool((got[0] == 0).all())


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Hq,Hkv", [(34, 2), (40, 2), (64, 2), (96, 1)])
def test_dense_more_than_sixteen_query_heads(dtype, Hq, Hkv):
    """n_rep 17, 20, 32 and 96 run as virtual kv heads of <= 16 query heads each
    (the reference pads its head block to next_pow2(n_rep), packed_attention_triton.py:209)."""
    lens = (0, 33, 300)
    kp, vp, table, sl = _pages(90 + Hq, lens, Hkv, 16, dtype=dtype)
    q = torch.randn(len(lens), Hq, 1, 128, generator=torch.Generator().manual_seed(91))
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, 0.088)
    for splits in (None, 2):
        print(f"dense n_rep={Hq // Hkv} {dtype} splits={splits}", flush=True)
        got = _run(q, kp, vp, table, sl, 0.088, num_splits=splits, out_dtype=torch.float32).cpu()
        assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()


@pytest.mark.gpu
def test_dense_rejections():
    from winnow_amd import packed_attention as pa
    kp, vp, table, sl = _pages(61, (20,), 2, 16)
    q = torch.randn(1, 4, 1, 128)
    with pytest.raises(pa.UnsupportedLayout):        # more than one query token
        _run(torch.randn(1, 4, 2, 128), kp, vp, table, sl, 0.1)
    kp8, vp8, table8, sl8 = _pages(62, (20,), 2, 8)
    with pytest.raises(pa.UnsupportedLayout):        # page size below 16
        _run(q, kp8, vp8, table8, sl8, 0.1)
    kv = pa.DenseKV(kp.to(DEV), vp.to(DEV)[:, :, :, :64].contiguous(), table.to(DEV), sl.to(DEV), 128)
    with pytest.raises(pa.UnsupportedLayout):        # K and V strides differ
        pa.dense_decode_attention(q.to(DEV), kv, 0.1)


@pytest.mark.gpu
def test_dense_rejects_bad_metadata_before_launch():
    """A live page id outside the pool or a length beyond the table never reaches the
    kernel; with ``check_ranges=False`` the same call on good metadata still runs."""
    from winnow_amd import packed_attention as pa
    kp, vp, table, sl = _pages(73, (20, 40), 2, 16, spare=0)
    q = torch.randn(2, 4, 1, 128, generator=torch.Generator().manual_seed(5))
    P = kp.shape[0]
    for bad_table, bad_len, why in ((torch.tensor([[0, P, -1], [1, 2, 3]], dtype=torch.int32), sl, "sequence 0"),
                                    (torch.tensor([[0, 4, -1], [1, -1, 3]], dtype=torch.int32), sl, "sequence 1"),
                                    (table, torch.tensor([20, 49], dtype=torch.int32), "out of range")):
        with pytest.raises(pa.UnsupportedLayout, match=why):
            _run(q, kp, vp, bad_table, bad_len, 0.1)
    got = _run(q, kp, vp, table, sl, 0.1, check_ranges=False, out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, 0.1)
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL)


def test_dense_decode_has_no_host_path():
    from winnow_amd import packed_attention as pa
    kp, vp, table, sl = _pages(71, (20,), 2, 16)
    with pytest.raises(pa.UnsupportedLayout):
        pa.dense_decode_attention(torch.randn(1, 4, 1, 128), pa.DenseKV(kp, vp, table, sl, 128), 0.1)


@pytest.mark.gpu
@pytest.mark.parametrize("waves", [1, 5, 37])
@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (64, 4)])
def test_dense_balanced_plan_with_few_waves(waves, Hq, Hkv):
    """The dense scan's balanced loop with each wave walking many chunks across
    (sequence, kv head) boundaries and over zero-length sequences mid-share."""
    lens = (0, 130, 0, 0, 64, 1, 700, 0, 65, 2000, 0)
    kp, vp, table, sl = _pages(600 + waves + Hq, lens, Hkv, 16)
    q = torch.randn(len(lens), Hq, 1, 128, generator=torch.Generator().manual_seed(waves))
    scale = 128 ** -0.5
    got = _run(q, kp, vp, table, sl, scale, plan=(0, waves), out_dtype=torch.float32).cpu()
    ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
    assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), (got.double() - ref).abs().max()
    assert bool((got[[0, 2, 3, 7, 10]] == 0).all())
