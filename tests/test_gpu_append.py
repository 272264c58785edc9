"""GPU parity of the append path: quantize, pack/unpack, scatter into pool pages, dequantize.

Codes and fp16 norms must be bit-exact versus the CPU oracle (the reference's
``TurboQuantMSE.quantize`` + ``pack`` + page scatter, cache.py:108-115,
packing.py:37-64, packed_backend.py:155-161) under the adjudication protocol of
``adjudicate.py``; packed bytes of identical codes must be identical. Covers
the round trip of test_packing.py:20-46 on the device, the fp16-norm budget of
test_cache.py:26-60, and BASELINE config 3's append shape.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from adjudicate import adjudicate_codes, adjudicate_fp16_norms
from oracle import append as oapp
from oracle import packing as opk
from oracle.quantizer import get_quantizer as oracle_quantizer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _q(bw, D, seed):
    from winnow_amd.quantizer import get_quantizer
    return get_quantizer(bw, D, DEV, seed)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_pack_unpack_match_oracle(bw, D):
    from winnow_amd import packing
    g = torch.Generator().manual_seed(bw * 100 + D)
    idx = torch.randint(0, 2 ** bw, (7, 4, 33, D), dtype=torch.uint8, generator=g)
    got = packing.pack(idx.to(DEV), bw)
    want = opk.pack(idx.numpy(), bw)
    assert got.shape == (7, 4, 33, opk.packed_bytes(D, bw))
    assert np.array_equal(got.cpu().numpy(), want)
    back = packing.unpack(got, bw, D)
    assert torch.equal(back.cpu(), idx)


@pytest.mark.parametrize("bw", [3, 4, 6, 8])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_bit_exact(bw, dtype):
    D = 128
    g = torch.Generator().manual_seed(bw)
    x = torch.randn(4096, D, generator=g).to(dtype)
    x[0] = 0                                                     # zero vector: norm clamps to 1e-10
    x[1, :] = 0
    x[1, 5] = 3.0                                                # one-hot: y is a column of Pi
    x[2] *= 1e-30                                                # tiny but non-zero
    tq = _q(bw, D, 42)
    oq = oracle_quantizer(bw, D, 42)
    assert torch.equal(tq.Pi.cpu(), oq.Pi) and torch.equal(tq.boundaries.cpu(), oq.boundaries)
    codes, norms = tq.quantize(x.to(DEV))
    ocodes, onorms = oq.quantize(x)
    flips = adjudicate_codes(x, codes, ocodes, oq)
    print(f"bw={bw} {dtype}: {flips} adjudicated code flips of {codes.numel()}")
    assert flips <= max(2, codes.numel() // 20000)
    assert torch.allclose(norms.cpu(), onorms, rtol=2e-6, atol=0)
    nflips = adjudicate_fp16_norms(norms, onorms, norms.half(), onorms.half())
    assert nflips <= 2
    assert int(codes[0, 0]) == int((oq.boundaries < 0).sum())   # #{b < 0}


def test_quantize_on_exact_boundaries():
    """y exactly on a boundary must not count that boundary (bucketize right=False)."""
    D = 128
    tq = _q(4, D, 42)
    Pi = tq.Pi.cpu().double()
    bnd = tq.boundaries.cpu()
    # x = Pi^T e aligns y with a scaled unit vector: y_j = n * e_j / n
    rows = []
    for j, b in enumerate(bnd.tolist()):
        e = torch.zeros(D, dtype=torch.float64)
        e[j] = b
        e[(j + 1) % D] = (1 - b * b) ** 0.5
        rows.append((e @ Pi).float())
    x = torch.stack(rows)
    codes, _ = tq.quantize(x.to(DEV))
    ocodes, _ = oracle_quantizer(4, D, 42).quantize(x)
    adjudicate_codes(x, codes, ocodes, oracle_quantizer(4, D, 42))


def _shuffled_pool(g, B, Hkv, n, D, S, bw, prior):
    """Pages for ``prior[b] + n`` tokens per sequence in random order, full of random bytes."""
    P = int(sum((int(L) + n + S - 1) // S for L in prior)) + 5
    order = torch.randperm(P, generator=g)
    width = max((int(L) + n + S - 1) // S for L in prior) + 1
    table = torch.full((B, width), -1, dtype=torch.int32)
    nxt = 0
    for b in range(B):
        for t in range((int(prior[b]) + n + S - 1) // S):
            table[b, t] = int(order[nxt])
            nxt += 1
    nb = opk.packed_bytes(D, bw)
    pages = [torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g) for _ in range(2)]
    norms = [torch.randn(P, Hkv, S, generator=g).half() for _ in range(2)]
    return P, table, pages, norms


def _compare_append(got, before, want, src, oq, table, prior, n, bw, D):
    """Bytes outside the appended slots unchanged (always checked); inside them, the
    oracle's bytes, or codes that differ only by adjudicated flips."""
    S = got.shape[2]
    pos = oapp.positions(prior, n)
    pids, slots = oapp.locate(table, pos, S)
    written = torch.zeros(got.shape[:3], dtype=torch.bool)
    written[pids, :, slots] = True
    assert torch.equal(got[~written], before[~written]), "bytes outside the appended slots changed"
    if torch.equal(got, want):
        return 0
    gc = torch.from_numpy(opk.unpack(got.numpy(), bw, D))
    wc = torch.from_numpy(opk.unpack(want.numpy(), bw, D))
    return adjudicate_codes(src, gc[pids, :, slots].permute(0, 2, 1, 3), wc[pids, :, slots].permute(0, 2, 1, 3), oq)


@pytest.mark.parametrize("bw", [4, 6])
def test_append_config3_shape(bw):
    """BASELINE config 3 append: 16 new tokens per sequence, (16, 8, 16, 128) bf16, into
    shuffled pages holding random bytes; codes and norms against the pinned oracle scatter."""
    from winnow_amd import packed_backend as pb
    B, Hkv, n, D, S = 16, 8, 16, 128, 16
    g = torch.Generator().manual_seed(2)
    prior = torch.randint(0, 200, (B,), generator=g)            # tokens already stored per sequence
    P, table, (kp0, vp0), (kn0, vn0) = _shuffled_pool(g, B, Hkv, n, D, S, bw, prior)
    k = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
    v = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
    kq, vq = _q(bw, D, 42), _q(bw, D, 43)
    dk, dv, dkn, dvn = (t.to(DEV) for t in (kp0, vp0, kn0, vn0))
    pb.append_kv(k.to(DEV), v.to(DEV), kq, vq, dk, dv, dkn, dvn, table.to(DEV),
                 prior.to(torch.int32).to(DEV))
    okq, ovq = oracle_quantizer(bw, D, 42), oracle_quantizer(bw, D, 43)
    want = [kp0.clone(), vp0.clone()]
    wantn = [kn0.clone(), vn0.clone()]
    oapp.append(k, okq, want[0], wantn[0], table, prior.tolist())
    oapp.append(v, ovq, want[1], wantn[1], table, prior.tolist())
    flips = 0
    for got, before, w, src, oq in ((dk, kp0, want[0], k, okq), (dv, vp0, want[1], v, ovq)):
        flips += _compare_append(got.cpu(), before, w, src, oq, table, prior.tolist(), n, bw, D)
    print(f"config-3 append {bw} bits: {flips} adjudicated code flips", flush=True)
    pos = oapp.positions(prior.tolist(), n)
    pids, slots = oapp.locate(table, pos, S)
    for got, before, w, src in ((dkn, kn0, wantn[0], k), (dvn, vn0, wantn[1], v)):
        got = got.cpu()
        written = torch.zeros(got.shape, dtype=torch.bool)
        written[pids, :, slots] = True
        assert torch.equal(got[~written].view(torch.int16), before[~written].view(torch.int16))
        if not torch.equal(got.view(torch.int16), w.view(torch.int16)):
            n32 = src.float().norm(dim=-1).clamp(min=1e-10).permute(0, 2, 1)
            adjudicate_fp16_norms(n32, n32, got[pids, :, slots], w[pids, :, slots])


def test_append_k_only_leaves_v_alone():
    """v = None appends K alone (the C ABI's NULL V): K bytes as the oracle's, V pages and
    norms untouched."""
    from winnow_amd import packed_backend as pb
    B, Hkv, n, D, S, bw = 3, 4, 5, 128, 16, 4
    g = torch.Generator().manual_seed(21)
    prior = torch.tensor([14, 0, 33])                           # starts mid-page, empty, mid-page
    P, table, (kp0, vp0), (kn0, vn0) = _shuffled_pool(g, B, Hkv, n, D, S, bw, prior)
    k = torch.randn(B, Hkv, n, D, generator=g)
    kq = _q(bw, D, 42)
    dk, dv, dkn, dvn = (t.to(DEV) for t in (kp0, vp0, kn0, vn0))
    pb.append_kv(k.to(DEV), None, kq, None, dk, None, dkn, None, table.to(DEV), prior.to(torch.int32).to(DEV))
    want, wantn = kp0.clone(), kn0.clone()
    okq = oracle_quantizer(bw, D, 42)
    oapp.append(k, okq, want, wantn, table, prior.tolist())
    _compare_append(dk.cpu(), kp0, want, k, okq, table, prior.tolist(), n, bw, D)
    assert torch.equal(dv.cpu(), vp0) and torch.equal(dvn.cpu().view(torch.int16), vn0.view(torch.int16))


def test_append_plan_matches_append_kv():
    """An AppendPlan kept across steps (as PagedPackedCache keeps one per layer) writes the
    same bytes as append_kv, step after step, and refuses a step whose operands do not
    match the pages it was built on."""
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    B, Hkv, n, D, S, bw = 4, 8, 3, 128, 16, 6
    g = torch.Generator().manual_seed(33)
    prior = torch.tensor([0, 17, 40, 5])
    P, table, (kp0, vp0), (kn0, vn0) = _shuffled_pool(g, B, Hkv, 3 * n, D, S, bw, prior)
    kq, vq = _q(bw, D, 42), _q(bw, D, 43)
    a = [t.to(DEV) for t in (kp0, vp0, kn0, vn0)]
    b = [t.clone() for t in a]
    plan = pb.AppendPlan(kq, vq, *b[:2], *b[2:])
    dtab = table.to(DEV)
    for step in range(3):
        start = (prior + step * n).to(torch.int32).to(DEV)
        k = torch.randn(B, Hkv, n, D, generator=g).bfloat16().to(DEV)
        v = torch.randn(B, Hkv, n, D, generator=g).bfloat16().to(DEV)
        pb.append_kv(k, v, kq, vq, a[0], a[1], a[2], a[3], dtab, start)
        plan.launch(plan.bind(k, v, dtab, start))
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    k = torch.randn(B, Hkv, n, D, device=DEV)
    start = prior.to(torch.int32).to(DEV)
    with pytest.raises(pa.UnsupportedLayout, match="does not match pages"):
        plan.bind(k[:, :4], k[:, :4], dtab, start)                # fewer kv heads than the pages
    with pytest.raises(pa.UnsupportedLayout, match="no V"):
        plan.bind(k, None, dtab, start)                           # V pages without V
    with pytest.raises(pa.UnsupportedLayout, match="page_table"):
        plan.bind(k, k, dtab[:2], start)                          # table rows != batch


def test_pages_from_dense_matches_oracle():
    """pages_from_dense on the GPU (packed_attention.py:341-377): with the generator in the
    same state, the reference's page table; codes and fp16 norms of every stored token
    as the oracle's under the adjudication protocol; the unused bytes zero."""
    from oracle.attention import pages_from_dense as oracle_pages
    from winnow_amd import packed_attention as pa
    B, Hkv, D, S = 4, 4, 128, 16
    lens = [37, 0, 70, 16]
    g = torch.Generator().manual_seed(5)
    k = torch.randn(B, Hkv, max(lens), D, generator=g)
    v = torch.randn(B, Hkv, max(lens), D, generator=g)
    okq, ovq = oracle_quantizer(4, D, 42), oracle_quantizer(6, D, 43)
    want = oracle_pages(k, v, lens, okq, ovq, S, num_pages=16, generator=torch.Generator().manual_seed(9))
    got = pa.pages_from_dense(k.to(DEV), v.to(DEV), lens, _q(4, D, 42), _q(6, D, 43), S, num_pages=16,
                              generator=torch.Generator().manual_seed(9))
    assert torch.equal(got.page_table.cpu(), want.page_table) and torch.equal(got.page_table_host, want.page_table)
    assert torch.equal(got.seq_lens.cpu(), want.seq_lens)
    flips = 0
    for src, gp, wp, gn, wn, oq, bw in ((k, got.k_pages, want.k_pages, got.k_norms, want.k_norms, okq, 4),
                                        (v, got.v_pages, want.v_pages, got.v_norms, want.v_norms, ovq, 6)):
        gp, gn = gp.cpu(), gn.cpu()
        for b, L in enumerate(lens):
            for t in range((L + S - 1) // S):
                pid, lo, hi = int(want.page_table[b, t]), t * S, min((t + 1) * S, L)
                x = src[b, :, lo:hi]
                flips += adjudicate_codes(x, oapp_unpack(gp[pid, :, :hi - lo], bw, D),
                                          oapp_unpack(wp[pid, :, :hi - lo], bw, D), oq)
                n32 = x.float().norm(dim=-1).clamp(min=1e-10)
                adjudicate_fp16_norms(n32, n32, gn[pid, :, :hi - lo], wn[pid, :, :hi - lo])
                assert not gp[pid, :, hi - lo:].any() and not gn[pid, :, hi - lo:].view(torch.int16).any()
    print(f"pages_from_dense: {flips} adjudicated code flips", flush=True)


def oapp_unpack(packed, bw, D):
    return torch.from_numpy(opk.unpack(packed.numpy(), bw, D))


def test_append_rejects_before_launch():
    """Positions past the table row, pages outside the pool and V of another shape are
    refused before any launch, and the pool is left as it was (the reference raises in
    its gather, packed_backend.py:144)."""
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    B, Hkv, n, D, S, bw = 2, 2, 4, 128, 16, 4
    kq = _q(bw, D, 42)
    P = 4
    kp = torch.zeros(P, Hkv, S, 64, dtype=torch.uint8, device=DEV)
    kn = torch.zeros(P, Hkv, S, dtype=torch.float16, device=DEV)
    k = torch.randn(B, Hkv, n, D, device=DEV)
    table = torch.tensor([[0, 1], [2, -1]], dtype=torch.int32)
    ok = torch.tensor([10, 3], dtype=torch.int32)
    pb.append_kv(k, k, kq, kq, kp, kp.clone(), kn, kn.clone(), table.to(DEV), ok.to(DEV))
    for tab, start, why in ((table, torch.tensor([30, 3], dtype=torch.int32), "outside its 2-page"),
                            (table, torch.tensor([0, 14], dtype=torch.int32), "sequence 1"),
                            (torch.tensor([[0, 9], [2, -1]], dtype=torch.int32), ok + 4, "outside \\[0, 4\\)")):
        snap = kp.clone()
        with pytest.raises(pa.UnsupportedLayout, match=why):
            pb.append_kv(k, None, kq, None, kp, None, kn, None, tab.to(DEV), start.to(DEV))
        with pytest.raises(pa.UnsupportedLayout, match=why):      # same through host mirrors
            pb.append_kv(k, None, kq, None, kp, None, kn, None, tab.to(DEV), start.to(DEV),
                         page_table_host=tab, start_pos_host=start)
        assert torch.equal(kp, snap)
    with pytest.raises(pa.UnsupportedLayout, match="differs"):
        pb.append_kv(k, k[:, :, :2], kq, kq, kp, kp.clone(), kn, kn.clone(), table.to(DEV), ok.to(DEV))
    with pytest.raises(pa.UnsupportedLayout, match="norms"):
        pb.append_kv(k, None, kq, None, kp, None, kn[:, :1], None, table.to(DEV), ok.to(DEV))


def test_dequantize_matches_oracle_and_fp16_budget():
    """test_cache.py:26-60 on the device: packing lossless; fp16-norm error << quantization error."""
    from winnow_amd import packing
    D = 128
    for bw in (3, 4):
        tq = _q(bw, D, 42)
        g = torch.Generator().manual_seed(bw)
        x = torch.randn(2, 4, 64, D, generator=g)
        idx, norms = tq.quantize(x.to(DEV))
        assert torch.equal(packing.unpack(packing.pack(idx, bw), bw, D), idx)
        out = torch.empty(2, 4, 64, D, device=DEV)
        tq.dequantize_into(idx, norms.half(), out)
        ref = (tq.centroids.cpu()[idx.cpu().long()] @ tq.Pi.cpu()) * norms.cpu()[..., None]
        delta = (out.cpu() - ref).abs().max().item()
        quant_err = (ref - x).abs().max().item()
        assert delta / quant_err < 0.01, (delta, quant_err)


def test_paged_cache_prefill_then_decode():
    """PagedPackedCache over a GPU PagePool: prefill chunk then decode steps, two layers,
    bytes equal to the oracle's scatter and attention equal to the oracle on those pages."""
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    from winnow_amd.page_pool import PagePool
    from cases import to_host
    from oracle import attention as oa
    D, Hkv, Hq, S, bw, layers = 128, 4, 16, 16, 4, 2
    pool = PagePool(num_layers=layers, num_pages=64, num_kv_heads=Hkv, page_size=S,
                    nb_k=opk.packed_bytes(D, bw), nb_v=opk.packed_bytes(D, bw), device=DEV)
    kq, vq = _q(bw, D, 42), _q(bw, D, 43)
    owners = ["a", "b"]
    lengths = [0, 0]
    g = torch.Generator().manual_seed(5)
    for step, n in enumerate([37, 1, 1, 1]):
        for o, L in zip(owners, lengths):
            pool.ensure(o, L + n)
        cache = pb.PagedPackedCache(pool, owners, lengths, k_quant=kq, v_quant=vq, head_dim=D)
        for layer in range(layers):
            k = torch.randn(2, Hkv, n, D, generator=g).bfloat16().to(DEV)
            v = torch.randn(2, Hkv, n, D, generator=g).bfloat16().to(DEV)
            kv, _ = cache.update(k, v, layer)
            if n == 1:
                q = torch.randn(2, Hq, 1, D, generator=g)
                out = pb.winnow_packed_attention(None, q.to(DEV), kv, kv, None)[0]
                ref = oa.tiled_compressed_attention(q, to_host(kv), oa.default_scale(D))
                got = out.transpose(1, 2).float().cpu()
                assert torch.allclose(got, ref, atol=2e-3, rtol=1e-3)
        lengths = cache.lengths
    assert lengths == [40, 40]
    assert pb.BACKEND_COUNTS["hip_packed"] >= 6
    assert isinstance(kv, pa.PackedKV)
