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


@pytest.mark.parametrize("bw", [4, 6])
def test_append_config3_shape(bw):
    """BASELINE config 3 append: 16 new tokens per sequence, (16, 8, 16, 128) bf16, into shuffled pages."""
    from winnow_amd import packed_backend as pb
    B, Hkv, n, D, S = 16, 8, 16, 128, 16
    g = torch.Generator().manual_seed(2)
    prior = torch.randint(0, 200, (B,), generator=g)            # tokens already stored per sequence
    P = int(sum((int(L) + n + S - 1) // S for L in prior)) + 5
    order = torch.randperm(P, generator=g)
    width = max((int(L) + n + S - 1) // S for L in prior)
    table = torch.full((B, width), -1, dtype=torch.int32)
    nxt = 0
    for b in range(B):
        for t in range((int(prior[b]) + n + S - 1) // S):
            table[b, t] = int(order[nxt])
            nxt += 1
    k = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
    v = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
    nb = opk.packed_bytes(D, bw)
    ref_kp = torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g)   # pre-existing bytes
    ref_vp = torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g)
    ref_kn = torch.randn(P, Hkv, S, generator=g).half()
    ref_vn = torch.randn(P, Hkv, S, generator=g).half()
    kq, vq = _q(bw, D, 42), _q(bw, D, 43)
    dk, dv, dkn, dvn = (t.to(DEV) for t in (ref_kp, ref_vp, ref_kn, ref_vn))
    pb.append_kv(k.to(DEV), v.to(DEV), kq, vq, dk, dv, dkn, dvn, table.to(DEV),
                 prior.to(torch.int32).to(DEV))
    okq, ovq = oracle_quantizer(bw, D, 42), oracle_quantizer(bw, D, 43)
    oapp.append(k, okq, ref_kp, ref_kn, table, prior.tolist())
    oapp.append(v, ovq, ref_vp, ref_vn, table, prior.tolist())
    for got, want, src, oq in ((dk, ref_kp, k, okq), (dv, ref_vp, v, ovq)):
        got = got.cpu()
        if not torch.equal(got, want):
            # identical bytes except where an adjudicated code flip changed the packing
            gc = torch.from_numpy(opk.unpack(got.numpy(), bw, D))
            wc = torch.from_numpy(opk.unpack(want.numpy(), bw, D))
            pos = torch.tensor([[int(L) + i for i in range(n)] for L in prior])
            pids = torch.gather(table.long(), 1, pos // S)
            slots = pos % S
            sel_g = gc[pids, :, slots].permute(0, 2, 1, 3)
            sel_w = wc[pids, :, slots].permute(0, 2, 1, 3)
            adjudicate_codes(src, sel_g, sel_w, oq)
            mask = torch.ones(P, Hkv, S, dtype=torch.bool)
            mask[pids, :, slots] = False
            assert torch.equal(got[mask], want[mask]), "bytes outside the appended slots changed"
    for got, want, src in ((dkn, ref_kn, k), (dvn, ref_vn, v)):
        got = got.cpu()
        if not torch.equal(got.view(torch.int16), want.view(torch.int16)):
            n32 = src.float().norm(dim=-1).clamp(min=1e-10)
            pos = torch.tensor([[int(L) + i for i in range(n)] for L in prior])
            pids = torch.gather(table.long(), 1, pos // S)
            slots = pos % S
            adjudicate_fp16_norms(n32.permute(0, 2, 1), n32.permute(0, 2, 1),
                                  got[pids, :, slots], want[pids, :, slots])


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
