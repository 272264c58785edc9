"""GPU parity at head dims 16, 32 and 256: the reference kernel takes any power of two
>= 16 (packed_attention_triton.py:160-172), the reference's quantizer, packing and
dequantize any head_dim (cache.py:88-131, packing.py:27-89).

At these head dims the packed decode runs the vector-ALU scan for every pair of
widths, the dense decode the vector-ALU dense scan for bf16, fp16 and fp32 pages,
and the append / quantize the vector-ALU float64 kernel. Each is checked as its
head_dim 64 / 128 counterpart is: packed decode against the oracle's tiled path
(fp32 within 2e-3 abs / 1e-3 rel, rows of empty sequences exactly zero), dense
decode against the float64 oracle on the same page values, codes and norms bit-exact
against the oracle under the adjudication protocol, packed bytes equal to the
oracle's packer, and bytes outside the appended slots unchanged.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from adjudicate import adjudicate_codes, adjudicate_fp16_norms
from cases import build, to_device
from oracle import append as oapp
from oracle import attention as oa
from oracle import packing as opk
from oracle.quantizer import get_quantizer as oracle_quantizer

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-3, 1e-3
HEAD_DIMS = (16, 32, 256)
WIDTHS = (2, 3, 4, 5, 6, 8)


def _check(got, ref, lens):
    got = got.float().cpu()
    assert torch.isfinite(got).all()
    err = (got - ref.float()).abs().max().item()
    assert torch.allclose(got, ref.float(), atol=ATOL, rtol=RTOL), f"max abs err {err:.3e}"
    for b, L in enumerate(lens):
        if L == 0:
            assert (got[b] == 0).all()
    return err


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_packed_decode_every_width_pair(D):
    """All 36 (bw_k, bw_v) pairs at n_rep 4, ragged lengths with an empty sequence,
    the library's plan and fixed splits 1 and 3."""
    from winnow_amd import packed_attention as pa
    lens = (0, 5, 40, 333)
    scale = oa.default_scale(D)
    pairs = [(k, v) for k in WIDTHS for v in WIDTHS]
    if D == 256:  # the long rows: one pair per K width, plus the tuned pairs of head_dim 128
        pairs = [(2, 3), (3, 5), (4, 4), (4, 6), (5, 2), (6, 6), (6, 4), (8, 8), (4, 8)]
    for bwk, bwv in pairs:
        print(f"D={D} widths {bwk}/{bwv}", flush=True)
        q, kv = build(900 + D + 10 * bwk + bwv, len(lens), 8, 2, D, lens, 16, bwk, bw_v=bwv)
        ref = oa.tiled_compressed_attention(q, kv, scale)
        kvd = to_device(kv, DEV)
        for splits in (None, 1, 3):
            got = pa.packed_decode_attention(q.to(DEV), kvd, scale, num_splits=splits, out_dtype=torch.float32)
            _check(got, ref, lens)


@pytest.mark.parametrize("D,Hq,Hkv,S", [(16, 8, 8, 16), (32, 34, 2, 32), (256, 16, 1, 16), (256, 40, 2, 64),
                                         (32, 128, 4, 16)])
def test_packed_decode_head_groups(D, Hq, Hkv, S):
    """n_rep 1, 16, 17 (virtual groups of a prime count), 20 and 32, page sizes 16-64,
    lengths around page and chunk edges; bf16 output."""
    from winnow_amd import packed_attention as pa
    lens = (1, 15, 16, 17, 64, 65, 700)
    print(f"D={D} Hq={Hq} Hkv={Hkv} S={S}", flush=True)
    q, kv = build(1000 + D + Hq, len(lens), Hq, Hkv, D, lens, S, 4)
    scale = oa.default_scale(D)
    ref = oa.tiled_compressed_attention(q, kv, scale)
    kvd = to_device(kv, DEV)
    got = pa.packed_decode_attention(q.to(DEV), kvd, scale, out_dtype=torch.float32)
    _check(got, ref, lens)
    got16 = pa.packed_decode_attention(q.to(DEV).bfloat16(), kvd, scale)
    assert got16.dtype == torch.bfloat16
    assert torch.allclose(got16.float().cpu(), ref.float(), atol=2e-2, rtol=2e-2)


def _dense_pages(seed, lens, Hkv, S, D, dtype):
    g = torch.Generator().manual_seed(seed)
    need = [(L + S - 1) // S for L in lens]
    P = sum(need) + 2
    kp = torch.randn(P, Hkv, S, D, generator=g).to(dtype)
    vp = torch.randn(P, Hkv, S, D, generator=g).to(dtype)
    order = torch.randperm(P, generator=g).tolist()
    table = torch.full((len(lens), max(max(need), 1)), -1, dtype=torch.int32)
    for b, L in enumerate(lens):
        for t in range(need[b]):
            table[b, t] = order.pop()
    return kp, vp, table, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", HEAD_DIMS)
def test_dense_decode(D, dtype):
    """bf16, fp16 and fp32 pages on the vector-ALU dense scan (fixed splits), n_rep 1, 4
    and 17, against the float64 oracle on the same page values."""
    from winnow_amd import packed_attention as pa
    lens = (0, 1, 17, 64, 300)
    for Hq, Hkv in ((8, 8), (16, 4), (34, 2)):
        print(f"dense D={D} {dtype} Hq={Hq} Hkv={Hkv}", flush=True)
        kp, vp, table, sl = _dense_pages(D + Hq, lens, Hkv, 16, D, dtype)
        q = torch.randn(len(lens), Hq, 1, D, generator=torch.Generator().manual_seed(Hq))
        scale = 1.0 / D ** 0.5
        ref = oa.dense_paged_attention_f64(q, kp, vp, table, sl, scale)
        kv = pa.DenseKV(kp.to(DEV), vp.to(DEV), table.to(DEV), sl.to(DEV), D)
        for splits in (None, 2):
            got = pa.dense_decode_attention(q.to(DEV), kv, scale, num_splits=splits, out_dtype=torch.float32).cpu()
            err = (got.double() - ref).abs().max().item()
            assert torch.allclose(got.double(), ref, atol=ATOL, rtol=RTOL), err
            assert bool((got[0] == 0).all())


def _q(bw, D, seed):
    from winnow_amd.quantizer import get_quantizer
    return get_quantizer(bw, D, DEV, seed)


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_quantize_pack_dequantize(D):
    """Codes and norms against the oracle quantizer (zero, one-hot and tiny vectors
    included), packed bytes against the oracle packer with the round trip, and the
    dequantized rows against the oracle's dequantize of the same codes."""
    from winnow_amd import packing
    for bw in WIDTHS:
        print(f"quantize D={D} bw={bw}", flush=True)
        g = torch.Generator().manual_seed(D + bw)
        x = torch.randn(1000, D, generator=g)
        x[0] = 0
        x[1, :] = 0
        x[1, 3] = 2.0
        x[2] *= 1e-30
        tq, oq = _q(bw, D, 42), oracle_quantizer(bw, D, 42)
        assert torch.equal(tq.Pi.cpu(), oq.Pi) and torch.equal(tq.boundaries.cpu(), oq.boundaries)
        codes, norms = tq.quantize(x.to(DEV))
        ocodes, onorms = oq.quantize(x)
        assert adjudicate_codes(x, codes, ocodes, oq) <= max(2, codes.numel() // 20000)
        assert torch.allclose(norms.cpu(), onorms, rtol=2e-6, atol=0)
        assert int(codes[0, 0]) == int((oq.boundaries < 0).sum())
        packed = packing.pack(codes, bw)
        assert np.array_equal(packed.cpu().numpy(), opk.pack(codes.cpu().numpy(), bw))
        assert torch.equal(packing.unpack(packed, bw, D), codes)
        out = torch.empty(1000, D, device=DEV)
        tq.dequantize_into(codes, norms.half(), out)
        ref = (tq.centroids.cpu()[codes.cpu().long()].double() @ tq.Pi.cpu().double()) * \
            norms.half().cpu().double()[:, None]
        assert torch.allclose(out.cpu().double(), ref, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("D", HEAD_DIMS)
def test_append_into_shuffled_pages(D):
    """wn_append_kv at 4 and 6 bits: starts mid-page, an empty sequence, spans of two
    pages, into shuffled pages of random bytes; codes and fp16 norms against the
    oracle's scatter, everything outside the appended slots unchanged."""
    from winnow_amd import packed_backend as pb
    B, Hkv, n, S = 3, 2, 20, 16
    for bw in (4, 6):
        print(f"append D={D} bw={bw}", flush=True)
        g = torch.Generator().manual_seed(D * 10 + bw)
        prior = [14, 0, 33]
        P = sum((L + n + S - 1) // S for L in prior) + 3
        order = torch.randperm(P, generator=g)
        width = max((L + n + S - 1) // S for L in prior) + 1
        table = torch.full((B, width), -1, dtype=torch.int32)
        nxt = 0
        for b in range(B):
            for t in range((prior[b] + n + S - 1) // S):
                table[b, t] = int(order[nxt])
                nxt += 1
        nb = opk.packed_bytes(D, bw)
        kp0 = torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g)
        vp0 = torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g)
        kn0 = torch.randn(P, Hkv, S, generator=g).half()
        vn0 = torch.randn(P, Hkv, S, generator=g).half()
        k = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
        v = torch.randn(B, Hkv, n, D, generator=g).bfloat16()
        kq, vq = _q(bw, D, 42), _q(bw, D, 43)
        dk, dv, dkn, dvn = (t.to(DEV) for t in (kp0, vp0, kn0, vn0))
        pb.append_kv(k.to(DEV), v.to(DEV), kq, vq, dk, dv, dkn, dvn, table.to(DEV),
                     torch.tensor(prior, dtype=torch.int32).to(DEV))
        okq, ovq = oracle_quantizer(bw, D, 42), oracle_quantizer(bw, D, 43)
        pos = oapp.positions(prior, n)
        pids, slots = oapp.locate(table, pos, S)
        for got, gotn, before, beforen, src, oq in ((dk, dkn, kp0, kn0, k, okq), (dv, dvn, vp0, vn0, v, ovq)):
            want, wantn = before.clone(), beforen.clone()
            oapp.append(src, oq, want, wantn, table, prior)
            got, gotn = got.cpu(), gotn.cpu()
            written = torch.zeros(got.shape[:3], dtype=torch.bool)
            written[pids, :, slots] = True
            assert torch.equal(got[~written], before[~written])
            assert torch.equal(gotn[~written].view(torch.int16), beforen[~written].view(torch.int16))
            if not torch.equal(got, want):
                gc = torch.from_numpy(opk.unpack(got.numpy(), bw, D))
                wc = torch.from_numpy(opk.unpack(want.numpy(), bw, D))
                flips = adjudicate_codes(src, gc[pids, :, slots].permute(0, 2, 1, 3),
                                         wc[pids, :, slots].permute(0, 2, 1, 3), oq)
                assert flips <= max(2, src.numel() // 20000)
            if not torch.equal(gotn.view(torch.int16), wantn.view(torch.int16)):
                n32 = src.float().norm(dim=-1).clamp(min=1e-10).permute(0, 2, 1)
                adjudicate_fp16_norms(n32, n32, gotn[pids, :, slots], wantn[pids, :, slots])


@pytest.mark.parametrize("D", [32, 256])
def test_paged_cache_round_trip(D):
    """Append through the paged cache, then decode over the pages it wrote and
    reconstruct the history (the standalone unpack + dequantize path at these head
    dims): decode within tolerance of the oracle on the same pages, history equal to
    the oracle's dequantize."""
    from cases import to_host
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    bw, B, Hkv, Hq, n, S = 4, 2, 2, 8, 40, 16
    g = torch.Generator().manual_seed(D)
    P = 2 * ((n + S - 1) // S) + 1
    table = torch.arange(2 * ((n + S - 1) // S), dtype=torch.int32).view(B, -1)
    nb = opk.packed_bytes(D, bw)
    kp = torch.zeros(P, Hkv, S, nb, dtype=torch.uint8, device=DEV)
    vp, kn, vn = kp.clone(), torch.zeros(P, Hkv, S, dtype=torch.float16, device=DEV), None
    vn = kn.clone()
    k = torch.randn(B, Hkv, n, D, generator=g)
    v = torch.randn(B, Hkv, n, D, generator=g)
    kq, vq = _q(bw, D, 42), _q(bw, D, 43)
    pb.append_kv(k.to(DEV), v.to(DEV), kq, vq, kp, vp, kn, vn, table.to(DEV), torch.zeros(B, dtype=torch.int32).to(DEV))
    lens = torch.tensor([n, n - 7], dtype=torch.int32)
    kv = pa.PackedKV(kp, kn, vp, vn, table.to(DEV), lens.to(DEV), pa.Quantizer(kq.Pi, kq.centroids, bw),
                     pa.Quantizer(vq.Pi, vq.centroids, bw), D, seq_lens_host=lens, page_table_host=table)
    q = torch.randn(B, Hq, 1, D, generator=g)
    scale = oa.default_scale(D)
    ref = oa.tiled_compressed_attention(q, to_host(kv), scale)
    got = pa.packed_decode_attention(q.to(DEV), kv, scale, out_dtype=torch.float32)
    _check(got, ref, [n, n - 7])
    hist = pb.dequantize_history(kv, kp, kn, kv.k_quant, 1, torch.float32)
    okq = oa.OracleQuant(kq.Pi.cpu(), kq.centroids.cpu(), bw)
    rows = kp.cpu()[table[1].long()].transpose(0, 1).reshape(Hkv, -1, nb)[:, :n - 7]
    nrm = kn.cpu()[table[1].long()].transpose(0, 1).reshape(Hkv, -1)[:, :n - 7]
    codes = torch.from_numpy(opk.unpack(rows.numpy(), bw, D)).long()
    want = (okq.centroids[codes].double() @ okq.Pi.double()) * nrm.double()[..., None]
    assert torch.allclose(hist[0].cpu().double(), want, atol=1e-5, rtol=1e-5)
