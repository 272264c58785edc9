"""GPU parity of the fused dequantization (``wn_tq_dequant``, ``wn_dequantize_history``).

The reference's ``tq_dequant`` (``kernel.py:33-115``, ``csrc/tq_dequant.cu:125-215``)
computes ``out = (centroids[unpack(packed)] @ Pi) * norm`` and writes it once in the
output dtype; its paged caller gathers a sequence's pages first
(``packed_backend.py:192-208``). The check is against the float64 closed form on
codes and fp16 norms made by the CPU oracle (``oracle.quantizer``, ``oracle.packing``):
fp32 output within 2e-5 of the largest output (the matrix-core product is carried
as bf16 hi + lo pairs, error below 2^-16 per term); bf16 output within one bf16 step of
the float64 value plus that absolute error, and equal to its rounding for over 98 %
of the elements (the rest are near-ties and elements near zero, 0.4 % measured). Layouts: every width, a cache
buffer sliced to its first L positions (``kernel.py:46-51``), shuffled pool pages.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import packing as opk
from oracle.quantizer import get_quantizer as oracle_quantizer

DEV = "cuda"


def _rows(bw, D, shape, seed):
    """(packed uint8 (*shape, NB), fp16 norms (*shape), float64 reference (*shape, D))."""
    tq = oracle_quantizer(bw, D, 42)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, D, generator=g) * (1.0 + 3.0 * torch.rand(*shape, 1, generator=g))
    idx, norms = tq.quantize(x)
    packed = torch.from_numpy(opk.pack(idx.numpy(), bw))
    n16 = norms.half()
    ref = (tq.centroids.double()[idx.long()] @ tq.Pi.double()) * n16.double()[..., None]
    return packed, n16, ref, tq


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [2, 3, 4, 5, 6, 8])
def test_tq_dequant_matches_the_closed_form(bw):
    from winnow_amd.kernel import tq_dequant
    D = 128
    packed, n16, ref, tq = _rows(bw, D, (2, 4, 77), 300 + bw)
    c, Pi = tq.centroids.to(DEV), tq.Pi.to(DEV)
    out32 = torch.empty(2, 4, 77, D, device=DEV)
    tq_dequant(packed.to(DEV), n16.to(DEV), c, Pi, bw, D, out=out32)
    err = (out32.cpu().double() - ref).abs().max().item()
    assert err <= 2e-5 * ref.abs().max().item(), (err, ref.abs().max().item())
    # default bf16 output: the float64 value rounded once, up to one bf16 step at ties
    got = tq_dequant(packed.to(DEV), n16.to(DEV), c, Pi, bw, D).cpu()
    assert got.dtype == torch.bfloat16
    # within one bf16 step of the float64 value, plus the absolute error allowed in fp32
    # (it decides the rounding of elements near zero and at near-ties)
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp(min=1e-30))) - 7)
    assert bool(((got.double() - ref).abs() <= ulp + 2e-5 * ref.abs().max()).all())
    want = ref.float().to(torch.bfloat16)
    assert (got == want).float().mean().item() > 0.98


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [4, 6])
def test_tq_dequant_fast_mode_stays_in_the_tf32_class(bw):
    """allow_tf32=True: one fp16 product per term, within 2e-3 of the largest output
    (the reference documents its tf32 path as faster and measurably less accurate)."""
    from winnow_amd.kernel import tq_dequant
    D = 128
    packed, n16, ref, tq = _rows(bw, D, (2, 4, 77), 400 + bw)
    out = torch.empty(2, 4, 77, D, device=DEV)
    tq_dequant(packed.to(DEV), n16.to(DEV), tq.centroids.to(DEV), tq.Pi.to(DEV), bw, D, out=out, allow_tf32=True)
    err = (out.cpu().double() - ref).abs().max().item()
    assert err <= 2e-3 * ref.abs().max().item(), err
    assert err > 0.0


@pytest.mark.gpu
@pytest.mark.parametrize("bw,shape", [(4, (1, 1, 5)), (3, (1,)), (4, (4, 3, 17011)), (3, (3, 2, 23459))])
def test_tq_dequant_short_and_multi_pass_inputs(bw, shape):
    """Fewer rows than one 32-row pass, and more rows than the persistent grid covers
    in one pass per wave (up to 512 work-groups x 4 waves x 32 rows = 65,536), so every
    wave runs its pipeline over several passes; the last pass is partial. Checked on
    the first and last rows and a seeded sample in between."""
    from winnow_amd.kernel import tq_dequant
    D = 128
    tq = oracle_quantizer(bw, D, 42)
    g = torch.Generator().manual_seed(11 + bw)
    N = int(np.prod(shape))
    nb = D * bw // 8
    packed = torch.randint(0, 256, (*shape, nb), dtype=torch.uint8, generator=g)
    n16 = (torch.rand(*shape, generator=g) * 8 + 0.5).half()
    out = torch.empty(*shape, D, device=DEV)
    tq_dequant(packed.to(DEV), n16.to(DEV), tq.centroids.to(DEV), tq.Pi.to(DEV), bw, D, out=out)
    rows = torch.unique(torch.cat([torch.arange(min(N, 2048)), torch.arange(max(0, N - 2048), N),
                                   torch.randint(0, N, (4096,), generator=g)]))
    pk = packed.reshape(N, nb)[rows].numpy()
    idx = torch.from_numpy(opk.unpack(pk, bw, D)).long()
    ref = (tq.centroids.double()[idx] @ tq.Pi.double()) * n16.reshape(N)[rows].double()[:, None]
    got = out.reshape(N, D)[rows.to(DEV)].cpu().double()
    err = (got - ref).abs().max().item()
    assert err <= 2e-5 * ref.abs().max().item(), err


@pytest.mark.gpu
def test_tq_dequant_reads_a_sliced_cache_buffer():
    """A (B, H, MAXLEN, NB) buffer sliced to its first L positions is read in place."""
    from winnow_amd.kernel import tq_dequant
    D, bw, MAXLEN, L = 128, 4, 96, 61
    packed, n16, ref, tq = _rows(bw, D, (3, 2, MAXLEN), 7)
    buf, nbuf = packed.to(DEV), n16.to(DEV)
    view, nview = buf[:, :, :L], nbuf[:, :, :L]
    assert not view.is_contiguous()
    c, Pi = tq.centroids.to(DEV), tq.Pi.to(DEV)
    a = tq_dequant(view, nview, c, Pi, bw, D, out=torch.empty(3, 2, L, D, device=DEV))
    b = tq_dequant(view.contiguous(), nview.contiguous(), c, Pi, bw, D, out=torch.empty(3, 2, L, D, device=DEV))
    assert torch.equal(a, b)
    err = (a.cpu().double() - ref[:, :, :L]).abs().max().item()
    assert err <= 2e-5 * ref.abs().max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("bw", [3, 4, 6])
def test_history_from_shuffled_pages_matches_the_oracle_gather(bw):
    """packed_backend.dequantize_history (fused) against the oracle's page gather + closed form."""
    from cases import build, to_device
    from oracle import attention as oa
    from winnow_amd import packed_backend as pb
    _, kv = build(900 + bw, 3, 8, 4, 128, (0, 45, 300), 16, bw)
    dkv = to_device(kv, DEV)
    for b in range(3):
        L = int(kv.seq_lens[b])
        for pages, norms, quant in ((kv.k_pages, kv.k_norms, kv.k_quant), (kv.v_pages, kv.v_norms, kv.v_quant)):
            dp = dkv.k_pages if pages is kv.k_pages else dkv.v_pages
            dn = dkv.k_norms if norms is kv.k_norms else dkv.v_norms
            dq = dkv.k_quant if quant is kv.k_quant else dkv.v_quant
            got = pb.dequantize_history(dkv, dp, dn, dq, b, torch.float32)
            assert got.shape == (1, 4, L, 128)
            if L == 0:
                continue
            p, n = oa._gather_history(pages, norms, kv, b)
            idx = oa.unpack_t(p, bw, 128)
            ref = (quant.centroids.double()[idx.long()] @ quant.Pi.double()) * n.double()[..., None]
            err = (got[0].cpu().double() - ref).abs().max().item()
            assert err <= 2e-5 * ref.abs().max().item(), (b, err)


@pytest.mark.gpu
def test_dequant_rejects_what_it_does_not_compile():
    from winnow_amd import _lib
    from winnow_amd.kernel import tq_dequant
    tq = oracle_quantizer(4, 64, 42)
    packed = torch.zeros(5, 32, dtype=torch.uint8, device=DEV)
    with pytest.raises(_lib.WinnowHipError):
        tq_dequant(packed, torch.ones(5, dtype=torch.float16, device=DEV), tq.centroids.to(DEV), tq.Pi.to(DEV), 4, 64)
    with pytest.raises(ValueError):
        tq_dequant(packed, torch.ones(4, dtype=torch.float16, device=DEV), tq.centroids.to(DEV), tq.Pi.to(DEV), 4, 64)


def test_dequant_has_no_host_path():
    from winnow_amd.kernel import tq_dequant
    from winnow_amd.packing import UnsupportedDevice
    tq = oracle_quantizer(4, 128, 42)
    with pytest.raises(UnsupportedDevice):
        tq_dequant(torch.zeros(3, 64, dtype=torch.uint8), torch.ones(3, dtype=torch.float16), tq.centroids, tq.Pi, 4, 128)


def test_closed_form_reference_is_the_oracle_dequantize():
    """The float64 reference above equals the oracle's own dequantize to fp32 rounding."""
    packed, n16, ref, tq = _rows(4, 128, (2, 9), 5)
    idx = torch.from_numpy(opk.unpack(packed.numpy(), 4, 128))
    got = tq.dequantize(idx, n16.float())
    assert np.allclose(got.double().numpy(), ref.numpy(), rtol=0, atol=1e-6 * ref.abs().max().item())
