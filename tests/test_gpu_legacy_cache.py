"""GPU checks of the contiguous packed cache (``winnow_amd.cache``), the drop-in for the
reference's ``TQPackedLayer`` / ``TQPackedCache`` (turboquant_kv/cache.py:154-419).

* Stored bytes: after a prefill and decode steps, every packed code equals the
  oracle quantizer's (``oracle.quantizer``, pinned to the reference's constants) under
  the adjudication protocol, packed as the oracle packer packs, fp16 norms alike; with
  outlier channels the split follows the top-RMS channels of the first keys
  (cache.py:196-201) and each group matches its own quantizer (seeds 42 and 43).
* Returned history: the float64 closed form ``(c[codes] @ Pi) * n`` of the stored
  codes, within 2e-5 of the largest value on the fp32 paths (fused kernel, chunked
  standalone kernels) and within the fast mode's 2e-3 for ``triton_tf32``; the
  outlier channels land in their columns.
* The cache protocol: overflow raises, ``reset``, mask sizes, accounting
  (``persistent_bytes``, ``effective_bits``).
* A tiny Qwen2 generating greedily with ``TQPackedCache`` (8-bit, the reference's
  quantized reference, test_packed_model.py:44-61) gives the tokens of the paged
  engine with the HIP decode, logits within 1e-3 of their scale.
"""
from __future__ import annotations

import pytest
import torch

from adjudicate import adjudicate_codes, adjudicate_fp16_norms
from oracle import packing as opk
from oracle.quantizer import get_quantizer as oracle_quantizer

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _closed_form(codes_u8, norms16, q):
    """float64 (c[codes] @ Pi) * n of stored codes (B, H, L, D) and fp16 norms (B, H, L)."""
    c = q.centroids.cpu().double()[codes_u8.long()]
    return (c @ q.Pi.cpu().double()) * norms16.double()[..., None]


def _stored(group, L, bw, dim):
    codes = torch.from_numpy(opk.unpack(group.codes[:, :, :L].cpu().numpy(), bw, dim))
    return codes, group.norms[:, :, :L].cpu()


def _fill(layer, xs_k, xs_v):
    out = None
    for k, v in zip(xs_k, xs_v):
        out = layer.update(k.to(DEV), v.to(DEV))
    return out


@pytest.mark.parametrize("backend,tol", [("auto", 2e-3), ("triton_fp32", 2e-5), ("native_cuda_fp32", 2e-5),
                                         ("torch_fp32", 2e-5), ("triton_tf32", 2e-3)])
def test_layer_bytes_and_history(backend, tol):
    from winnow_amd.cache import TQPackedLayer
    B, H, D, bw = 2, 3, 128, 4
    g = torch.Generator().manual_seed(5)
    steps = [37, 1, 1, 5]
    xs_k = [torch.randn(B, H, n, D, generator=g) for n in steps]
    xs_v = [torch.randn(B, H, n, D, generator=g) for n in steps]
    layer = TQPackedLayer(D, bw, DEV, max_cache_len=50, kernel_backend=backend)
    k_hist, v_hist = _fill(layer, xs_k, xs_v)
    L = sum(steps)
    assert layer.get_seq_length() == L and k_hist.shape == (B, H, L, D) and k_hist.dtype == torch.float32
    assert layer.last_dispatch_decision.backend == ("chunked" if backend == "torch_fp32" else "fused")
    oq = oracle_quantizer(bw, D, 42)
    for xs, grp, hist in ((xs_k, layer._k_groups[0], k_hist), (xs_v, layer._v_groups[0], v_hist)):
        x = torch.cat(xs, dim=2)
        codes, norms = _stored(grp, L, bw, D)
        ocodes, onorms = oq.quantize(x)
        assert adjudicate_codes(x, codes, ocodes, oq) <= 2
        if not torch.equal(norms.view(torch.int16), onorms.half().view(torch.int16)):
            adjudicate_fp16_norms(onorms, onorms, norms, onorms.half())
        want = _closed_form(codes, norms, oq)
        err = (hist.cpu().double() - want).abs().max().item()
        assert err <= tol * want.abs().max().item(), (backend, err)


@pytest.mark.parametrize("D,n_out,bw,bw_out", [(128, 8, 4, 8), (64, 16, 3, 6), (128, 0, 6, 0), (32, 0, 4, 0)])
def test_layer_outlier_channels_and_other_widths(D, n_out, bw, bw_out):
    """Outlier channels (regular 120 / 48 channels: the run-time head_dim kernels), and
    the chunked path at head dims without the fused kernel."""
    from winnow_amd.cache import TQPackedLayer
    B, H = 1, 2
    g = torch.Generator().manual_seed(D + n_out)
    k0 = torch.randn(B, H, 20, D, generator=g)
    if n_out:
        k0[..., 5] *= 12.0      # make some channels the high-RMS ones
        k0[..., 17] *= 9.0
    xs_k = [k0, torch.randn(B, H, 1, D, generator=g)]
    xs_v = [torch.randn(B, H, 20, D, generator=g), torch.randn(B, H, 1, D, generator=g)]
    layer = TQPackedLayer(D, bw, DEV, max_cache_len=21, num_outlier_channels=n_out, outlier_bits=bw_out,
                          chunk=8, allow_tf32=False)
    k_hist, v_hist = _fill(layer, xs_k, xs_v)
    L = 21
    assert layer.last_dispatch_decision.backend == ("fused" if (D == 128 and not n_out) else "chunked")
    if n_out:
        rms = k0.pow(2).mean(dim=(0, 1, 2)).sqrt()
        mask = torch.zeros(D, dtype=torch.bool)
        mask[rms.topk(n_out).indices] = True
        assert torch.equal(layer._outlier_channels.cpu(), mask) and bool(mask[5]) and bool(mask[17])
        groups = [(~mask, bw, D - n_out, 42, 0), (mask, bw_out, n_out, 43, 1)]
    else:
        mask = torch.zeros(D, dtype=torch.bool)
        groups = [(~mask, bw, D, 42, 0)]
    for xs, side, hist in ((xs_k, layer._k_groups, k_hist), (xs_v, layer._v_groups, v_hist)):
        x = torch.cat(xs, dim=2)
        want = torch.empty(B, H, L, D, dtype=torch.float64)
        for chan, w, dim, seed, gi in groups:
            oq = oracle_quantizer(w, dim, seed)
            xp = x[..., chan]
            codes, norms = _stored(side[gi], L, w, dim)
            ocodes, onorms = oq.quantize(xp)
            assert adjudicate_codes(xp, codes, ocodes, oq) <= 2
            if not torch.equal(norms.view(torch.int16), onorms.half().view(torch.int16)):
                adjudicate_fp16_norms(onorms, onorms, norms, onorms.half())
            want[..., chan] = _closed_form(codes, norms, oq)
        err = (hist.cpu().double() - want).abs().max().item()
        assert err <= 2e-5 * want.abs().max().item(), err


@pytest.mark.parametrize("backend", ["triton_fp32", "triton_tf32", "native_cuda_fp32"])
def test_explicit_backend_with_outlier_channels_takes_the_chunked_path(backend):
    """The reference uses the requested kernel only without outlier channels and otherwise
    dequantizes on its chunked path (cache.py:245-246): a caller passing kernel_backend
    together with num_outlier_channels gets the history, not an error."""
    from winnow_amd.cache import TQPackedLayer
    B, H, D, n_out, bw, bw_out = 1, 2, 128, 8, 4, 8
    g = torch.Generator().manual_seed(77)
    k0 = torch.randn(B, H, 12, D, generator=g)
    k0[..., 3] *= 10.0
    xs_k = [k0, torch.randn(B, H, 1, D, generator=g)]
    xs_v = [torch.randn(B, H, 12, D, generator=g), torch.randn(B, H, 1, D, generator=g)]
    layer = TQPackedLayer(D, bw, DEV, max_cache_len=16, num_outlier_channels=n_out, outlier_bits=bw_out,
                          kernel_backend=backend)
    k_hist, v_hist = _fill(layer, xs_k, xs_v)
    assert layer.last_dispatch_decision.backend == "chunked"
    mask = layer._outlier_channels.cpu()
    for xs, side, hist in ((xs_k, layer._k_groups, k_hist), (xs_v, layer._v_groups, v_hist)):
        x = torch.cat(xs, dim=2)
        want = torch.empty(B, H, 13, D, dtype=torch.float64)
        for chan, w, dim, seed, gi in ((~mask, bw, D - n_out, 42, 0), (mask, bw_out, n_out, 43, 1)):
            codes, norms = _stored(side[gi], 13, w, dim)
            want[..., chan] = _closed_form(codes, norms, oracle_quantizer(w, dim, seed))
        err = (hist.cpu().double() - want).abs().max().item()
        assert err <= 2e-5 * want.abs().max().item(), err


def test_protocol_and_accounting():
    from winnow_amd.cache import TQPackedLayer
    B, H, D, bw, M = 2, 2, 128, 4, 10
    layer = TQPackedLayer(D, bw, DEV, max_cache_len=M)
    assert layer.persistent_bytes() == 0 and layer.get_seq_length() == 0
    k = torch.randn(B, H, 6, D, device=DEV, dtype=torch.bfloat16)
    kh, vh = layer.update(k, k)
    assert kh.dtype == torch.bfloat16 and kh.shape == (B, H, 6, D)
    assert layer.get_mask_sizes(1) == (7, 0) and layer.get_max_length() == M
    assert layer.persistent_bytes() == 2 * B * H * M * (64 + 2)
    assert layer.persistent_bytes_used() == int(2 * B * H * M * 66 * 6 / M)
    assert layer.transient_bytes() == 2 * B * H * 6 * D * 2
    with pytest.raises(RuntimeError, match="overflow"):
        layer.update(k, k)
    layer.reset()
    assert layer.get_seq_length() == 0
    layer.update(k[:, :, :2], k[:, :, :2])
    assert layer.get_seq_length() == 2
    with pytest.raises(ValueError, match="kernel_backend"):
        TQPackedLayer(D, bw, DEV, max_cache_len=M, kernel_backend="cuda")
    with pytest.raises(RuntimeError, match="requested triton_fp32"):
        bad = TQPackedLayer(64, bw, DEV, max_cache_len=M, kernel_backend="triton_fp32")
        bad.update(torch.randn(1, 1, 2, 64, device=DEV), torch.randn(1, 1, 2, 64, device=DEV))


def test_tiny_qwen_generates_the_paged_engines_tokens():
    """The reference's quantized reference (TQPackedCache under SDPA, 8-bit, K and V on
    the seed-42 quantizer) against the paged engine with the HIP decode on the same
    quantizer: same greedy tokens, logits within 1e-3 of their scale."""
    from tiny_qwen import prompts, tiny_qwen
    from winnow_amd import packed_backend as pb
    from winnow_amd.cache import TQPackedCache
    from winnow_amd.engine import Engine, EngineConfig, Request
    model = tiny_qwen(DEV)
    prompt, new = prompts(1, seed=7, lo=30, hi=31)[0], 10
    model.config._attn_implementation = "sdpa"
    cache = TQPackedCache(model.config, bit_width=8, max_cache_len=len(prompt) + new, device=DEV,
                          allow_tf32=False)
    ids = torch.tensor([prompt], device=DEV)
    ref_toks, ref_logits = [], []
    with torch.no_grad():
        for _ in range(new):
            out = model(input_ids=ids, past_key_values=cache, use_cache=True, logits_to_keep=1)
            lg = out.logits[0, -1].float()
            t = int(lg.argmax())
            ref_toks.append(t)
            ref_logits.append(lg)
            ids = torch.tensor([[t]], device=DEV)
    assert cache.get_seq_length() == len(prompt) + new - 1
    assert abs(cache.effective_bits() - (8 * 128 + 16) / 128) < 1e-12
    model.config._attn_implementation = pb.ATTN_NAME
    pool = pb.make_pool(model.config, bit_width=8, num_pages=16, page_size=16, device=DEV)
    kq, vq = pb.quantizers_for(model.config, 8, DEV)
    eng = Engine(model, pool, kq, vq, pb.head_dim_of(model.config), config=EngineConfig(prefill_chunk=512))
    got = []
    eng.on_logits = lambda reqs, lg: got.append(lg[0].clone())
    req = Request("r", prompt, new)
    eng.submit(req)
    eng.run_until_idle()
    assert req.generated == ref_toks
    scale = max(1.0, max(x.abs().max().item() for x in ref_logits))
    for a, b in zip(got[-new:], ref_logits):
        assert (a.float() - b).abs().max().item() < 1e-3 * scale
