"""GPU parity at the BASELINE.json shapes (configs 2-5), on the default balanced plan.

The reference keeps its long and batched cases for the GPU
(test_packed_attention_triton.py:51-68) and checks outputs before timing
(bench_packed_attention.py:157-166). Here each config runs at full size with the
plan ``wn_decode_plan`` chooses, where the batch has many more 64-token chunks than
resident waves, so every wave walks a run of chunks across (sequence, kv head)
boundaries (asserted). For each config:

* the first, middle and last sequences are held to the CPU oracle
  (``tiled_compressed_attention`` on the same pages) at 2e-3 max-abs / 1e-3 relative
  of the fp32 output, and their relative L2 against the float64 oracle is reported;
* the whole batch equals the one-split-per-(sequence, kv head) plan to fp32
  summation-order noise (a property that holds at any size);
* the codes of sequence 0's first 256 tokens, recomputed by the CPU oracle, equal the
  pool bytes under the adjudication protocol.

Config 4 is also run with three zero-length sequences spliced into the middle of the
batch, so the balanced scan's skip over sequences without chunks runs inside a wave's
share.
"""
from __future__ import annotations

import pytest
import torch

import workloads
from cases import to_host
from oracle import attention as oa

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL, RTOL = 2e-3, 1e-3


def _pa():
    from winnow_amd import packed_attention as pa
    return pa


def _chunks(lens, Hkv):
    return Hkv * sum(-(-L // 64) for L in lens)


def _same_plan_noise(a, b):
    scale = max(1.0, b.abs().max().item())
    return (a - b).abs().max().item() / scale


def _oracle_check(q, kv, got, seqs, scale):
    sub = to_host(kv, seqs)
    qs = q.float().cpu()[seqs]
    ref = oa.tiled_compressed_attention(qs, sub, scale)
    g = got.cpu()[seqs]
    err = (g - ref).abs().max().item()
    assert torch.isfinite(g).all()
    assert torch.allclose(g, ref, atol=ATOL, rtol=RTOL), f"sequences {seqs}: max abs err {err:.3e}"
    f64 = oa.reconstruct_attention_f64(qs, sub, scale)
    rel = ((g.double() - f64).norm() / f64.norm()).item()
    return err, rel


@pytest.mark.parametrize("cfg", [2, 3, 4, 5])
def test_baseline_config_on_the_balanced_plan(cfg):
    pa = _pa()
    print(f"BASELINE config {cfg}: building", flush=True)
    w = workloads.build(cfg, DEV)
    kv, q = w.kvs[0], w.q
    B, Hkv, D = len(w.lens), w.c["Hkv"], w.c["D"]
    scale = oa.default_scale(D)
    pps, ns = pa.plan_for(q, kv)
    chunks = _chunks(w.lens, Hkv)
    print(f"config {cfg}: plan {ns} waves x {pps}, {chunks} chunks", flush=True)
    assert pps == 0, "the row scan's balanced plan"
    assert chunks > 4 * ns, (chunks, ns)               # every wave scans several chunks
    got = pa.packed_decode_attention(q, kv, scale, out_dtype=torch.float32)
    one = pa.packed_decode_attention(q, kv, scale, num_splits=1, out_dtype=torch.float32)
    noise = _same_plan_noise(got, one)
    assert noise < 1e-5, noise
    seqs = [0, B // 2, B - 1]
    err, rel = _oracle_check(q, kv, got, seqs, scale)
    flips = workloads.requantize_flips(w)
    print(f"config {cfg}: max|err| {err:.2e} rel-L2 vs f64 {rel:.2e}, plans differ by {noise:.1e}, "
          f"{flips} adjudicated code flips", flush=True)
    assert rel < 1e-5
    if cfg == 4:
        _zero_length_splice(w, got, scale)


def _zero_length_splice(w, got, scale):
    """Config 4 with empty sequences inserted at rows 5, 6 and 40: those rows are exactly 0
    and every other row equals the unspliced batch's."""
    pa = _pa()
    kv = w.kvs[0]
    B = len(w.lens)
    at = (5, 6, 40)
    order = list(range(B))
    for i, r in enumerate(at):
        order.insert(r + i, -1)
    table = torch.full((len(order), w.table.shape[1]), -1, dtype=torch.int32)
    lens = torch.zeros(len(order), dtype=torch.int32)
    for row, b in enumerate(order):
        if b >= 0:
            table[row], lens[row] = w.table[b], w.lens[b]
    q = torch.stack([w.q[b] if b >= 0 else torch.zeros_like(w.q[0]) for b in order])
    kv2 = pa.PackedKV(kv.k_pages, kv.k_norms, kv.v_pages, kv.v_norms, table.to(DEV), lens.to(DEV),
                      kv.k_quant, kv.v_quant, kv.head_dim, seq_lens_host=lens, page_table_host=table)
    pps, ns = pa.plan_for(q, kv2)
    assert pps == 0 and _chunks(lens.tolist(), kv.num_kv_heads) > ns
    out = pa.packed_decode_attention(q, kv2, scale, out_dtype=torch.float32)
    real = [row for row, b in enumerate(order) if b >= 0]
    assert (out[[row for row, b in enumerate(order) if b < 0]] == 0).all()
    assert _same_plan_noise(out[real], got) < 1e-5


def test_config2_dense_matched_baseline_on_the_balanced_plan():
    """The matched unquantized decode at config 2's shape: bf16 pages, balanced plan with
    many chunks per wave, the first and last sequences (cut to 2048 tokens: the float64
    oracle gathers every page on the host) against the float64 oracle, and the full
    batch against the one-split plan."""
    pa = _pa()
    c = workloads.CONFIGS[2]
    B, Hq, Hkv, D, S, L = c["B"], c["Hq"], c["Hkv"], c["D"], c["S"], c["L"]
    P = B * L // S
    g = torch.Generator(device=DEV).manual_seed(99)
    kp = torch.randn(P, Hkv, S, D, generator=g, device=DEV, dtype=torch.bfloat16)
    vp = torch.randn(P, Hkv, S, D, generator=g, device=DEV, dtype=torch.bfloat16)
    table = torch.arange(P, dtype=torch.int32).view(B, L // S)
    lens = torch.full((B,), L, dtype=torch.int32)
    q = torch.randn(B, Hq, 1, D, generator=torch.Generator().manual_seed(1)).to(DEV, torch.bfloat16)
    kv = pa.DenseKV(kp, vp, table.to(DEV), lens.to(DEV), D, seq_lens_host=lens, page_table_host=table)
    pps, ns = pa.dense_plan_for(q, kv)
    assert pps == 0 and _chunks([L] * B, Hkv) > 4 * ns
    scale = oa.default_scale(D)
    got = pa.dense_decode_attention(q, kv, scale, out_dtype=torch.float32)
    one = pa.dense_decode_attention(q, kv, scale, num_splits=1, out_dtype=torch.float32)
    assert _same_plan_noise(got, one) < 1e-5
    cut, seqs = 2048, [0, B - 1]
    ct = torch.full((2,), cut, dtype=torch.int32)
    sub = pa.DenseKV(kp, vp, table[seqs].to(DEV), ct.to(DEV), D, seq_lens_host=ct, page_table_host=table[seqs])
    part = pa.dense_decode_attention(q[seqs], sub, scale, out_dtype=torch.float32).cpu()
    used = table[seqs, :cut // S]
    ref = oa.dense_paged_attention_f64(q[seqs].float().cpu(), kp[used.flatten().long().to(DEV)].cpu(),
                                       vp[used.flatten().long().to(DEV)].cpu(),
                                       torch.arange(used.numel(), dtype=torch.int32).view(2, -1), ct, scale)
    assert torch.allclose(part.double(), ref, atol=ATOL, rtol=RTOL), (part.double() - ref).abs().max()
