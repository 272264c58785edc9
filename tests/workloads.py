"""BASELINE.json configs 2-5 as device workloads, for the full-size GPU parity tests and bench.py.

Each config's pool is filled by the product's append kernel (``wn_append_kv``, itself
held bit-exact to the pinned oracle by ``test_gpu_append.py``), so building one takes
seconds. The CPU generator seeded with the config seed draws the sequence lengths, the
page order, the outlier channels, the per-head scales and q. K and V (up to 4.4e9
normals per config) are drawn on the device from a generator seeded with the same
seed; a CPU draw of that many normals takes minutes. The first ``sample_tokens``
tokens of sequence 0 (all of it with ``full_check``, plus two random pages of three
other sequences) are kept on the host so their codes and norms can be recomputed by
the oracle.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

# BASELINE.json configs 2-5 (config 1, the CPU plumbing case, is tests/cases.config1_*).
CONFIGS = {
    2: dict(B=16, Hq=32, Hkv=8, D=128, L=32768, S=16, bwk=4, bwv=4, seed=1, table="contiguous",
            data="outliers"),
    3: dict(B=16, Hq=32, Hkv=8, D=128, L=32768, S=16, bwk=6, bwv=6, seed=2, table="contiguous",
            data="outliers"),
    4: dict(B=64, Hq=32, Hkv=8, D=128, L=None, S=16, bwk=4, bwv=4, seed=3, table="shuffled",
            data="normal"),
    5: dict(B=4, Hq=64, Hkv=8, D=128, L=131072, S=16, bwk=4, bwv=6, seed=4, table="contiguous",
            data="lognormal_heads"),
}

DATA = {
    "outliers": "K/V ~N(0,1) bf16, one channel in 128 (1 %) per kv head scaled x10, chosen by seeded randperm",
    "normal": "K/V ~N(0,1) bf16",
    "lognormal_heads": "K/V ~N(0,1) bf16 times a per-(sequence, kv head) std ~ LogNormal(0, 0.5), K and V drawn "
                       "separately",
}


@dataclass
class Workload:
    cfg: int
    c: dict
    lens: list
    q: torch.Tensor          # (B, Hq, 1, D) bf16 on the device
    kvs: list                # PackedKV handles over `copies` identical pools
    quants: tuple            # (k TurboQuantMSE, v TurboQuantMSE) on the device
    sample: tuple            # host bf16 (1, Hkv, sample_tokens, D) K and V of sequence 0
    table: torch.Tensor      # host (B, max_pages) int32
    extra: list = None       # (b, page column, host K, host V) of re-checked random pages


def lengths(c, g) -> list:
    if c["L"] is None:
        return torch.randint(512, 65537, (c["B"],), generator=g).tolist()
    return [c["L"]] * c["B"]


def build(cfg: int, dev, copies: int = 1, sample_tokens: int = 256, full_check: bool = False) -> Workload:
    from winnow_amd import packed_attention as pa
    from winnow_amd import packed_backend as pb
    from winnow_amd.packing import packed_bytes
    from winnow_amd.quantizer import get_quantizer

    c = CONFIGS[cfg]
    B, Hq, Hkv, D, S = c["B"], c["Hq"], c["Hkv"], c["D"], c["S"]
    g = torch.Generator().manual_seed(c["seed"])
    gd = torch.Generator(device=dev).manual_seed(c["seed"])
    lens = lengths(c, g)
    need = [-(-L // S) for L in lens]
    P = sum(need)
    order = torch.randperm(P, generator=g) if c["table"] == "shuffled" else torch.arange(P)
    table = torch.full((B, max(need)), -1, dtype=torch.int32)
    off = 0
    for b in range(B):
        table[b, :need[b]] = order[off:off + need[b]].to(torch.int32)
        off += need[b]
    n_out = max(1, round(0.01 * D))
    k_ch = [torch.randperm(D, generator=g)[:n_out] for _ in range(Hkv)]
    v_ch = [torch.randperm(D, generator=g)[:n_out] for _ in range(Hkv)]
    head_std = torch.exp(torch.randn(B, Hkv, 2, generator=g) * 0.5)       # LogNormal(0, 0.5)
    q = torch.randn(B, Hq, 1, D, generator=g).to(dev, torch.bfloat16)

    kq = get_quantizer(c["bwk"], D, dev, 42)
    vq = get_quantizer(c["bwv"], D, dev, 42)
    nbk, nbv = packed_bytes(D, c["bwk"]), packed_bytes(D, c["bwv"])
    kp = torch.zeros(P, Hkv, S, nbk, dtype=torch.uint8, device=dev)
    vp = torch.zeros(P, Hkv, S, nbv, dtype=torch.uint8, device=dev)
    kn = torch.zeros(P, Hkv, S, dtype=torch.float16, device=dev)
    vn = torch.zeros(P, Hkv, S, dtype=torch.float16, device=dev)
    dtable = table.to(dev)
    zero = torch.zeros(1, dtype=torch.int32)
    sample = None
    # pages re-checked beside sequence 0, picked by a generator of their own so the
    # workload's draws are the same with and without the check
    gx = torch.Generator().manual_seed(c["seed"] + 7)
    pick = int(torch.randint(B, (1,), generator=gx))
    extra_b = sorted({B // 2, B - 1, pick} - {0}) if full_check else []
    extra = []
    for b in range(B):
        L = lens[b]
        k = torch.randn(1, Hkv, L, D, generator=gd, device=dev)
        v = torch.randn(1, Hkv, L, D, generator=gd, device=dev)
        if c["data"] == "outliers":
            for h in range(Hkv):
                k[:, h, :, k_ch[h].to(dev)] *= 10
                v[:, h, :, v_ch[h].to(dev)] *= 10
        elif c["data"] == "lognormal_heads":
            k *= head_std[b, :, 0].to(dev)[None, :, None, None]
            v *= head_std[b, :, 1].to(dev)[None, :, None, None]
        k, v = k.bfloat16(), v.bfloat16()
        if b == 0:
            n0 = L if full_check else sample_tokens
            sample = (k[:, :, :n0].cpu(), v[:, :, :n0].cpu())
        if b in extra_b:
            for col in torch.randperm(need[b], generator=gx)[:2].tolist():
                t0, t1 = col * S, min(col * S + S, L)
                extra.append((b, col, k[:, :, t0:t1].cpu(), v[:, :, t0:t1].cpu()))
        pb.append_kv(k, v, kq, vq, kp, vp, kn, vn, dtable[b:b + 1], zero.to(dev),
                     page_table_host=table[b:b + 1], start_pos_host=zero)
        del k, v
    seq = torch.tensor(lens, dtype=torch.int32)
    kvs = []
    for i in range(copies):
        t = (kp, kn, vp, vn) if i == 0 else tuple(x.clone() for x in (kp, kn, vp, vn))
        kvs.append(pa.PackedKV(t[0], t[1], t[2], t[3], dtable, seq.to(dev), pa.Quantizer.from_tq(kq),
                               pa.Quantizer.from_tq(vq), D, seq_lens_host=seq, page_table_host=table))
    torch.cuda.synchronize()
    return Workload(cfg, c, lens, q, kvs, (kq, vq), sample, table, extra)


def kv_bytes(lens, Hkv, nbk, nbv) -> int:
    """Algorithmic bytes of one decode step: sum_b L_b * Hkv * ((NB_K + 2) + (NB_V + 2))
    (the reference's traffic model, bench_packed_attention.py:91-98, at mixed widths)."""
    return sum(lens) * Hkv * ((nbk + 2) + (nbv + 2))


def requantize(w: Workload, kv=None) -> dict:
    """Codes and fp16 norms of the kept tokens (sequence 0's first ones, or all of it and
    the random pages with ``full_check``) recomputed by the CPU oracle against the pool
    bytes: counts checked and adjudicated flips (any other difference raises)."""
    from adjudicate import adjudicate_codes, adjudicate_fp16_norms
    from oracle import packing as opk
    from oracle.quantizer import get_quantizer as oq

    kv = kv or w.kvs[0]
    c, D, S = w.c, w.c["D"], w.c["S"]
    sets = [(0, 0, w.sample[0], w.sample[1])] + list(w.extra or [])
    out = {"vectors": 0, "code_flips": 0, "norm_flips": 0, "random_pages": len(w.extra or [])}
    for b, col, ks, vs in sets:
        n = ks.shape[2]
        ids = w.table[b, col:col - (-n // S)].long()
        for src, bw, pages, norms in ((ks, c["bwk"], kv.k_pages, kv.k_norms), (vs, c["bwv"], kv.v_pages, kv.v_norms)):
            quant = oq(bw, D, 42)
            codes, n32 = quant.quantize(src)                             # (1, Hkv, n, D), (1, Hkv, n)
            stored = pages[ids.to(pages.device)].cpu()                   # (pages, Hkv, S, NB)
            stored = torch.from_numpy(opk.unpack(stored.numpy(), bw, D))
            stored = stored.permute(1, 0, 2, 3).reshape(1, stored.shape[1], -1, D)[:, :, :n]
            out["code_flips"] += adjudicate_codes(src, stored, codes, quant)
            h = norms[ids.to(norms.device)].cpu().permute(1, 0, 2).reshape(1, norms.shape[1], -1)[:, :, :n]
            out["norm_flips"] += adjudicate_fp16_norms(n32, n32, h, n32.half())
            out["vectors"] += src.shape[1] * n
    return out


def requantize_flips(w: Workload, kv=None) -> int:
    """Adjudicated code flips of ``requantize``."""
    return requantize(w, kv)["code_flips"]
