"""A float64 decode of TF32-class operands: the reference the TF32-class scan
(``allow_tf32=True``) is checked against where TF32 rounding itself exceeds the fp32
bar. Test infrastructure; pinned on the CPU by ``test_tf32_reference.py`` (with the
rounding off it is the float64 oracle ``reconstruct_attention_f64``, and the rounding
is fp16's)."""
from __future__ import annotations

import math

import torch

from oracle import attention as oa


def round11(x: torch.Tensor, bits: int = 11) -> torch.Tensor:
    """x rounded to ``bits`` significant bits, ties to even (fp16's significand at 11,
    no range limit)."""
    m, e = torch.frexp(x.double())
    return torch.ldexp(torch.round(m * (1 << bits)) / (1 << bits), e)


def tf32_class_reference(q: torch.Tensor, kv, scale: float, rnd=round11,
                         q_log2: torch.Tensor | None = None) -> torch.Tensor:
    """float64 attention whose score and value operands are first rounded as the
    TF32-class scans (decode with ``allow_tf32=True``, and the fused prefill) round
    them (``rnd``): the rotated, scaled query (in log2 units, as the scans carry it)
    and both codebooks to 11 significant bits. The p n_V operand's rounding (2^-12
    relative per term) is left out; everything else is exact. The query is rotated in
    float64 before its rounding, the scans round their fp32 rotation: the two can
    differ by one step of the 11-bit grid where they fall on either side of a halfway
    point. q is (B, Hq, Q, D): query i of a sequence of length L sees keys
    j <= L - Q + i and a query that sees none gives 0, as in the oracle's
    reconstruct_attention (packed_attention.py:198-231, here in float64). ``q_log2``
    (B, Hq, Q, D), when given, replaces the float64 rotation: the scan's own fp32
    rotated query in log2 units (scale log2(e) q Pi_K^T), which the scan rounds as
    ``rnd`` does, so that no component can round the other way."""
    B, Hq, Q, D = q.shape
    log2e = 1.0 / math.log(2.0)
    ck_t, cv_t = rnd(kv.k_quant.centroids), rnd(kv.v_quant.centroids)
    if q_log2 is None:
        q_log2 = (q.double() @ kv.k_quant.Pi.double().T) * (scale * log2e)    # (B, Hq, Q, D)
    q_r = rnd(q_log2.double()) / log2e
    out = torch.zeros(B, Hq, Q, D, dtype=torch.float64)
    n_rep = Hq // kv.num_kv_heads
    heads = torch.arange(Hq) // n_rep
    for b in range(B):
        L = int(kv.seq_lens[b])
        if L == 0:
            continue
        pk, nk = oa._gather_history(kv.k_pages, kv.k_norms, kv, b)
        pv, nv = oa._gather_history(kv.v_pages, kv.v_norms, kv, b)
        ck = ck_t[oa.unpack_t(pk, kv.k_quant.bit_width, D).long()] * nk.double()[..., None]
        cv = cv_t[oa.unpack_t(pv, kv.v_quant.bit_width, D).long()] * nv.double()[..., None]
        s = q_r[b] @ ck[heads].transpose(-1, -2)                                # (Hq, Q, L)
        allowed = torch.arange(L)[None, :] <= (L - Q + torch.arange(Q))[:, None]
        s = s.masked_fill(~allowed[None], float("-inf"))
        p = torch.softmax(s, -1).nan_to_num(0.0)
        a = p @ cv[heads]                                                       # (Hq, Q, D)
        out[b] = (a @ kv.v_quant.Pi.double()) * allowed.any(-1)[None, :, None]
    return out


def prefill_q_log2(workspace: torch.Tensor, B: int, Hq: int, Hkv: int, Q: int) -> torch.Tensor:
    """The fused prefill's own fp32 rotated queries (log2 units), (B, Hq, Q, D) on the
    CPU, read back from the start of the caller-owned workspace of a
    ``packed_prefill_attention`` call: rows (sequence, kv head, qi n_rep + h), padded
    to a multiple of 64 per kv head."""
    n_rep = Hq // Hkv
    nrp = -(-n_rep * Q // 64) * 64
    rows = workspace[:B * Hkv * nrp * 128 * 4].view(torch.float32).view(B, Hkv, nrp, 128)[:, :, :n_rep * Q]
    return rows.reshape(B, Hkv, Q, n_rep, 128).permute(0, 1, 3, 2, 4).reshape(B, Hq, Q, 128).cpu()
