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


def tf32_class_reference(q: torch.Tensor, kv, scale: float, rnd=round11) -> torch.Tensor:
    """float64 decode attention whose score and value operands are first rounded as the
    TF32-class scan rounds them (``rnd``): the rotated, scaled query (in log2 units, as
    the scan carries it) and both codebooks to 11 significant bits. The p n_V
    operand's rounding (2^-12 relative per term) is left out; everything else is exact.
    The query is rotated in float64 before its rounding, the scan rounds its fp32
    rotation: the two can differ by one step of the 11-bit grid where they fall on
    either side of a halfway point. The algebra is the oracle's decode
    (packed_attention.py:260-334 in float64)."""
    B, Hq, _, D = q.shape
    n_rep = Hq // kv.num_kv_heads
    log2e = 1.0 / math.log(2.0)
    ck_t, cv_t = rnd(kv.k_quant.centroids), rnd(kv.v_quant.centroids)
    q_rot = (q[:, :, 0].double() @ kv.k_quant.Pi.double().T) * scale
    q_r = rnd(q_rot * log2e) / log2e
    out = torch.zeros(B, Hq, 1, D, dtype=torch.float64)
    heads = torch.arange(Hq) // n_rep
    for b in range(B):
        if int(kv.seq_lens[b]) == 0:
            continue
        pk, nk = oa._gather_history(kv.k_pages, kv.k_norms, kv, b)
        pv, nv = oa._gather_history(kv.v_pages, kv.v_norms, kv, b)
        ck = ck_t[oa.unpack_t(pk, kv.k_quant.bit_width, D).long()] * nk.double()[..., None]
        cv = cv_t[oa.unpack_t(pv, kv.v_quant.bit_width, D).long()] * nv.double()[..., None]
        s = (q_r[b][:, None, :] @ ck[heads].transpose(-1, -2))[:, 0]          # (Hq, L)
        a = torch.softmax(s, -1)[:, None, :] @ cv[heads]                        # (Hq, 1, D)
        out[b] = a @ kv.v_quant.Pi.double()
    return out
