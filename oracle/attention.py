"""Oracle: compressed-domain attention over paged packed KV -- test infrastructure only.

CPU (torch fp32) restatement of ``turboquant_kv/packed_attention.py``:

* ``reconstruct_attention``           packed_attention.py:208-231
* ``explicit_compressed_attention``   packed_attention.py:234-257
* ``tiled_compressed_attention``      packed_attention.py:260-311 (the reference's CPU
  production decode path, selected off-GPU by packed_backend.py:181-184; this is
  the function ``bench.py`` times as the CPU baseline)
* ``_online_update`` / ``_safe_exp`` / ``merge_partials``  packed_attention.py:314-334
* ``pages_from_dense``                packed_attention.py:341-377
* ``reconstruct_attention_f64``       float64 variant used for relative-L2 reports
  (the float64 operator check of model_contract.py:158-221)
* ``dense_paged_attention_f64``       attention over unquantized paged K/V in float64:
  the page gather + offset-causal softmax of packed_backend.py:229-246 (``_dense_sdpa``),
  which the dense decode (packed_attention_triton.py:190-201) must match

The algebraic pieces (``kv_head_for``, ``rotate_query``, ``rotate_output``,
``_online_update``, ``merge_partials``) are module attributes so tests can plant
the reference's seven mutants here, on the CPU, and prove the checks catch them.

``dense_paged_attention_f64`` is pinned against torch's scaled_dot_product_attention
over the contiguous K/V the pages were scattered from (no paging on that side),
with ragged, empty and one-token sequences, shuffled tables and GQA groups, and
against planted paging mistakes.

Pinned by (``tests/test_oracle_attention.py``): the three implementations agree
with each other and with an unquantized softmax attention over the dequantized
K/V computed in float64 by plain numpy; empty / one-page / tail pages; rows with
no visible key are exactly zero; scores in the thousands stay finite; zero
vectors; GQA head groups; a hand-built non-symmetric rotation; and each of the
reference's seven seeded mutants misses by >= 100x the tolerance
(test_packed_attention.py:209-264).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from oracle.packing import packed_bytes


@dataclass(frozen=True)
class OracleQuant:
    """What the operator reads of a quantizer (packed_attention.py:59-69)."""
    Pi: torch.Tensor
    centroids: torch.Tensor
    bit_width: int

    @classmethod
    def from_tq(cls, tq) -> "OracleQuant":
        return cls(tq.Pi, tq.centroids, tq.bit_width)


@dataclass
class OracleKV:
    """Paged packed K/V (packed_attention.py:72-92)."""
    k_pages: torch.Tensor          # (P, Hkv, S, NBK) uint8
    k_norms: torch.Tensor          # (P, Hkv, S) fp16
    v_pages: torch.Tensor
    v_norms: torch.Tensor
    page_table: torch.Tensor       # (B, max_pages) int32, -1 padded
    seq_lens: torch.Tensor         # (B,) int32
    k_quant: OracleQuant
    v_quant: OracleQuant
    head_dim: int
    extra: dict = field(default_factory=dict)

    @property
    def page_size(self) -> int:
        return self.k_pages.shape[2]

    @property
    def num_kv_heads(self) -> int:
        return self.k_pages.shape[1]


def unpack_t(packed: torch.Tensor, bit_width: int, head_dim: int) -> torch.Tensor:
    """torch restatement of packing.unpack (packing.py:67-89), used on the hot CPU loop."""
    if bit_width == 8:
        return packed
    lead, nbytes = packed.shape[:-1], packed.shape[-1]
    if bit_width == 4:
        flat = packed.reshape(-1, nbytes)
        out = torch.empty(flat.shape[0], head_dim, dtype=torch.uint8)
        out[:, 0::2] = flat & 0x0F
        out[:, 1::2] = flat >> 4
        return out.reshape(*lead, head_dim)
    sh = torch.arange(8, dtype=torch.uint8)
    bits = (packed.reshape(-1, nbytes).unsqueeze(-1) >> sh) & 1
    bits = bits.reshape(-1, nbytes * 8)[:, :head_dim * bit_width].reshape(-1, head_dim, bit_width)
    w = 1 << torch.arange(bit_width, dtype=torch.int16)
    return (bits.to(torch.int16) * w).sum(-1).to(torch.uint8).reshape(*lead, head_dim)


def pack_t(idx: torch.Tensor, bit_width: int) -> torch.Tensor:
    """torch restatement of packing.pack (packing.py:37-64)."""
    if bit_width == 8:
        return idx.contiguous()
    D = idx.shape[-1]
    nb = packed_bytes(D, bit_width)
    if bit_width == 4:
        flat = idx.reshape(-1, D)
        return (flat[:, 0::2] | (flat[:, 1::2] << 4)).reshape(*idx.shape[:-1], nb).contiguous()
    sh = torch.arange(bit_width, dtype=torch.uint8)
    bits = ((idx.reshape(-1, D).unsqueeze(-1) >> sh) & 1).reshape(-1, nb, 8)
    w = 1 << torch.arange(8, dtype=torch.int16)
    return (bits.to(torch.int16) * w).sum(-1).to(torch.uint8).reshape(*idx.shape[:-1], nb).contiguous()


class ContractError(ValueError):
    pass


def check(q: torch.Tensor, kv) -> None:
    """The metadata checks of check_contract (packed_attention.py:114-163) the oracle relies on."""
    if q.dim() != 4:
        raise ContractError("q must be (B, Hq, Q, D)")
    B, Hq, _, D = q.shape
    if D != kv.head_dim or Hq % kv.num_kv_heads:
        raise ContractError("head_dim / GQA mismatch")
    P, S = kv.k_pages.shape[0], kv.page_size
    lens = kv.seq_lens.to("cpu", torch.int64)
    if (lens < 0).any() or (lens > kv.page_table.shape[1] * S).any():
        raise ContractError("seq_lens out of range")
    table = kv.page_table.to("cpu", torch.int64)
    for b in range(B):
        ids = table[b, :(int(lens[b]) + S - 1) // S]
        if ((ids < 0) | (ids >= P)).any():
            raise ContractError(f"sequence {b} references a page outside [0, {P})")


def kv_head_for(q_head: torch.Tensor, n_rep: int) -> torch.Tensor:
    """GQA: query head h reads kv head h // n_rep (packed_attention.py:168-170)."""
    return q_head // n_rep


def rotate_query(q: torch.Tensor, Pi: torch.Tensor) -> torch.Tensor:
    """q Pi^T (packed_attention.py:173-175)."""
    return q @ Pi.T


def rotate_output(a_rot: torch.Tensor, Pi: torch.Tensor) -> torch.Tensor:
    """a Pi (packed_attention.py:178-180)."""
    return a_rot @ Pi


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def _centroids(pages, quant, head_dim):
    idx = unpack_t(pages, quant.bit_width, head_dim)
    return quant.centroids.index_select(0, idx.reshape(-1).to(torch.int32)).view(idx.shape)


def _gather_history(pages, norms, kv, b):
    L = int(kv.seq_lens[b])
    S = kv.page_size
    ids = kv.page_table[b, :(L + S - 1) // S].long()
    p = pages[ids].permute(1, 0, 2, 3).reshape(pages.shape[1], -1, pages.shape[3])
    n = norms[ids].permute(1, 0, 2).reshape(norms.shape[1], -1)
    return p[:, :L], n[:, :L]


def _causal_limit(kv, Q):
    pos = torch.arange(Q)
    return kv.seq_lens.long()[:, None] - Q + pos[None, :]


def reconstruct_attention(q: torch.Tensor, kv, scale: float) -> torch.Tensor:
    """Dequantize each history, then masked softmax attention in fp32."""
    check(q, kv)
    B, Hq, Q, D = q.shape
    n_rep = Hq // kv.num_kv_heads
    out = torch.zeros(B, Hq, Q, D, dtype=torch.float32)
    limit = _causal_limit(kv, Q)
    heads = kv_head_for(torch.arange(Hq), n_rep)
    for b in range(B):
        L = int(kv.seq_lens[b])
        if L == 0:
            continue
        pk, nk = _gather_history(kv.k_pages, kv.k_norms, kv, b)
        pv, nv = _gather_history(kv.v_pages, kv.v_norms, kv, b)
        k = (_centroids(pk, kv.k_quant, D) @ kv.k_quant.Pi) * nk.float()[..., None]
        v = (_centroids(pv, kv.v_quant, D) @ kv.v_quant.Pi) * nv.float()[..., None]
        k, v = k[heads], v[heads]
        s = (q[b].float() @ k.transpose(-1, -2)) * scale
        allowed = torch.arange(L)[None, :] <= limit[b][:, None]
        s = s.masked_fill(~allowed[None], float("-inf"))
        p = torch.softmax(s, dim=-1).nan_to_num(0.0)
        out[b] = (p @ v) * allowed.any(-1)[None, :, None]
    return out


def explicit_compressed_attention(q: torch.Tensor, kv, scale: float) -> torch.Tensor:
    """One full softmax per row in the quantizer bases, no x_hat history."""
    check(q, kv)
    B, Hq, Q, D = q.shape
    n_rep = Hq // kv.num_kv_heads
    heads = kv_head_for(torch.arange(Hq), n_rep)
    out = torch.zeros(B, Hq, Q, D, dtype=torch.float32)
    limit = _causal_limit(kv, Q)
    for b in range(B):
        L = int(kv.seq_lens[b])
        if L == 0:
            continue
        pk, nk = _gather_history(kv.k_pages, kv.k_norms, kv, b)
        pv, nv = _gather_history(kv.v_pages, kv.v_norms, kv, b)
        ck = _centroids(pk, kv.k_quant, D)[heads]
        cv = _centroids(pv, kv.v_quant, D)[heads]
        q_rot = rotate_query(q[b].float(), kv.k_quant.Pi)
        s = (q_rot @ ck.transpose(-1, -2)) * nk.float()[heads][:, None, :] * scale
        allowed = torch.arange(L)[None, :] <= limit[b][:, None]
        s = s.masked_fill(~allowed[None], float("-inf"))
        p = torch.softmax(s, dim=-1).nan_to_num(0.0)
        a_rot = (p * nv.float()[heads][:, None, :]) @ cv
        out[b] = rotate_output(a_rot, kv.v_quant.Pi) * allowed.any(-1)[None, :, None]
    return out


def tiled_compressed_attention(q: torch.Tensor, kv, scale: float,
                               split_pages: int | None = None,
                               page_range: tuple[int, int] | None = None) -> torch.Tensor:
    """Page-at-a-time online softmax (packed_attention.py:260-311).

    ``page_range`` restricts the loop to page-table columns [lo, hi) -- used only
    by the bench to time a bounded sample of the CPU path.
    """
    check(q, kv)
    B, Hq, Q, D = q.shape
    S = kv.page_size
    n_rep = Hq // kv.num_kv_heads
    heads = kv_head_for(torch.arange(Hq), n_rep)
    q_rot = rotate_query(q.float(), kv.k_quant.Pi) * scale
    limit = _causal_limit(kv, Q)
    lo_all, hi_all = page_range or (0, kv.page_table.shape[1])
    chunks = [(lo_all, hi_all)] if not split_pages else [
        (s, min(s + split_pages, hi_all)) for s in range(lo_all, hi_all, split_pages)]
    partials = []
    for lo, hi in chunks:
        m = torch.full((B, Hq, Q), float("-inf"))
        l = torch.zeros(B, Hq, Q)
        a = torch.zeros(B, Hq, Q, D)
        for t in range(lo, hi):
            ids = kv.page_table[:, t].long().clamp(0, kv.k_pages.shape[0] - 1)
            ck = _centroids(kv.k_pages[ids], kv.k_quant, D)[:, heads]
            cv = _centroids(kv.v_pages[ids], kv.v_quant, D)[:, heads]
            nk = kv.k_norms[ids].float()[:, heads]
            nv = kv.v_norms[ids].float()[:, heads]
            s = (q_rot @ ck.transpose(-1, -2)) * nk[:, :, None, :]
            key_pos = t * S + torch.arange(S)
            ok = key_pos[None, None, :] <= limit[:, :, None]
            s = s.masked_fill(~ok[:, None], float("-inf"))
            m, l, a = _online_update(m, l, a, s, nv, cv)
        partials.append((m, l, a))
    m, l, a = partials[0]
    for part in partials[1:]:
        m, l, a = merge_partials((m, l, a), part)
    out = torch.where(l[..., None] > 0, a / l.clamp(min=1e-30)[..., None], 0.0)
    return rotate_output(out, kv.v_quant.Pi)


def _online_update(m, l, a, s, nv, cv):
    m_new = torch.maximum(m, s.amax(-1))
    alpha = _safe_exp(m, m_new)
    p = _safe_exp(s, m_new[..., None])
    l = alpha * l + p.sum(-1)
    a = alpha[..., None] * a + (p * nv[:, :, None, :]) @ cv
    return m_new, l, a


def _safe_exp(x, m):
    return torch.where(torch.isneginf(m) | torch.isneginf(x), 0.0, torch.exp(x - m))


def merge_partials(left, right):
    m1, l1, a1 = left
    m2, l2, a2 = right
    m = torch.maximum(m1, m2)
    w1, w2 = _safe_exp(m1, m), _safe_exp(m2, m)
    return m, w1 * l1 + w2 * l2, w1[..., None] * a1 + w2[..., None] * a2


def reconstruct_attention_f64(q: torch.Tensor, kv, scale: float) -> torch.Tensor:
    """Decode-only reconstruct attention with every operation in float64."""
    B, Hq, Q, D = q.shape
    assert Q == 1
    n_rep = Hq // kv.num_kv_heads
    out = torch.zeros(B, Hq, 1, D, dtype=torch.float64)
    for b in range(B):
        L = int(kv.seq_lens[b])
        if L == 0:
            continue
        pk, nk = _gather_history(kv.k_pages, kv.k_norms, kv, b)
        pv, nv = _gather_history(kv.v_pages, kv.v_norms, kv, b)
        ck = kv.k_quant.centroids.double()[unpack_t(pk, kv.k_quant.bit_width, D).long()]
        cv = kv.v_quant.centroids.double()[unpack_t(pv, kv.v_quant.bit_width, D).long()]
        k = (ck @ kv.k_quant.Pi.double()) * nk.double()[..., None]
        v = (cv @ kv.v_quant.Pi.double()) * nv.double()[..., None]
        heads = torch.arange(Hq) // n_rep
        s = (q[b].double() @ k[heads].transpose(-1, -2)) * scale
        out[b] = torch.softmax(s, -1) @ v[heads]
    return out


def dense_paged_attention_f64(q: torch.Tensor, k_pages: torch.Tensor, v_pages: torch.Tensor,
                              page_table: torch.Tensor, seq_lens: torch.Tensor, scale: float) -> torch.Tensor:
    """q (B, Hq, Q, D) over pages (P, Hkv, S, D) -> (B, Hq, Q, D) float64.

    Per sequence (packed_backend.py:229-246): gather its first ceil(L/S) pages, keep
    L rows, query i sees keys j <= L - Q + i, head h reads kv head h // n_rep; a
    sequence without tokens gives zeros.
    """
    B, Hq, Q, D = q.shape
    P, Hkv, S, _ = k_pages.shape
    n_rep = Hq // Hkv
    out = torch.zeros(B, Hq, Q, D, dtype=torch.float64)
    for b in range(B):
        L = int(seq_lens[b])
        if L == 0:
            continue
        ids = page_table[b, :(L + S - 1) // S].long()
        hist = lambda pg: pg[ids].double().permute(1, 0, 2, 3).reshape(Hkv, -1, D)[:, :L]  # noqa: E731
        k, v = hist(k_pages), hist(v_pages)
        heads = torch.arange(Hq) // n_rep
        s = (q[b].double() @ k[heads].transpose(-1, -2)) * scale                  # (Hq, Q, L)
        visible = torch.arange(L)[None, :] <= (L - Q + torch.arange(Q))[:, None]  # (Q, L)
        s = s.masked_fill(~visible, float("-inf"))
        out[b] = torch.softmax(s, -1) @ v[heads]
    return out


@torch.no_grad()
def pages_from_dense(k, v, seq_lens, k_tq, v_tq, page_size, num_pages=None, generator=None) -> OracleKV:
    """Quantize dense (B, Hkv, Lmax, D) K/V into randomly ordered pages (packed_attention.py:341-377)."""
    B, Hkv, _, D = k.shape
    lens = [int(x) for x in seq_lens]
    need = [(L + page_size - 1) // page_size for L in lens]
    total = num_pages or max(sum(need), 1)
    order = torch.randperm(total, generator=generator).tolist()
    nb_k, nb_v = packed_bytes(D, k_tq.bit_width), packed_bytes(D, v_tq.bit_width)
    kp = torch.zeros(total, Hkv, page_size, nb_k, dtype=torch.uint8)
    vp = torch.zeros(total, Hkv, page_size, nb_v, dtype=torch.uint8)
    kn = torch.zeros(total, Hkv, page_size, dtype=torch.float16)
    vn = torch.zeros(total, Hkv, page_size, dtype=torch.float16)
    table = torch.full((B, max(max(need), 1)), -1, dtype=torch.int32)
    nxt = 0
    for b in range(B):
        for t in range(need[b]):
            pid = order[nxt]
            nxt += 1
            table[b, t] = pid
            lo, hi = t * page_size, min((t + 1) * page_size, lens[b])
            for src, tq, pages, norms in ((k, k_tq, kp, kn), (v, v_tq, vp, vn)):
                idx, nrm = tq.quantize(src[b, :, lo:hi])
                pages[pid, :, :hi - lo] = pack_t(idx, tq.bit_width)
                norms[pid, :, :hi - lo] = nrm.to(torch.float16)
    return OracleKV(kp, kn, vp, vn, table, torch.tensor(lens, dtype=torch.int32),
                    OracleQuant.from_tq(k_tq), OracleQuant.from_tq(v_tq), D)
