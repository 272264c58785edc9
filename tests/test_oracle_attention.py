"""Pins of the CPU attention oracle (``oracle/attention.py``).

The oracle restates the reference's three compressed-domain operators
(``turboquant_kv/packed_attention.py:208-334``). Retyping their formulas here
would pin nothing, so each check compares against something fixed elsewhere:

* ``closed_form`` -- plain numpy float64 softmax attention over K/V dequantized
  from the packed bytes by the numpy bit unpacker (``oracle.packing``), a
  codebook gather and ``x_hat = c Pi * n``. It shares no code with the torch
  oracle beyond reading the same bytes.
* equalities between the oracle's own operators at the reference's kernel
  tolerance (test_packed_attention.py:22-23, 73-81);
* the edge cases of test_packed_attention.py:84-146 (causal prefill, empty and
  tail pages, all-masked rows, huge scores, zero vectors, GQA groups) and a
  hand-built non-symmetric rotation (:160-186);
* the seven seeded mutants of test_packed_attention.py:209-264, planted in the
  oracle on the CPU: each must miss the closed form by >= 100x the tolerance.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import packing as opk
from oracle.quantizer import OracleTQ, get_quantizer

ATOL = 2e-4
RTOL = 2e-4
MUTANT_MIN_ERR = 100 * ATOL


def make(seed=0, B=3, Hq=8, Hkv=2, D=64, lens=(37, 1, 64), Q=1, S=16, bw=8, q_scale=1.0, bw_v=None):
    g = torch.Generator().manual_seed(seed)
    Lmax = max(max(lens), 1)
    k = torch.randn(B, Hkv, Lmax, D, generator=g)
    v = torch.randn(B, Hkv, Lmax, D, generator=g)
    q = torch.randn(B, Hq, Q, D, generator=g) * q_scale
    kv = oa.pages_from_dense(k, v, lens, get_quantizer(bw, D, 42), get_quantizer(bw_v or bw, D, 43), S,
                             generator=g)
    return q, k, v, kv


def dequant_np(pages, norms, quant, D):
    """(N, NB) packed bytes + (N,) fp16 norms -> (N, D) float64 x_hat, in numpy."""
    codes = opk.unpack(pages.numpy(), quant.bit_width, D).astype(np.int64)
    c = quant.centroids.double().numpy()[codes]
    return (c @ quant.Pi.double().numpy()) * norms.double().numpy()[:, None]


def closed_form(q, kv, scale):
    """float64 numpy softmax attention over the dequantized history of every sequence."""
    qn = q.double().numpy()
    B, Hq, Q, D = qn.shape
    Hkv, S = kv.num_kv_heads, kv.page_size
    n_rep = Hq // Hkv
    out = np.zeros((B, Hq, Q, D))
    for b in range(B):
        L = int(kv.seq_lens[b])
        if L == 0:
            continue
        pids = [int(kv.page_table[b, t // S]) for t in range(L)]
        slots = [t % S for t in range(L)]
        for h in range(Hq):
            g = h // n_rep
            kp = torch.stack([kv.k_pages[p, g, s] for p, s in zip(pids, slots)])
            vp = torch.stack([kv.v_pages[p, g, s] for p, s in zip(pids, slots)])
            kn = torch.stack([kv.k_norms[p, g, s] for p, s in zip(pids, slots)])
            vn = torch.stack([kv.v_norms[p, g, s] for p, s in zip(pids, slots)])
            kh = dequant_np(kp, kn, kv.k_quant, D)
            vh = dequant_np(vp, vn, kv.v_quant, D)
            for i in range(Q):
                lim = L - Q + i                      # key j visible iff j <= lim
                if lim < 0:
                    continue
                s = kh[:lim + 1] @ qn[b, h, i] * scale
                p = np.exp(s - s.max())
                out[b, h, i] = (p / p.sum()) @ vh[:lim + 1]
    return torch.from_numpy(out)


def close(a, b, atol=ATOL, rtol=RTOL):
    return torch.allclose(a.double(), b.double(), atol=atol, rtol=rtol)


def err(a, b):
    return (a.double() - b.double()).abs().max().item()


OPS = {
    "reconstruct": oa.reconstruct_attention,
    "explicit": oa.explicit_compressed_attention,
    "tiled": oa.tiled_compressed_attention,
    "tiled_split2": lambda q, kv, s: oa.tiled_compressed_attention(q, kv, s, split_pages=2),
    "tiled_split3": lambda q, kv, s: oa.tiled_compressed_attention(q, kv, s, split_pages=3),
}


@pytest.mark.parametrize("op", sorted(OPS))
@pytest.mark.parametrize("seed,bw", [(0, 8), (1, 4), (2, 3)])
def test_operators_match_float64_closed_form(op, seed, bw):
    q, _, _, kv = make(seed=seed, bw=bw)
    scale = oa.default_scale(q.shape[-1])
    ref = closed_form(q, kv, scale)
    got = OPS[op](q, kv, scale)
    assert close(got, ref), err(got, ref)


def test_f64_operator_matches_closed_form():
    q, _, _, kv = make(seed=3, bw=4, lens=(70, 5, 33))
    scale = oa.default_scale(q.shape[-1])
    assert err(oa.reconstruct_attention_f64(q, kv, scale), closed_form(q, kv, scale)) < 1e-10


@pytest.mark.parametrize("op", sorted(OPS))
def test_causal_prefill_chunk(op):
    q, _, _, kv = make(seed=5, lens=(40, 17, 5), Q=5)
    scale = oa.default_scale(q.shape[-1])
    assert close(OPS[op](q, kv, scale), closed_form(q, kv, scale))


@pytest.mark.parametrize("op", sorted(OPS))
def test_empty_one_page_and_tail(op):
    q, _, _, kv = make(seed=7, lens=(0, 16, 17), S=16)
    scale = oa.default_scale(q.shape[-1])
    got = OPS[op](q, kv, scale)
    assert torch.isfinite(got).all()
    assert (got[0] == 0).all()
    assert close(got, closed_form(q, kv, scale))


@pytest.mark.parametrize("op", sorted(OPS))
def test_rows_without_visible_key_are_zero(op):
    q, _, _, kv = make(seed=8, lens=(2, 9, 30), Q=3)
    scale = oa.default_scale(q.shape[-1])
    got = OPS[op](q, kv, scale)
    assert torch.isfinite(got).all()
    assert (got[0, :, 0] == 0).all()
    assert close(got, closed_form(q, kv, scale))


@pytest.mark.parametrize("op", sorted(OPS))
def test_huge_scores_stay_finite(op):
    q, _, _, kv = make(seed=9, q_scale=3e3, lens=(50, 33, 64))
    scale = oa.default_scale(q.shape[-1])
    got = OPS[op](q, kv, scale)
    assert torch.isfinite(got).all()
    # scores in the thousands: fp32 score rounding is amplified, so compare at the
    # reference's own looser GPU tolerance (test_packed_attention_triton.py:26-27)
    assert close(got, closed_form(q, kv, scale), atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize("op", sorted(OPS))
def test_zero_vectors(op):
    g = torch.Generator().manual_seed(10)
    B, H, L, D = 2, 2, 20, 64
    k, v = torch.randn(B, H, L, D, generator=g), torch.randn(B, H, L, D, generator=g)
    k[0, :, 3] = 0
    v[1, :, 5:9] = 0
    kv = oa.pages_from_dense(k, v, (L, L), get_quantizer(8, D, 42), get_quantizer(8, D, 43), 8, generator=g)
    q = torch.randn(B, 4, 1, D, generator=g)
    scale = oa.default_scale(D)
    got = OPS[op](q, kv, scale)
    assert torch.isfinite(got).all()
    assert close(got, closed_form(q, kv, scale))


def test_gqa_groups_read_their_own_kv_head():
    q, _, _, kv = make(seed=11, Hq=12, Hkv=3)
    scale = oa.default_scale(q.shape[-1])
    ref = closed_form(q, kv, scale)
    assert close(oa.tiled_compressed_attention(q, kv, scale), ref)
    # the same answer from plain MHA over kv heads repeated in repeat_kv order
    rep = oa.OracleKV(kv.k_pages.repeat_interleave(4, 1), kv.k_norms.repeat_interleave(4, 1),
                      kv.v_pages.repeat_interleave(4, 1), kv.v_norms.repeat_interleave(4, 1),
                      kv.page_table, kv.seq_lens, kv.k_quant, kv.v_quant, kv.head_dim)
    assert close(oa.tiled_compressed_attention(q, rep, scale), ref)


def test_quantization_error_is_separate_from_arithmetic_error():
    q, k, v, kv = make(seed=12, bw=8)
    scale = oa.default_scale(q.shape[-1])
    B, Hq = q.shape[:2]
    n_rep = Hq // k.shape[1]
    exact = torch.zeros_like(q)
    for b in range(B):
        L = int(kv.seq_lens[b])
        kk = k[b, :, :L].repeat_interleave(n_rep, 0)
        vv = v[b, :, :L].repeat_interleave(n_rep, 0)
        exact[b] = torch.softmax(q[b] @ kk.transpose(-1, -2) * scale, -1) @ vv
    quant = closed_form(q, kv, scale)
    kern = oa.tiled_compressed_attention(q, kv, scale)
    assert err(kern, quant) < ATOL < err(quant, exact) < 0.1


def _nonsymmetric_rotation(D=8):
    c, s = math.cos(0.7), math.sin(0.7)
    R = torch.eye(D)
    R[0, 0], R[0, 1], R[1, 0], R[1, 1] = c, -s, s, c
    perm = torch.eye(D)[[2, 0, 1, 5, 3, 4, 7, 6]]
    return (perm @ R).contiguous()


def test_rotation_direction_with_a_nonsymmetric_matrix():
    D = 8
    Pi = _nonsymmetric_rotation(D)
    assert torch.allclose(Pi @ Pi.T, torch.eye(D), atol=1e-6) and not torch.allclose(Pi, Pi.T)
    k_tq, v_tq = OracleTQ(8, D, 42), OracleTQ(8, D, 7)
    k_tq.Pi = Pi
    g = torch.Generator().manual_seed(13)
    k, v = torch.randn(1, 1, 6, D, generator=g), torch.randn(1, 1, 6, D, generator=g)
    kv = oa.pages_from_dense(k, v, (6,), k_tq, v_tq, 4, generator=g)
    q = torch.randn(1, 2, 1, D, generator=g)
    scale = oa.default_scale(D)
    ref = closed_form(q, kv, scale)
    for op in OPS.values():
        assert close(op(q, kv, scale), ref)
    wrong = oa.OracleKV(**{**kv.__dict__, "k_quant": oa.OracleQuant(Pi.T.contiguous(), k_tq.centroids, 8)})
    assert err(oa.tiled_compressed_attention(q, wrong, scale), ref) > MUTANT_MIN_ERR


def test_contract_rejections():
    q, _, _, kv = make(seed=14)
    with pytest.raises(oa.ContractError):
        oa.tiled_compressed_attention(q[..., :32], kv, 1.0)
    with pytest.raises(oa.ContractError):
        oa.tiled_compressed_attention(q[:, :7], kv, 1.0)
    bad = oa.OracleKV(**{**kv.__dict__, "page_table": kv.page_table.clone()})
    bad.page_table[0, 0] = kv.k_pages.shape[0]
    with pytest.raises(oa.ContractError):
        oa.tiled_compressed_attention(q, bad, 1.0)
    bad = oa.OracleKV(**{**kv.__dict__, "seq_lens": kv.seq_lens + 1000})
    with pytest.raises(oa.ContractError):
        oa.tiled_compressed_attention(q, bad, 1.0)


# -- the reference's seven seeded mutants, planted in the oracle ---------------

def _mutant_err(monkeypatch, attr, fn, op="tiled", **case):
    q, _, _, kv = make(seed=21, **case)
    scale = oa.default_scale(q.shape[-1])
    ref = closed_form(q, kv, scale)
    assert close(OPS[op](q, kv, scale), ref)
    monkeypatch.setattr(oa, attr, fn)
    return err(OPS[op](q, kv, scale), ref)


@pytest.mark.parametrize("op", ["explicit", "tiled"])
def test_mutant_query_rotation_transposed(monkeypatch, op):
    assert _mutant_err(monkeypatch, "rotate_query", lambda q, Pi: q @ Pi, op) > MUTANT_MIN_ERR


@pytest.mark.parametrize("op", ["explicit", "tiled"])
def test_mutant_output_rotation_transposed(monkeypatch, op):
    assert _mutant_err(monkeypatch, "rotate_output", lambda a, Pi: a @ Pi.T, op) > MUTANT_MIN_ERR


@pytest.mark.parametrize("op", ["explicit", "tiled"])
def test_mutant_gqa_interleaved(monkeypatch, op):
    assert _mutant_err(monkeypatch, "kv_head_for", lambda h, n: h % 2, op) > MUTANT_MIN_ERR


def test_mutant_missing_scale():
    q, _, _, kv = make(seed=22)
    ref = closed_form(q, kv, oa.default_scale(q.shape[-1]))
    assert err(oa.tiled_compressed_attention(q, kv, 1.0), ref) > MUTANT_MIN_ERR


def test_mutant_value_in_key_basis():
    q, _, _, kv = make(seed=23)
    scale = oa.default_scale(q.shape[-1])
    ref = closed_form(q, kv, scale)
    swapped = oa.OracleKV(**{**kv.__dict__, "v_quant": kv.k_quant})
    assert err(oa.tiled_compressed_attention(q, swapped, scale), ref) > MUTANT_MIN_ERR


def test_mutant_online_softmax_without_rescale(monkeypatch):
    def no_alpha(m, l, a, s, nv, cv):
        m_new = torch.maximum(m, s.amax(-1))
        p = oa._safe_exp(s, m_new[..., None])
        return m_new, l + p.sum(-1), a + (p * nv[:, :, None, :]) @ cv
    assert _mutant_err(monkeypatch, "_online_update", no_alpha, lens=(64, 48, 64), q_scale=4.0) > MUTANT_MIN_ERR


def test_mutant_split_merge_without_rescale(monkeypatch):
    def naive(left, right):
        return torch.maximum(left[0], right[0]), left[1] + right[1], left[2] + right[2]
    assert _mutant_err(monkeypatch, "merge_partials", naive, op="tiled_split2",
                       lens=(64, 48, 64), q_scale=4.0) > MUTANT_MIN_ERR


def test_tiled_reads_one_page_at_a_time(monkeypatch):
    """The tiled oracle never builds a (.., L, D) history: every gather is one page."""
    q, _, _, kv = make(seed=24, lens=(64, 64, 64), S=16)
    seen = []
    real = oa._centroids

    def spy(pages, quant, d):
        out = real(pages, quant, d)
        seen.append(tuple(out.shape))
        return out
    monkeypatch.setattr(oa, "_centroids", spy)
    oa.tiled_compressed_attention(q, kv, 1.0)
    assert seen and all(s[-2] == 16 for s in seen)
