"""Pins the oracle's page scatter (``oracle.append``) on the CPU, against the closed form
of ``PagedPackedCache.update`` (turboquant_kv/packed_backend.py:143-161):

    token i of sequence b, kv head h lands at
        pages[table[b, (L_b + i) // S], h, (L_b + i) % S] = pack(quantize(x[b, h, i]))
        norms[table[b, (L_b + i) // S], h, (L_b + i) % S] = fp16(||x[b, h, i]||)

The expected pages are built token by token in plain Python with the numpy packer
(``oracle.packing``, pinned by its own known answers), from the codes of the pinned
quantizer. Every byte outside the appended slots must keep its previous (random)
value. The tables are built by hand: shuffled page ids, a start in the middle of a
page, a start on a page boundary, an empty sequence, spans of two and three pages.
Mistakes planted in the oracle's three scatter steps must each fail the check.
"""
from __future__ import annotations

import pytest
import torch

from oracle import append as oapp
from oracle import packing as opk
from oracle.quantizer import get_quantizer

D = 64


def _case(bw, B, Hkv, S, n, lengths, table, P, seed):
    g = torch.Generator().manual_seed(seed)
    src = torch.randn(B, Hkv, n, D, generator=g)
    if n:
        src[0, 0, 0] = 0                                  # a zero vector: norm clamps, codes #{b < 0}
    nb = opk.packed_bytes(D, bw)
    pages = torch.randint(0, 256, (P, Hkv, S, nb), dtype=torch.uint8, generator=g)
    norms = torch.randn(P, Hkv, S, generator=g).half()
    return src, pages, norms, torch.tensor(table, dtype=torch.int32), list(lengths)


HAND = dict(B=3, Hkv=2, S=4, n=7, lengths=(2, 4, 0), P=13,
            # b0: positions 2..8 span three pages (start mid-page); b1: 4..10 start on a
            # page boundary and skip column 0; b2: 0..6 from an empty sequence
            table=[[11, 3, 7, -1], [5, 0, 9, -1], [12, 2, -1, -1]])


def _shuffled(seed=7, B=5, Hkv=3, S=8, n=12):
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(0, 40, (B,), generator=g).tolist()
    need = [(L + n + S - 1) // S for L in lengths]
    P = sum(need) + 4
    order = torch.randperm(P, generator=g).tolist()
    width = max(need) + 1
    table, k = [], 0
    for b in range(B):
        row = order[k:k + need[b]] + [-1] * (width - need[b])
        k += need[b]
        table.append(row)
    return dict(B=B, Hkv=Hkv, S=S, n=n, lengths=tuple(lengths), P=P, table=table)


def expected(src, tq, pages, norms, table, lengths):
    """The closed form, token by token: (pages, norms, mask of the written slots)."""
    B, Hkv, n, _ = src.shape
    S = pages.shape[2]
    pages, norms = pages.clone(), norms.clone()
    idx, nrm = tq.quantize(src)
    idx = idx.numpy()
    nrm16 = nrm.to(torch.float16)
    written = torch.zeros(pages.shape[:3], dtype=torch.bool)
    for b in range(B):
        for i in range(n):
            pos = int(lengths[b]) + i
            page = int(table[b][pos // S])
            slot = pos % S
            assert 0 <= page < pages.shape[0], "the case's table must cover every position"
            for h in range(Hkv):
                pages[page, h, slot] = torch.from_numpy(opk.pack(idx[b, h, i], tq.bit_width))
                norms[page, h, slot] = nrm16[b, h, i]
                written[page, h, slot] = True
    return pages, norms, written


def check_append(bw, case, seed=0):
    """Run the oracle's append on random pre-existing bytes and hold it to the closed form."""
    src, pages, norms, table, lengths = _case(bw, seed=seed, **case)
    tq = get_quantizer(bw, D, 42)
    want_p, want_n, written = expected(src, tq, pages, norms, table, lengths)
    got_p, got_n = pages.clone(), norms.clone()
    oapp.append(src, tq, got_p, got_n, table, lengths)
    assert torch.equal(got_p[~written], pages[~written]), "bytes outside the appended slots changed"
    assert torch.equal(got_n[~written].view(torch.int16), norms[~written].view(torch.int16)), \
        "norms outside the appended slots changed"
    assert torch.equal(got_p, want_p), "packed rows are not where the table puts them"
    assert torch.equal(got_n.view(torch.int16), want_n.view(torch.int16)), "fp16 norms misplaced"
    return written


@pytest.mark.parametrize("bw", [3, 4, 6, 8])
def test_hand_table_matches_closed_form(bw):
    written = check_append(bw, HAND)
    assert int(written.sum()) == 3 * 7 * 2                # every vector written exactly once
    # b0 spans three pages, b1 two (starting at column 1), b2 two
    assert written[11].any() and written[3].all() and written[7, :, 0].all()
    assert not written[5].any() and written[0].all() and written[9, :, :3].all()


@pytest.mark.parametrize("bw", [4, 6])
def test_shuffled_table_matches_closed_form(bw):
    check_append(bw, _shuffled(), seed=3)


def test_single_token_decode_appends():
    case = dict(B=3, Hkv=2, S=4, n=1, lengths=(3, 4, 0), P=6, table=[[4, 1, -1], [0, 5, -1], [2, -1, -1]])
    written = check_append(4, case)
    assert written[4, :, 3].all() and written[5, :, 0].all() and written[2, :, 0].all()
    assert int(written.sum()) == 6


def test_zero_new_tokens_changes_nothing():
    case = dict(HAND, n=0)
    written = check_append(4, case)
    assert not written.any()


# -- planted mistakes: each must fail the closed-form check ---------------------------

def _swapped(table, pos, S):
    return torch.gather(table.cpu().long(), 1, pos % S), pos // S


def _wrong_row(table, pos, S):
    return torch.gather(table.cpu().long().roll(1, 0), 1, pos // S), pos % S


def _off_by_one(lengths, n):
    return torch.as_tensor([int(L) + 1 for L in lengths])[:, None] + torch.arange(n)[None, :]


def _norm_one_slot_off(pages, norms, pids, slots, rows, nrm16):
    pages[pids, :, slots] = rows
    norms[pids, :, (slots + 1) % pages.shape[2]] = nrm16


def _heads_not_permuted(pages, norms, pids, slots, rows, nrm16):
    # rows of (B, Hkv, n, NB) reinterpreted as (B, n, Hkv, NB) instead of permuted
    pages[pids, :, slots] = rows.permute(0, 2, 1, 3).reshape(rows.shape)
    norms[pids, :, slots] = nrm16


@pytest.mark.parametrize("name,attr,fn", [
    ("page and slot swapped", "locate", _swapped),
    ("wrong sequence row", "locate", _wrong_row),
    ("off-by-one start", "positions", _off_by_one),
    ("norm one slot off", "write", _norm_one_slot_off),
    ("head axis not permuted", "write", _heads_not_permuted),
])
def test_planted_scatter_mistakes_are_caught(monkeypatch, name, attr, fn):
    monkeypatch.setattr(oapp, attr, fn)
    with pytest.raises(AssertionError):
        check_append(4, HAND)
