"""Oracle: quantize + pack + page scatter of one KV append -- test infrastructure only.

CPU restatement of the packed branch of ``PagedPackedCache.update``
(``turboquant_kv/packed_backend.py:136-170``): for K and V,
``idx, nrm = tq.quantize(src)`` (cache.py:108-115), ``pack(idx, bw)`` permuted to
``(B, n, Hkv, NB)`` (packing.py:37-64), then
``pages[layer][pids, :, slots] = packed`` and ``norms[...] = nrm.fp16`` with
``pids = table[b, pos // S]``, ``slots = pos % S``, ``pos = lengths[b] + i``
(packed_backend.py:143-161).

The three steps of the scatter (``positions``, ``locate``, ``write``) are module
attributes so the tests can plant mistakes in each one, here on the CPU.

Pinned by ``tests/test_oracle_append.py``: on hand-built tables (shuffled page
ids, a start in the middle of a page, spans of several pages, several sequences)
every appended vector's packed row and fp16 norm must sit at the page the table
names for ``(L_b + i) // S``, slot ``(L_b + i) % S``, computed token by token in
plain Python with the numpy packer, and every other byte of the pages and norms
must keep its previous value. Planted mistakes (page and slot roles swapped, an
off-by-one start, the wrong sequence's table row, the norm one slot off, the
head axis not permuted) each fail that check. The quantizer and the packer are
pinned by their own tests.
"""
from __future__ import annotations

import torch

from oracle.attention import pack_t


def positions(lengths, n: int) -> torch.Tensor:
    """(B, n) int64 token positions ``lengths[b] + i`` (packed_backend.py:143)."""
    start = torch.as_tensor([int(L) for L in lengths], dtype=torch.long)
    return start[:, None] + torch.arange(n, dtype=torch.long)[None, :]


def locate(table: torch.Tensor, pos: torch.Tensor, page_size: int):
    """Page id ``table[b, pos // S]`` and slot ``pos % S`` of every position (packed_backend.py:144-146)."""
    pids = torch.gather(table.cpu().long(), 1, pos // page_size)
    return pids, pos % page_size


def write(pages: torch.Tensor, norms: torch.Tensor, pids: torch.Tensor, slots: torch.Tensor,
          rows: torch.Tensor, nrm16: torch.Tensor) -> None:
    """``pages[pids, :, slots] = rows`` (B, n, Hkv, NB) and the fp16 norms beside them (packed_backend.py:160-161)."""
    pages[pids, :, slots] = rows
    norms[pids, :, slots] = nrm16


@torch.no_grad()
def append(src: torch.Tensor, tq, pages: torch.Tensor, norms: torch.Tensor,
           table: torch.Tensor, lengths) -> None:
    """Write ``src`` (B, Hkv, n, D) at positions ``lengths[b] + i`` of each sequence."""
    n = src.shape[2]
    pids, slots = locate(table, positions(lengths, n), pages.shape[2])
    idx, nrm = tq.quantize(src)
    rows = pack_t(idx, tq.bit_width).permute(0, 2, 1, 3)
    write(pages, norms, pids, slots, rows, nrm.permute(0, 2, 1).to(torch.float16))
