"""Oracle: quantize + pack + page scatter of one KV append -- test infrastructure only.

CPU restatement of the packed branch of ``PagedPackedCache.update``
(``turboquant_kv/packed_backend.py:136-170``): for K and V,
``idx, nrm = tq.quantize(src)`` (cache.py:108-115), ``pack(idx, bw)`` permuted to
``(B, n, Hkv, NB)`` (packing.py:37-64), then
``pages[layer][pids, :, slots] = packed`` and ``norms[...] = nrm.fp16`` with
``pids = table[b, pos // S]``, ``slots = pos % S``, ``pos = lengths[b] + i``
(packed_backend.py:143-161).

Pinned by the quantizer and packing pins plus scatter checks on hand-built
tables (``tests/test_oracle_append.py``): every written row lands in the page
the table names at the slot ``pos % S``, and nothing else changes.
"""
from __future__ import annotations

import torch

from oracle.attention import pack_t


@torch.no_grad()
def append(src: torch.Tensor, tq, pages: torch.Tensor, norms: torch.Tensor,
           table: torch.Tensor, lengths) -> None:
    """Write ``src`` (B, Hkv, n, D) at positions ``lengths[b] + i`` of each sequence."""
    B, Hkv, n, D = src.shape
    S = pages.shape[2]
    pos = torch.tensor([[int(L) + i for i in range(n)] for L in lengths], dtype=torch.long)
    pids = torch.gather(table.cpu().long(), 1, pos // S)
    slots = pos % S
    idx, nrm = tq.quantize(src)
    packed = pack_t(idx, tq.bit_width).permute(0, 2, 1, 3)
    pages[pids, :, slots] = packed
    norms[pids, :, slots] = nrm.permute(0, 2, 1).to(torch.float16)
