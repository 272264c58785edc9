"""Model-side integration: the paged packed cache's append path and the decode dispatcher.

Drop-in for ``turboquant_kv/packed_backend.py``:

* ``PagedPackedCache.update`` (packed_backend.py:136-170) quantizes, bit-packs
  and scatters the new K/V into the pool pages with ONE ``wn_append_kv`` launch
  per layer (K and V together). Token i of sequence b goes to page
  ``table[b, (L_b + i) // S]`` slot ``(L_b + i) % S``; the page-table lookup
  happens on the device, so unlike the reference there is no per-layer
  device-to-host copy of the table (packed_backend.py:144).
* ``winnow_packed_attention`` (packed_backend.py:260-290) serves decode with the
  HIP operator (packed pages) or the HIP dense kernel (unquantized pages), and a
  prefill chunk by dequantizing the sequence's history on the GPU and calling SDPA
  (packed_backend.py:192-226).
* ``make_pool``, ``quantizers_for``, ``select_decode_backend``, ``BACKEND_COUNTS``
  keep the reference's names and meaning. There is no host fallback: a decode on
  a non-HIP tensor raises.
"""
from __future__ import annotations

from collections import Counter

import torch
import torch.nn.functional as F

from winnow_amd import _lib
from winnow_amd import packed_attention as pa
from winnow_amd.packing import packed_bytes, unpack
from winnow_amd.page_pool import PagePool, StalePage
from winnow_amd.quantizer import get_quantizer

ATTN_NAME = "winnow_packed"
SUPPORTED_ARCH = ("Qwen2ForCausalLM",)
DECODE_BACKENDS = ("hip_packed", "reconstruct_sdpa", "hip_dense", "dense_sdpa")

# How many attention calls each backend served (packed_backend.py:38-40).
BACKEND_COUNTS: Counter = Counter()


class UnsupportedModel(ValueError):
    pass


def check_model(config, bit_width: int) -> None:
    """Reject unsupported model configurations before load (packed_backend.py:58-68)."""
    arch = (getattr(config, "architectures", None) or ["?"])[0]
    if arch not in SUPPORTED_ARCH:
        raise UnsupportedModel(f"{arch} is not a supported architecture {SUPPORTED_ARCH}")
    if getattr(config, "use_sliding_window", False):
        raise UnsupportedModel("sliding-window attention is not supported")
    types = set(getattr(config, "layer_types", None) or ["full_attention"])
    if types != {"full_attention"}:
        raise UnsupportedModel(f"layer types {sorted(types)} are not all full attention")
    packed_bytes(head_dim_of(config), bit_width)


def head_dim_of(config) -> int:
    return getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads


def make_pool(config, *, bit_width: int | None, num_pages: int, page_size: int, device,
              max_pages_per_request=None, fence_factory=None,
              dense_dtype: torch.dtype | None = None) -> PagePool:
    """Packed pool at ``bit_width``, or with ``dense_dtype`` an unquantized pool (packed_backend.py:75-85)."""
    D = head_dim_of(config)
    nb = D if dense_dtype is not None else packed_bytes(D, bit_width)
    return PagePool(num_layers=config.num_hidden_layers, num_pages=num_pages,
                    num_kv_heads=config.num_key_value_heads, page_size=page_size,
                    nb_k=nb, nb_v=nb, device=device, max_pages_per_request=max_pages_per_request,
                    fence_factory=fence_factory, dense_dtype=dense_dtype)


def quantizers_for(config, bit_width: int, device, k_seed: int = 42, v_seed: int = 42):
    """K and V quantizers; seed 42/42 by default, as the reference (packed_backend.py:298-303)."""
    D = head_dim_of(config)
    return get_quantizer(bit_width, D, device, seed=k_seed), get_quantizer(bit_width, D, device, seed=v_seed)


class PagedPackedCache:
    """Duck-typed cache for one forward over a batch of pool-backed sequences.

    ``owners[b]`` is the request id whose pages hold sequence b and
    ``lengths[b]`` the tokens already stored; every sequence appends the same n
    tokens per forward; lengths advance after the last layer (packed_backend.py:88-112).
    """

    def __init__(self, pool: PagePool, owners, lengths, *, k_quant, v_quant,
                 head_dim: int, decode_backend: str = "auto"):
        self.pool = pool
        self.owners = list(owners)
        self.lengths = list(lengths)
        self.kq, self.vq = k_quant, v_quant
        self.head_dim = head_dim
        self.decode_backend = decode_backend
        self._table = self._table_host = self._seq = self._seq_host = self._start = None
        self._refs = None

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if len(set(self.lengths)) != 1:
            raise RuntimeError("mixed lengths: pass explicit position_ids")
        return self.lengths[0]

    def _prepare(self, n: int, device) -> None:
        """Once per forward: check ownership and reservation, build the table (packed_backend.py:114-133).

        Never allocates pages: a forward racing a release must fail.
        """
        refs = [self.pool.held(o) for o in self.owners]
        for o, r, L in zip(self.owners, refs, self.lengths):
            if self.pool.pages_for(L + n) > len(r):
                raise StalePage(f"{o} holds {len(r)} pages, needs {self.pool.pages_for(L + n)}")
            self.pool.validate(o, r)
        width = max(max(len(r) for r in refs), 1)
        table = torch.full((len(refs), width), -1, dtype=torch.int32)
        for b, r in enumerate(refs):
            if r:
                table[b, :len(r)] = torch.tensor([x.page for x in r], dtype=torch.int32)
        self._refs = refs
        self._table_host = table
        self._seq_host = torch.tensor([L + n for L in self.lengths], dtype=torch.int32)
        start = torch.tensor(self.lengths, dtype=torch.int32)
        self._table = table.to(device, non_blocking=True)
        self._seq = self._seq_host.to(device, non_blocking=True)
        self._start = start.to(device, non_blocking=True)

    @torch.no_grad()
    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        B, Hkv, n, D = key_states.shape
        if B != len(self.owners):
            raise RuntimeError(f"batch {B} != {len(self.owners)} owners")
        if layer_idx == 0:
            self._prepare(n, key_states.device)
        S = self.pool.page_size
        if self.pool.dense:
            pos = torch.tensor([[L + i for i in range(n)] for L in self.lengths])
            pids = torch.gather(self._table_host.long(), 1, pos // S).to(key_states.device)
            slots = (pos % S).to(key_states.device)
            for src, pages in ((key_states, self.pool.k_pages), (value_states, self.pool.v_pages)):
                pages[layer_idx][pids, :, slots] = src.permute(0, 2, 1, 3).to(pages.dtype)
            handle = pa.DenseKV(self.pool.k_pages[layer_idx], self.pool.v_pages[layer_idx],
                                self._table, self._seq, D)
        else:
            append_kv(key_states, value_states, self.kq, self.vq,
                      self.pool.k_pages[layer_idx], self.pool.v_pages[layer_idx],
                      self.pool.k_norms[layer_idx], self.pool.v_norms[layer_idx],
                      self._table, self._start)
            handle = pa.PackedKV(
                self.pool.k_pages[layer_idx], self.pool.k_norms[layer_idx],
                self.pool.v_pages[layer_idx], self.pool.v_norms[layer_idx],
                self._table, self._seq, pa.Quantizer.from_tq(self.kq), pa.Quantizer.from_tq(self.vq), D,
                seq_lens_host=self._seq_host, page_table_host=self._table_host)
        handle.decode_backend = self.decode_backend
        if layer_idx == self.pool.num_layers - 1:
            self.lengths = [L + n for L in self.lengths]
        return handle, handle


@torch.no_grad()
def append_kv(k: torch.Tensor, v: torch.Tensor | None, k_tq, v_tq,
              k_pages: torch.Tensor, v_pages: torch.Tensor | None,
              k_norms: torch.Tensor, v_norms: torch.Tensor | None,
              page_table: torch.Tensor, start_pos: torch.Tensor) -> None:
    """Quantize + pack + scatter (B, Hkv, n, D) K (and V) into one layer's pages, one launch.

    Token i of sequence b lands at position ``start_pos[b] + i``.
    """
    for t in (k, k_pages, k_norms, page_table, start_pos):
        if not _lib.is_hip(t):
            raise pa.UnsupportedLayout("append_kv needs every operand on a HIP device")
    B, Hkv, n, D = k.shape
    if k.dtype not in _lib.DTYPE_CODE:
        k = k.float()
    if v is not None and v.dtype != k.dtype:
        v = v.to(k.dtype)
    for x in (k, v):
        if x is not None and x.stride(-1) != 1:
            raise pa.UnsupportedLayout("K/V states need a contiguous head_dim")
    if page_table.dtype != torch.int32 or start_pos.dtype != torch.int32 or page_table.stride(-1) != 1:
        raise pa.UnsupportedLayout("page_table / start_pos must be int32 with contiguous rows")
    for pages, norms, tq in ((k_pages, k_norms, k_tq), (v_pages, v_norms, v_tq)):
        if pages is None:
            continue
        if pages.shape[1:] != (Hkv, pages.shape[2], packed_bytes(D, tq.bit_width)) or \
                pages.stride(-1) != 1 or pages.stride(-2) != pages.shape[-1] or norms.stride(-1) != 1:
            raise pa.UnsupportedLayout("pages must be (P, Hkv, S, NB) with contiguous rows")
    S = k_pages.shape[2]
    dev = k.device
    vv = v if v is not None else None
    with torch.cuda.device(dev):
        _lib.call(
            "wn_append_kv",
            _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
            _lib.ptr(vv), vv.stride(0) if vv is not None else 0, vv.stride(1) if vv is not None else 0,
            vv.stride(2) if vv is not None else 0, _lib.DTYPE_CODE[k.dtype],
            _lib.ptr(k_tq.Pi), _lib.ptr(k_tq.boundaries), k_tq.bit_width,
            _lib.ptr(v_tq.Pi) if vv is not None else None,
            _lib.ptr(v_tq.boundaries) if vv is not None else None,
            v_tq.bit_width if vv is not None else 0,
            _lib.ptr(page_table), page_table.stride(0), _lib.ptr(start_pos),
            _lib.ptr(k_pages), k_pages.stride(0), k_pages.stride(1),
            _lib.ptr(v_pages) if vv is not None else None,
            v_pages.stride(0) if vv is not None else 0, v_pages.stride(1) if vv is not None else 0,
            _lib.ptr(k_norms), k_norms.stride(0), k_norms.stride(1),
            _lib.ptr(v_norms) if vv is not None else None,
            v_norms.stride(0) if vv is not None else 0, v_norms.stride(1) if vv is not None else 0,
            B, Hkv, n, D, S, k_pages.shape[0], page_table.shape[1], _lib.stream_of(dev))


def select_decode_backend(query: torch.Tensor, kv, requested: str) -> str:
    """Which operator serves a decode step; unsupported requests fail loudly (packed_backend.py:173-189)."""
    if isinstance(kv, pa.DenseKV):
        # packed_backend.py:175-179: the dense kernel where it runs, else dense SDPA
        if requested == "dense_sdpa":
            return requested
        if requested not in ("auto", "triton_dense", "hip_dense"):
            raise ValueError(f"backend {requested!r} does not read dense pages")
        if not _lib.is_hip(query):
            raise RuntimeError("the dense decode operator needs a HIP device; there is no host fallback")
        if pa.dense_supported(query, kv):
            return "hip_dense"
        if requested == "hip_dense":
            raise ValueError("hip_dense does not compile this shape (head_dim 128, bf16/fp16 pages, S >= 16)")
        return "dense_sdpa"
    if requested in ("auto", "triton_packed", "hip_packed"):
        if not _lib.is_hip(query):
            raise RuntimeError("the packed decode operator needs a HIP device; there is no host fallback")
        return "hip_packed"
    if requested not in DECODE_BACKENDS:
        raise ValueError(f"unknown decode backend {requested!r}")
    return requested


def dequantize_history(kv: pa.PackedKV, pages, norms, quant, b: int, dtype) -> torch.Tensor:
    """(1, Hkv, L, D) reconstruction of sequence b on the GPU (packed_backend.py:192-208).

    head_dim 128: one fused HIP kernel (``wn_dequantize_history``) reads the pool
    pages through the page table, so nothing is gathered or unpacked first."""
    L = int(kv.seq_lens_host[b]) if kv.seq_lens_host is not None else int(kv.seq_lens[b])
    S = kv.page_size
    D = kv.head_dim
    if D == 128 and pages.stride(-1) == 1 and pages.stride(-2) == pages.shape[-1] and norms.stride(-1) == 1:
        Hkv = pages.shape[1]
        out = torch.empty(1, Hkv, L, D, dtype=dtype if dtype in _lib.DTYPE_CODE else torch.float32,
                          device=pages.device)
        if L == 0:
            return out.to(dtype)
        with torch.cuda.device(pages.device):
            _lib.call("wn_dequantize_history", _lib.ptr(pages), pages.stride(0), pages.stride(1),
                      _lib.ptr(norms), norms.stride(0), norms.stride(1), _lib.ptr(kv.page_table[b]), L, Hkv, S,
                      _lib.ptr(quant.centroids), _lib.ptr(quant.Pi), quant.bit_width, D, _lib.ptr(out),
                      _lib.DTYPE_CODE[out.dtype], 0, _lib.stream_of(pages.device))
        return out.to(dtype)
    table = kv.page_table_host if kv.page_table_host is not None else kv.page_table.cpu()
    ids = table[b, :(L + S - 1) // S].long().to(pages.device)
    rows = pages[ids].permute(1, 0, 2, 3).reshape(pages.shape[1], -1, pages.shape[3])[:, :L].contiguous()
    nrm = norms[ids].permute(1, 0, 2).reshape(norms.shape[1], -1)[:, :L].contiguous()
    codes = unpack(rows, quant.bit_width, D).contiguous()
    out = torch.empty(1, rows.shape[0], L, D, dtype=dtype if dtype in _lib.DTYPE_CODE else torch.float32,
                      device=rows.device)
    with torch.cuda.device(rows.device):
        _lib.call("wn_dequantize", _lib.ptr(codes), _lib.ptr(nrm), codes.numel() // D, _lib.ptr(quant.Pi),
                  _lib.ptr(quant.centroids), quant.bit_width, D, _lib.ptr(out), _lib.DTYPE_CODE[out.dtype],
                  _lib.stream_of(rows.device))
    return out.to(dtype)


def _reconstruct_sdpa(query, kv: pa.PackedKV, scaling):
    """Per sequence: dequantize on the GPU, then SDPA with an offset causal mask (packed_backend.py:211-226)."""
    B, Hq, Q, D = query.shape
    out = torch.zeros(B, Hq, Q, D, dtype=query.dtype, device=query.device)
    lens = kv.seq_lens_host if kv.seq_lens_host is not None else kv.seq_lens.cpu()
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        k = dequantize_history(kv, kv.k_pages, kv.k_norms, kv.k_quant, b, query.dtype)
        v = dequantize_history(kv, kv.v_pages, kv.v_norms, kv.v_quant, b, query.dtype)
        mask = torch.arange(L, device=query.device)[None, :] <= (
            L - Q + torch.arange(Q, device=query.device))[:, None]
        out[b] = F.scaled_dot_product_attention(query[b:b + 1], k, v, attn_mask=mask, scale=scaling,
                                                enable_gqa=Hq != k.shape[1])[0]
    return out


def _dense_sdpa(query, kv: pa.DenseKV, scaling):
    """Per sequence: gather unquantized pages, SDPA with an offset causal mask (packed_backend.py:229-245)."""
    B, Hq, Q, D = query.shape
    out = torch.zeros(B, Hq, Q, D, dtype=query.dtype, device=query.device)
    S = kv.page_size
    lens = kv.seq_lens.cpu()
    table = kv.page_table.cpu()
    for b in range(B):
        L = int(lens[b])
        if L == 0:
            continue
        ids = table[b, :(L + S - 1) // S].long().to(query.device)

        def hist(p):
            return p[ids].permute(1, 0, 2, 3).reshape(p.shape[1], -1, D)[None, :, :L].to(query.dtype)

        mask = torch.arange(L, device=query.device)[None, :] <= (
            L - Q + torch.arange(Q, device=query.device))[:, None]
        out[b] = F.scaled_dot_product_attention(query[b:b + 1], hist(kv.k_pages), hist(kv.v_pages),
                                                attn_mask=mask, scale=scaling,
                                                enable_gqa=Hq != kv.num_kv_heads)[0]
    return out


def winnow_packed_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                            scaling=None, **kwargs):
    """``AttentionInterface`` entry point; returns ((B, Q, Hq, D), None) (packed_backend.py:260-290)."""
    scaling = scaling if scaling is not None else query.shape[-1] ** -0.5
    if not isinstance(key, (pa.PackedKV, pa.DenseKV)):
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        BACKEND_COUNTS["native_sdpa"] += 1
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scaling, **kwargs)
    Q = query.shape[2]
    if isinstance(key, pa.DenseKV):
        if Q > 1:
            BACKEND_COUNTS["prefill_dense_sdpa"] += 1
            return _dense_sdpa(query, key, scaling).transpose(1, 2).contiguous(), None
        backend = select_decode_backend(query, key, getattr(key, "decode_backend", "auto"))
        BACKEND_COUNTS[backend] += 1
        out = (pa.dense_decode_attention(query, key, scaling) if backend == "hip_dense"
               else _dense_sdpa(query, key, scaling))
        return out.transpose(1, 2).contiguous(), None
    if Q > 1:
        BACKEND_COUNTS["prefill_reconstruct_sdpa"] += 1
        out = _reconstruct_sdpa(query, key, scaling)
    else:
        backend = select_decode_backend(query, key, getattr(key, "decode_backend", "auto"))
        BACKEND_COUNTS[backend] += 1
        if backend == "hip_packed":
            out = pa.packed_decode_attention(query, key, scaling)
        else:
            out = _reconstruct_sdpa(query, key, scaling)
    return out.transpose(1, 2).contiguous(), None


def register() -> None:
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_NAME, winnow_packed_attention)
