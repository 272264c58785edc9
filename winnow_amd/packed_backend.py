"""Model-side integration: the paged packed cache's append path and the attention dispatcher.

Names, arguments and errors are those of ``turboquant_kv/packed_backend.py``
(``UnsupportedModel``, ``check_model``, ``head_dim_of``, ``make_pool``,
``quantizers_for``, ``PagedPackedCache``, ``select_decode_backend``,
``dequantize_history``, ``winnow_packed_attention``, ``register``,
``BACKEND_COUNTS``; packed_backend.py:38-303). How they run on MI355X:

* ``PagedPackedCache`` asks the pool once per forward for a ``PageTable`` (page
  table, start positions and lengths, uploaded in one copy). Every layer then
  appends K and V with ONE ``wn_append_kv`` launch: quantize, bit-pack and scatter
  into the pool, the table lookup ``table[b, (L_b + i) // S]`` done on the device.
  The reference copies the table back to the host in every layer
  (packed_backend.py:144); nothing here reads device memory.
* ``append_kv`` validates shapes, and that every position lands inside the table
  and every page it names inside the pool, on host copies of the metadata before
  the launch, raising ``UnsupportedLayout`` as the reference raises in its gather.
* Decode (one query token) runs the HIP compressed-domain operator on packed pages,
  the HIP dense operator on unquantized pages. A prefill chunk dequantizes the
  batch's histories on the GPU (``wn_dequantize_history``) into one padded tensor
  and runs ONE SDPA call with a per-sequence offset-causal mask (the reference loops
  over sequences, packed_backend.py:210-246).
* There is no host fallback: a decode on a non-HIP tensor raises.
"""
from __future__ import annotations

import ctypes
import weakref
from collections import Counter

import numpy as np
import torch
import torch.nn.functional as F

from winnow_amd import _lib
from winnow_amd import packed_attention as pa
from winnow_amd.packing import packed_bytes, unpack
from winnow_amd.page_pool import PagePool, PageTable
from winnow_amd.quantizer import get_quantizer

ATTN_NAME = "winnow_packed"
SUPPORTED_ARCH = ("Qwen2ForCausalLM",)
DECODE_BACKENDS = ("hip_packed", "reconstruct_sdpa", "hip_dense", "dense_sdpa")

# Attention calls served per backend (packed_backend.py:38-40); tests read it to see
# which operator ran.
BACKEND_COUNTS: Counter = Counter()


class UnsupportedModel(ValueError):
    pass


def head_dim_of(config) -> int:
    return getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads


# (what is wrong, test) pairs of the model contract (packed_backend.py:58-68)
_MODEL_RULES = (
    (lambda c: f"{_arch(c)} is not a supported architecture {SUPPORTED_ARCH}",
     lambda c: _arch(c) not in SUPPORTED_ARCH),
    (lambda c: "sliding-window attention is not supported",
     lambda c: bool(getattr(c, "use_sliding_window", False))),
    (lambda c: f"layer types {sorted(set(c.layer_types))} are not all full attention",
     lambda c: any(t != "full_attention" for t in (getattr(c, "layer_types", None) or ()))),
)


def _arch(config) -> str:
    return (getattr(config, "architectures", None) or ["?"])[0]


def check_model(config, bit_width: int) -> None:
    """Reject a model this path does not serve before it is loaded; ``ValueError`` when
    ``head_dim * bit_width`` is not a whole number of bytes."""
    for message, broken in _MODEL_RULES:
        if broken(config):
            raise UnsupportedModel(message(config))
    packed_bytes(head_dim_of(config), bit_width)


def make_pool(config, *, bit_width: int | None, num_pages: int, page_size: int, device,
              max_pages_per_request=None, fence_factory=None,
              dense_dtype: torch.dtype | None = None) -> PagePool:
    """A pool for every layer of ``config``: packed at ``bit_width``, or unquantized rows
    of ``dense_dtype`` (packed_backend.py:75-85)."""
    D = head_dim_of(config)
    row = D if dense_dtype is not None else packed_bytes(D, bit_width)
    return PagePool(num_layers=config.num_hidden_layers, num_pages=num_pages,
                    num_kv_heads=config.num_key_value_heads, page_size=page_size, nb_k=row, nb_v=row,
                    device=device, max_pages_per_request=max_pages_per_request,
                    fence_factory=fence_factory, dense_dtype=dense_dtype)


def quantizers_for(config, bit_width: int, device, k_seed: int = 42, v_seed: int = 42):
    """The K and V quantizers; rotation seeds 42 and 42 by default (packed_backend.py:298-303)."""
    D = head_dim_of(config)
    return get_quantizer(bit_width, D, device, seed=k_seed), get_quantizer(bit_width, D, device, seed=v_seed)


# ---------------------------------------------------------------------------- append

def _positions_in_range(start: torch.Tensor, table: torch.Tensor, n: int, num_pages: int,
                        page_size: int) -> None:
    """Every position start[b] + i (i < n) lies inside row b of the table and names a
    page in [0, num_pages). Reads host tensors only (in numpy: small-array operations
    cost far less host time there than in torch)."""
    start = start.detach().numpy().astype(np.int64)
    width = table.shape[1]
    if n == 0 or start.size == 0:
        return
    out = (start < 0) | (start + n > width * page_size)
    if out.any():
        b = int(np.flatnonzero(out)[0])
        raise pa.UnsupportedLayout(f"append: sequence {b} writes positions {int(start[b])}.."
                                   f"{int(start[b]) + n - 1} outside its {width}-page table row")
    cols = np.arange(width)[None, :]
    first, last = start // page_size, (start + n - 1) // page_size
    touched = (cols >= first[:, None]) & (cols <= last[:, None])
    ids = table.detach().numpy()
    bad = touched & ((ids < 0) | (ids >= num_pages))
    if bad.any():
        b = int(np.flatnonzero(bad.any(1))[0])
        raise pa.UnsupportedLayout(f"append: sequence {b} writes to a page outside [0, {num_pages})")


class AppendPlan:
    """The operands of ``append_kv`` that stay the same from one step of a layer to the
    next: its pages, norms and quantizers, checked once here. ``bind`` checks the
    step's K/V, page table and start positions, ``launch`` calls ``wn_append_kv`` with
    the other arguments built once. On the decode path the wrapper's checks and the
    conversion of forty C arguments otherwise cost more host time than the kernel
    takes on the GPU.

    Raises ``UnsupportedLayout`` for operands off the GPU or of the wrong shape."""

    def __init__(self, k_tq, v_tq, k_pages: torch.Tensor, v_pages: torch.Tensor | None,
                 k_norms: torch.Tensor, v_norms: torch.Tensor | None):
        self.has_v = v_pages is not None or v_norms is not None or v_tq is not None
        ops = [k_pages, k_norms] + ([v_pages, v_norms] if self.has_v else [])
        if any(t is None for t in ops) or (self.has_v and v_tq is None):
            raise pa.UnsupportedLayout("append: V needs its pages and norms")
        if not all(_lib.is_hip(t) for t in ops) or len({t.device for t in ops}) != 1:
            raise pa.UnsupportedLayout("append: every operand must be on one HIP device")
        if k_pages.dim() != 4:
            raise pa.UnsupportedLayout(f"append: pages must be (P, Hkv, S, NB), got {tuple(k_pages.shape)}")
        self.device = k_pages.device
        self.dev_index = k_pages.get_device()
        self.P, self.Hkv, self.S = k_pages.shape[0], k_pages.shape[1], k_pages.shape[2]
        self.D = D = k_tq.Pi.shape[-1]
        P, Hkv, S = self.P, self.Hkv, self.S
        sides = [(k_pages, k_norms, k_tq)] + ([(v_pages, v_norms, v_tq)] if self.has_v else [])
        for pages, norms, tq in sides:
            nb = packed_bytes(D, tq.bit_width)
            if pages.dtype != torch.uint8 or pages.shape != (P, Hkv, S, nb) or pages.stride(-1) != 1 \
                    or pages.stride(-2) != nb:
                raise pa.UnsupportedLayout(f"append: pages must be (P={P}, Hkv={Hkv}, S={S}, NB={nb}) uint8 "
                                           f"with contiguous rows, got {tuple(pages.shape)}")
            if norms.dtype != torch.float16 or norms.shape != (P, Hkv, S) or norms.stride(-1) != 1:
                raise pa.UnsupportedLayout("append: norms must be (P, Hkv, S) fp16 with a contiguous slot axis")
            if tq.Pi.shape != (D, D) or tq.Pi.device != self.device or tq.boundaries.numel() != 2 ** tq.bit_width - 1:
                raise pa.UnsupportedLayout("append: quantizer does not match head_dim or device")
        self._keep = (k_tq, v_tq, k_pages, v_pages, k_norms, v_norms)   # the pointers below stay valid
        # the C arguments of these operands, as plain integers (None: no V side)
        self._quant = (k_tq.Pi.data_ptr(), k_tq.boundaries.data_ptr(), k_tq.bit_width,
                       *((v_tq.Pi.data_ptr(), v_tq.boundaries.data_ptr(), v_tq.bit_width) if self.has_v
                         else (None, None, 0)))
        self._store = (k_pages.data_ptr(), k_pages.stride(0), k_pages.stride(1),
                       *((v_pages.data_ptr(), v_pages.stride(0), v_pages.stride(1)) if self.has_v
                         else (None, 0, 0)),
                       k_norms.data_ptr(), k_norms.stride(0), k_norms.stride(1),
                       *((v_norms.data_ptr(), v_norms.stride(0), v_norms.stride(1)) if self.has_v
                         else (None, 0, 0)))

    def bind(self, k: torch.Tensor, v: torch.Tensor | None, page_table: torch.Tensor,
             start_pos: torch.Tensor) -> tuple:
        """Check one step's operands; returns what ``launch`` takes (None: nothing to write)."""
        if (v is not None) != self.has_v:
            raise pa.UnsupportedLayout("append: V needs its pages and norms" if v is not None
                                       else "append: the pages hold V, but no V was given")
        for t in ((k, page_table, start_pos, v) if v is not None else (k, page_table, start_pos)):
            if t is None or not t.is_cuda or t.get_device() != self.dev_index:
                raise pa.UnsupportedLayout("append: every operand must be on one HIP device")
        if k.dim() != 4:
            raise pa.UnsupportedLayout(f"append: K must be (B, Hkv, n, D), got {tuple(k.shape)}")
        B, Hkv, n, D = k.shape
        if v is not None and v.shape != k.shape:
            raise pa.UnsupportedLayout(f"append: V {tuple(v.shape)} differs from K {tuple(k.shape)}")
        if Hkv != self.Hkv or D != self.D:
            raise pa.UnsupportedLayout(f"append: K {tuple(k.shape)} does not match pages of {self.Hkv} kv heads "
                                       f"and a quantizer of head_dim {self.D}")
        if k.dtype not in _lib.DTYPE_CODE:
            k = k.float()
        if v is not None and v.dtype != k.dtype:
            v = v.to(k.dtype)
        if k.stride(-1) != 1 or (v is not None and v.stride(-1) != 1):
            raise pa.UnsupportedLayout("append: K/V need a contiguous head_dim")
        if page_table.dtype != torch.int32 or page_table.dim() != 2 or page_table.shape[0] != B \
                or page_table.stride(-1) != 1:
            raise pa.UnsupportedLayout("append: page_table must be (B, max_pages) int32 with contiguous rows")
        if start_pos.dtype != torch.int32 or start_pos.shape != (B,):
            raise pa.UnsupportedLayout("append: start_pos must be (B,) int32")
        return (k, v, page_table, start_pos, B, n)

    def launch(self, bound: tuple, timing_events=None) -> None:
        k, v, page_table, start_pos, B, n = bound
        if B == 0 or n == 0:
            return
        # raw integers for the pointers and strides: ctypes converts them faster than
        # it takes c_void_p objects built in Python
        ks = k.stride()
        if v is not None:
            vs = v.stride()
            vargs = (v.data_ptr(), vs[0], vs[1], vs[2])
        else:
            vargs = (None, 0, 0, 0)
        ev0, ev1 = timing_events or (None, None)
        args = (k.data_ptr(), ks[0], ks[1], ks[2], *vargs, _lib.DTYPE_CODE[k.dtype], *self._quant,
                page_table.data_ptr(), page_table.stride(0), start_pos.data_ptr(), *self._store,
                B, self.Hkv, n, self.D, self.S, self.P, page_table.shape[1])
        if torch.cuda.current_device() == self.dev_index:
            _lib.call("wn_append_kv", *args, _lib.stream_of(self.device), ev0, ev1)
        else:
            with torch.cuda.device(self.device):
                _lib.call("wn_append_kv", *args, _lib.stream_of(self.device), ev0, ev1)


# AppendPlans of the layers of live pools, built on a layer's first append and kept
# with the pool tensors they were built on (a plan is rebuilt if those are replaced)
_APPEND_PLANS: "weakref.WeakKeyDictionary[PagePool, dict]" = weakref.WeakKeyDictionary()


def _layer_append_plan(pool: PagePool, layer: int, kq, vq) -> AppendPlan:
    plans = _APPEND_PLANS.get(pool)
    if plans is None:
        plans = _APPEND_PLANS[pool] = {}
    key = (layer, id(kq), id(vq))
    hit = plans.get(key)
    whole = (pool.k_pages, pool.v_pages, pool.k_norms, pool.v_norms)
    ptrs = tuple(t.data_ptr() for t in whole)   # a tensor given new storage in place gets a new plan
    if hit is not None and hit[1] == ptrs and all(a is b for a, b in zip(hit[0], whole)):
        return hit[2]
    plan = AppendPlan(kq, vq, pool.k_pages[layer], pool.v_pages[layer], pool.k_norms[layer], pool.v_norms[layer])
    plans[key] = (whole, ptrs, plan)
    return plan


@torch.no_grad()
def append_kv(k: torch.Tensor, v: torch.Tensor | None, k_tq, v_tq,
              k_pages: torch.Tensor, v_pages: torch.Tensor | None,
              k_norms: torch.Tensor, v_norms: torch.Tensor | None,
              page_table: torch.Tensor, start_pos: torch.Tensor, *,
              page_table_host: torch.Tensor | None = None,
              start_pos_host: torch.Tensor | None = None,
              check_ranges: bool = True, timing_events=None) -> None:
    """Quantize, pack and scatter (B, Hkv, n, D) K (and V, unless ``v`` is None) into one
    layer's pages in one launch; token i of sequence b lands at position
    ``start_pos[b] + i``: page ``page_table[b, pos // S]``, slot ``pos % S``
    (packed_backend.py:143-161).

    Raises ``UnsupportedLayout`` before the launch for operands off the GPU or of the
    wrong shape, and (``check_ranges``) for a position beyond the table row or a page
    id outside the pool. The range check reads ``page_table_host`` /
    ``start_pos_host`` when given, else copies the two small tensors to the host.
    ``timing_events`` is an optional pair of raw ``hipEvent_t`` handles recorded
    around the kernel. A caller that appends to the same pages step after step can
    keep an ``AppendPlan`` and skip the checks of the parts that do not change.
    """
    if v is not None and (v_pages is None or v_norms is None):
        raise pa.UnsupportedLayout("append: V needs its pages and norms")
    has_v = v is not None   # without V, its pages, norms and quantizer are not used
    plan = AppendPlan(k_tq, v_tq if has_v else None, k_pages, v_pages if has_v else None,
                      k_norms, v_norms if has_v else None)
    bound = plan.bind(k, v, page_table, start_pos)
    if check_ranges:
        table = page_table_host if page_table_host is not None else page_table.cpu()
        start = start_pos_host if start_pos_host is not None else start_pos.cpu()
        _positions_in_range(start, table, bound[5], plan.P, plan.S)
    plan.launch(bound, timing_events)


def _append_dense_rows(src: torch.Tensor, pages: torch.Tensor, meta: PageTable) -> None:
    """Unquantized append: row (page, h, slot) of a contiguous (P, Hkv, S, D) layer is
    flat row (page * Hkv + h) * S + slot; the addresses are formed on the device."""
    B, Hkv, n, D = src.shape
    S = pages.shape[2]
    dev = src.device
    pos = meta.start.to(torch.int64)[:, None] + torch.arange(n, device=dev)[None, :]          # (B, n)
    page = meta.table.to(torch.int64).gather(1, pos // S)                                       # (B, n)
    heads = torch.arange(Hkv, device=dev)
    rows = (page[:, :, None] * Hkv + heads[None, None, :]) * S + (pos % S)[:, :, None]           # (B, n, Hkv)
    flat = pages.view(-1, D)
    flat.index_copy_(0, rows.reshape(-1), src.permute(0, 2, 1, 3).reshape(-1, D).to(pages.dtype))


class PagedPackedCache:
    """Duck-typed transformers cache for one forward over pool-backed sequences.

    ``owners[b]`` names the lease whose pages hold sequence b and ``lengths[b]`` the
    tokens it already stores. A forward appends the same n tokens to every sequence
    (n = 1 for a batched decode step, a chunk for a single-sequence prefill); the
    lengths advance once the last layer has written (packed_backend.py:88-112).
    """

    def __init__(self, pool: PagePool, owners, lengths, *, k_quant, v_quant,
                 head_dim: int, decode_backend: str = "auto", allow_tf32: bool = False):
        if len(owners) != len(lengths):
            raise ValueError("one length per owner")
        self.pool = pool
        self.owners = list(owners)
        self.lengths = [int(L) for L in lengths]
        self.kq, self.vq = k_quant, v_quant
        self.head_dim = head_dim
        self.decode_backend = decode_backend
        # TF32-class decode products (the operator's allow_tf32; the reference reaches
        # it through its tuned schedule, packed_backend.py:248-257, which is bypassed)
        self.allow_tf32 = allow_tf32
        self.meta: PageTable | None = None

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if any(L != self.lengths[0] for L in self.lengths):
            raise RuntimeError("mixed lengths: pass explicit position_ids")
        return self.lengths[0] if self.lengths else 0

    def begin(self, n: int, device) -> PageTable:
        """Page metadata of this forward: checked against the pool's leases (a short or
        released lease raises ``StalePage``; pages are never granted here), range-checked
        on the host, and uploaded to ``device`` in one copy."""
        meta = self.pool.batch_table(self.owners, self.lengths, n)
        _positions_in_range(meta.start_host, meta.table_host, n, self.pool.num_pages, self.pool.page_size)
        self.meta = meta.to(device)
        return self.meta

    @torch.no_grad()
    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        B, Hkv, n, D = key_states.shape
        if B != len(self.owners):
            raise RuntimeError(f"batch {B} != {len(self.owners)} owners")
        if layer_idx == 0 or self.meta is None:
            self.begin(n, key_states.device)
        meta, pool = self.meta, self.pool
        if pool.dense:
            _append_dense_rows(key_states, pool.k_pages[layer_idx], meta)
            _append_dense_rows(value_states, pool.v_pages[layer_idx], meta)
            handle = pa.DenseKV(pool.k_pages[layer_idx], pool.v_pages[layer_idx], meta.table, meta.seq, D,
                                seq_lens_host=meta.seq_host, page_table_host=meta.table_host)
        else:
            plan = _layer_append_plan(pool, layer_idx, self.kq, self.vq)
            plan.launch(plan.bind(key_states, value_states, meta.table, meta.start))  # ranges: begin()
            handle = pa.PackedKV(pool.k_pages[layer_idx], pool.k_norms[layer_idx],
                                 pool.v_pages[layer_idx], pool.v_norms[layer_idx],
                                 meta.table, meta.seq, pa.Quantizer.from_tq(self.kq),
                                 pa.Quantizer.from_tq(self.vq), D,
                                 seq_lens_host=meta.seq_host, page_table_host=meta.table_host)
        handle.decode_backend = self.decode_backend
        handle.allow_tf32 = self.allow_tf32
        if layer_idx == pool.num_layers - 1:
            self.lengths = meta.seq_host.tolist()
        return handle, handle


# ---------------------------------------------------------------------------- attention

def select_decode_backend(query: torch.Tensor, kv, requested: str) -> str:
    """The operator that serves a one-token decode step (packed_backend.py:173-189).

    Packed pages: ``auto`` (and the reference's ``triton_packed``) is the HIP operator;
    ``reconstruct_sdpa`` is the dequantize-then-SDPA path. Dense pages: the HIP dense
    operator where it compiles the shape, else dense SDPA. Requests that cannot be
    served raise; nothing falls back to the host."""
    if isinstance(kv, pa.DenseKV):
        if requested == "dense_sdpa":
            return requested
        if requested not in ("auto", "triton_dense", "hip_dense"):
            raise ValueError(f"backend {requested!r} does not read dense pages")
        if not _lib.is_hip(query):
            raise RuntimeError("the dense decode operator needs a HIP device; there is no host fallback")
        if pa.dense_supported(query, kv):
            return "hip_dense"
        if requested == "hip_dense":
            raise ValueError("hip_dense does not compile this shape (head_dim 16-256, fp32/bf16/fp16 pages, S >= 16)")
        return "dense_sdpa"
    if requested in ("auto", "triton_packed", "hip_packed"):
        if not _lib.is_hip(query):
            raise RuntimeError("the packed decode operator needs a HIP device; there is no host fallback")
        return "hip_packed"
    if requested not in DECODE_BACKENDS:
        raise ValueError(f"unknown decode backend {requested!r}")
    return requested


def prefill_fused(query: torch.Tensor, kv) -> bool:
    """Whether a Q > 1 step runs the fused prefill over the packed pages
    (``packed_prefill_attention``) instead of the reference's dequantize-then-SDPA
    route (packed_backend.py:278-280). The fused scan takes single fp16 operands: it
    serves bf16 and fp16 queries, whose reference route computes in bf16 / fp16 SDPA
    over a history dequantized to that type, and fp32 queries only when the handle
    allows TF32-class products (``allow_tf32``); otherwise an fp32 query keeps the
    fp32 reconstruct route, as in the reference. Shapes the scan does not compile
    (``prefill_supported``) keep the reconstruct route too."""
    if query.dtype == torch.float32 and not getattr(kv, "allow_tf32", False):
        return False
    return pa.prefill_supported(query, kv)


def _host_lens(kv) -> torch.Tensor:
    return kv.seq_lens_host if kv.seq_lens_host is not None else kv.seq_lens.cpu()


def _host_table(kv) -> torch.Tensor:
    return kv.page_table_host if kv.page_table_host is not None else kv.page_table.cpu()


def dequantize_history(kv: pa.PackedKV, pages, norms, quant, b: int, dtype) -> torch.Tensor:
    """(1, Hkv, L, D) reconstruction of sequence b's history, on the GPU (packed_backend.py:192-208).

    head_dim 128 with contiguous page rows: one ``wn_dequantize_history`` launch reads
    the pool pages through the table row. Other shapes gather the rows, unpack and
    dequantize with the standalone kernels."""
    L = int(_host_lens(kv)[b])
    S, D, Hkv = kv.page_size, kv.head_dim, pages.shape[1]
    odt = dtype if dtype in _lib.DTYPE_CODE else torch.float32
    out = torch.empty(1, Hkv, L, D, dtype=odt, device=pages.device)
    if L == 0:
        return out.to(dtype)
    fused = D == 128 and pages.stride(-1) == 1 and pages.stride(-2) == pages.shape[-1] and norms.stride(-1) == 1
    with torch.cuda.device(pages.device):
        if fused:
            _lib.call("wn_dequantize_history", _lib.ptr(pages), pages.stride(0), pages.stride(1),
                      _lib.ptr(norms), norms.stride(0), norms.stride(1), _lib.ptr(kv.page_table[b]), L, Hkv, S,
                      _lib.ptr(quant.centroids), _lib.ptr(quant.Pi), quant.bit_width, D, _lib.ptr(out),
                      _lib.DTYPE_CODE[odt], 0, _lib.stream_of(pages.device))
        else:
            ids = _host_table(kv)[b, :-(-L // S)].to(torch.int64).to(pages.device)
            rows = pages[ids].transpose(0, 1).reshape(Hkv, -1, pages.shape[-1])[:, :L].contiguous()
            nrm = norms[ids].transpose(0, 1).reshape(Hkv, -1)[:, :L].contiguous()
            codes = unpack(rows, quant.bit_width, D).contiguous()
            _lib.call("wn_dequantize", _lib.ptr(codes), _lib.ptr(nrm), Hkv * L, _lib.ptr(quant.Pi),
                      _lib.ptr(quant.centroids), quant.bit_width, D, _lib.ptr(out), _lib.DTYPE_CODE[odt],
                      _lib.stream_of(pages.device))
    return out.to(dtype)


def _offset_causal(lens: torch.Tensor, Q: int, Lmax: int, device):
    """(B, 1, Q, Lmax) mask: query i of a sequence of length L sees keys j <= L - Q + i,
    and (B, 1, Q, 1) whether the row sees any key (packed_attention.py:200-205)."""
    last = lens.to(torch.int64)[:, None] - Q + torch.arange(Q)[None, :]                         # (B, Q)
    mask = torch.arange(Lmax)[None, None, :] <= last[:, :, None]
    return mask[:, None].to(device), (last >= 0)[:, None, :, None].to(device)


def _padded_sdpa(query, k, v, lens, scaling):
    """One SDPA call over histories padded to the longest; rows without a key are 0."""
    B, Hq, Q, _ = query.shape
    mask, live = _offset_causal(lens, Q, k.shape[2], query.device)
    out = F.scaled_dot_product_attention(query, k, v, attn_mask=mask, scale=scaling,
                                         enable_gqa=Hq != k.shape[1])
    return torch.where(live, out, torch.zeros((), dtype=out.dtype, device=out.device))


def _reconstruct_sdpa(query, kv: pa.PackedKV, scaling):
    """Dequantize every sequence's history on the GPU into one padded (B, Hkv, Lmax, D)
    pair, then one offset-causal SDPA over the batch (packed_backend.py:211-226)."""
    B, Hq, Q, D = query.shape
    lens = _host_lens(kv).to(torch.int64)
    Lmax = int(lens.max()) if B else 0
    if Lmax == 0:
        return torch.zeros(B, Hq, Q, D, dtype=query.dtype, device=query.device)
    hist = []
    for pages, norms, quant in ((kv.k_pages, kv.k_norms, kv.k_quant), (kv.v_pages, kv.v_norms, kv.v_quant)):
        buf = torch.zeros(B, kv.num_kv_heads, Lmax, D, dtype=query.dtype, device=query.device)
        for b in range(B):
            if lens[b]:
                buf[b, :, :int(lens[b])] = dequantize_history(kv, pages, norms, quant, b, query.dtype)[0]
        hist.append(buf)
    return _padded_sdpa(query, hist[0], hist[1], lens, scaling)


def _dense_sdpa(query, kv: pa.DenseKV, scaling):
    """Gather every sequence's unquantized rows into one padded (B, Hkv, Lmax, D) pair with
    one indexed read per side, then one offset-causal SDPA (packed_backend.py:229-246)."""
    B, Hq, Q, D = query.shape
    lens = _host_lens(kv).to(torch.int64)
    Lmax = int(lens.max()) if B else 0
    if Lmax == 0:
        return torch.zeros(B, Hq, Q, D, dtype=query.dtype, device=query.device)
    S = kv.page_size
    t = torch.arange(Lmax)
    table = _host_table(kv).to(torch.int64)
    page = table[:, t // S].clamp(min=0)                        # padding reads page 0; masked out
    page = torch.where(t[None, :] < lens[:, None], page, torch.zeros_like(page)).to(query.device)
    slot = (t % S).to(query.device)[None, :].expand(B, Lmax)
    k = kv.k_pages[page, :, slot].permute(0, 2, 1, 3).to(query.dtype)         # (B, Hkv, Lmax, D)
    v = kv.v_pages[page, :, slot].permute(0, 2, 1, 3).to(query.dtype)
    return _padded_sdpa(query, k, v, lens, scaling)


def _hip_packed(query, kv, scaling):
    return pa.packed_decode_attention(query, kv, scaling, allow_tf32=getattr(kv, "allow_tf32", False))


def _hip_dense(query, kv, scaling):
    return pa.dense_decode_attention(query, kv, scaling)


def _hip_prefill(query, kv, scaling):
    return pa.packed_prefill_attention(query, kv, scaling)


_ROUTES = {
    "hip_packed": _hip_packed,
    "reconstruct_sdpa": _reconstruct_sdpa,
    "prefill_reconstruct_sdpa": _reconstruct_sdpa,
    "prefill_hip_packed": _hip_prefill,
    "hip_dense": _hip_dense,
    "dense_sdpa": _dense_sdpa,
    "prefill_dense_sdpa": _dense_sdpa,
}


def _route(query, kv) -> str:
    if query.shape[2] > 1:
        if isinstance(kv, pa.DenseKV):
            return "prefill_dense_sdpa"
        return "prefill_hip_packed" if prefill_fused(query, kv) else "prefill_reconstruct_sdpa"
    return select_decode_backend(query, kv, getattr(kv, "decode_backend", "auto"))


def winnow_packed_attention(module, query, key, value, attention_mask, dropout: float = 0.0,
                            scaling=None, **kwargs):
    """``AttentionInterface`` entry point: ``(B, Q, Hq, D), None`` (packed_backend.py:260-290).

    A cache handle as ``key`` routes by page kind and query length; plain tensors go to
    transformers' SDPA, counted as ``native_sdpa``."""
    scale = query.shape[-1] ** -0.5 if scaling is None else scaling
    if not isinstance(key, (pa.PackedKV, pa.DenseKV)):
        from transformers.integrations.sdpa_attention import sdpa_attention_forward
        BACKEND_COUNTS["native_sdpa"] += 1
        return sdpa_attention_forward(module, query, key, value, attention_mask, dropout=dropout,
                                      scaling=scale, **kwargs)
    route = _route(query, key)
    BACKEND_COUNTS[route] += 1
    return _ROUTES[route](query, key, scale).transpose(1, 2).contiguous(), None


def register() -> None:
    from transformers import AttentionInterface
    AttentionInterface.register(ATTN_NAME, winnow_packed_attention)
