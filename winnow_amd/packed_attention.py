"""Decode attention over paged packed KV, computed in the compressed domain on MI355X.

Drop-in for the operator API of ``turboquant_kv/packed_attention.py`` (the
``UnsupportedLayout`` error, the ``Quantizer`` / ``PackedKV`` / ``DenseKV``
handles, ``check_contract``, ``kv_head_for``, ``default_scale``) and of
``turboquant_kv/packed_attention_triton.py`` (``packed_decode_attention``,
``check_kernel_contract``). The algebra is the reference's
(packed_attention.py:1-21):

    q . k_hat_j = n_K,j (q Pi_K^T) . c_K,j          sum_j p_j v_hat_j = (sum_j p_j n_V,j c_V,j) Pi_V

so the query is rotated once, every key is read as packed codes plus one fp16
norm, and the softmax-weighted value sum is accumulated in the value
quantizer's basis and rotated back once per output row. The work runs in the
``wn_decode_attention`` HIP entry point (rotate-q, split-K page scan, merge +
output rotation); nothing here computes attention on the host.

Page layout (packed_attention.py:23-28):

    k_pages, v_pages   (P, Hkv, S, NB) uint8   NB = D*bw/8, LSB-first codes
    k_norms, v_norms   (P, Hkv, S)     fp16
    page_table         (B, max_pages)  int32   -1 past the last page
    seq_lens           (B,)            int32
"""
from __future__ import annotations

import ctypes
import functools
import math
from dataclasses import dataclass

import numpy as np
import torch

from winnow_amd import _lib
from winnow_amd.packing import packed_bytes

SUPPORTED_HEAD_DIMS = (16, 32, 64, 128, 256)


class UnsupportedLayout(ValueError):
    """Raised before any launch when inputs violate the operator contract
    (packed_attention.py:55-56)."""


@dataclass(frozen=True)
class Quantizer:
    """The pieces of a ``TurboQuantMSE`` the attention operator reads (packed_attention.py:59-69)."""

    Pi: torch.Tensor          # (D, D) fp32, orthogonal
    centroids: torch.Tensor   # (2**bw,) fp32
    bit_width: int

    @classmethod
    def from_tq(cls, tq) -> "Quantizer":
        return cls(tq.Pi, tq.centroids, tq.bit_width)


@dataclass
class PackedKV:
    """Paged packed K/V plus the per-sequence view of it (packed_attention.py:72-92).

    ``seq_lens_host`` / ``page_table_host`` are optional CPU mirrors of the two
    metadata tensors. When present, ``check_contract`` validates against them and
    the decode call never synchronises with the device.
    """

    k_pages: torch.Tensor
    k_norms: torch.Tensor
    v_pages: torch.Tensor
    v_norms: torch.Tensor
    page_table: torch.Tensor
    seq_lens: torch.Tensor
    k_quant: Quantizer
    v_quant: Quantizer
    head_dim: int
    seq_lens_host: torch.Tensor | None = None
    page_table_host: torch.Tensor | None = None

    @property
    def page_size(self) -> int:
        return self.k_pages.shape[2]

    @property
    def num_kv_heads(self) -> int:
        return self.k_pages.shape[1]


@dataclass
class DenseKV:
    """Unquantized paged K/V: pages (P, Hkv, S, D) in the model dtype (packed_attention.py:95-111).

    ``seq_lens_host`` / ``page_table_host`` are optional CPU mirrors, read by the range
    checks in place of the device tensors, as on ``PackedKV``.
    """

    k_pages: torch.Tensor
    v_pages: torch.Tensor
    page_table: torch.Tensor
    seq_lens: torch.Tensor
    head_dim: int
    seq_lens_host: torch.Tensor | None = None
    page_table_host: torch.Tensor | None = None

    @property
    def page_size(self) -> int:
        return self.k_pages.shape[2]

    @property
    def num_kv_heads(self) -> int:
        return self.k_pages.shape[1]


def kv_head_for(q_head: torch.Tensor, n_rep: int) -> torch.Tensor:
    """Query head -> kv head under grouped-query attention (``repeat_kv`` order)."""
    return q_head // n_rep


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


@torch.no_grad()
def pages_from_dense(k: torch.Tensor, v: torch.Tensor, seq_lens, k_tq, v_tq, page_size: int,
                     num_pages: int | None = None, generator: torch.Generator | None = None) -> PackedKV:
    """Quantize dense (B, Hkv, Lmax, D) K/V on the GPU into pages taken in a random order
    (packed_attention.py:341-377). Unused table slots hold -1 and the bytes of a page past
    its sequence's last token stay zero. The page order comes from
    ``torch.randperm(total, generator)`` on the host, as the reference draws it, so a
    generator in the same state gives the reference's page table. Each sequence's
    history goes through one ``wn_append_kv`` launch (quantize, pack, scatter).

    K and V must be on a HIP device; the handle carries host mirrors of its table and
    lengths."""
    from winnow_amd.packed_backend import append_kv

    B, Hkv, _, D = k.shape
    lens = [int(x) for x in seq_lens]
    need = [(L + page_size - 1) // page_size for L in lens]
    total = num_pages or max(sum(need), 1)
    order = torch.randperm(total, generator=generator).tolist()
    dev = k.device
    kp = torch.zeros(total, Hkv, page_size, packed_bytes(D, k_tq.bit_width), dtype=torch.uint8, device=dev)
    vp = torch.zeros(total, Hkv, page_size, packed_bytes(D, v_tq.bit_width), dtype=torch.uint8, device=dev)
    kn = torch.zeros(total, Hkv, page_size, dtype=torch.float16, device=dev)
    vn = torch.zeros(total, Hkv, page_size, dtype=torch.float16, device=dev)
    table = torch.full((B, max(max(need, default=0), 1)), -1, dtype=torch.int32)
    nxt = 0
    for b in range(B):
        table[b, :need[b]] = torch.tensor(order[nxt:nxt + need[b]], dtype=torch.int32)
        nxt += need[b]
    dtable = table.to(dev)
    zero = torch.zeros(1, dtype=torch.int32)
    dzero = zero.to(dev)
    for b in range(B):
        if lens[b]:
            append_kv(k[b:b + 1, :, :lens[b]], v[b:b + 1, :, :lens[b]], k_tq, v_tq, kp, vp, kn, vn,
                      dtable[b:b + 1], dzero, page_table_host=table[b:b + 1], start_pos_host=zero)
    return PackedKV(kp, kn, vp, vn, dtable, torch.tensor(lens, dtype=torch.int32, device=dev),
                    Quantizer.from_tq(k_tq), Quantizer.from_tq(v_tq), D,
                    seq_lens_host=torch.tensor(lens, dtype=torch.int32), page_table_host=table)


def check_contract(q: torch.Tensor, kv: PackedKV, *, check_ranges: bool = True) -> None:
    """Reject anything the operator does not support, with the reason (packed_attention.py:114-163).

    q is (B, Hq, Q, D). The sequence-length and page-id range checks read the
    host mirrors when the handle carries them; otherwise they copy the two small
    metadata tensors to the host, as the reference does. ``check_ranges=False``
    skips only those two checks, for callers that own the metadata.
    """
    if q.dim() != 4:
        raise UnsupportedLayout(f"q must be (B, Hq, Q, D), got {tuple(q.shape)}")
    B, Hq, _, D = q.shape
    if D != kv.head_dim:
        raise UnsupportedLayout(f"q head_dim {D} != cache head_dim {kv.head_dim}")
    for name, quant in (("k", kv.k_quant), ("v", kv.v_quant)):
        if quant.Pi.shape != (D, D) or quant.Pi.dtype != torch.float32:
            raise UnsupportedLayout(f"{name} rotation must be fp32 ({D}, {D})")
        if quant.centroids.dtype != torch.float32 or quant.centroids.numel() != 2 ** quant.bit_width:
            raise UnsupportedLayout(f"{name} codebook must be fp32 with 2**bw entries")
    try:
        nb_k = packed_bytes(D, kv.k_quant.bit_width)
        nb_v = packed_bytes(D, kv.v_quant.bit_width)
    except ValueError as e:
        raise UnsupportedLayout(str(e)) from e
    P, Hkv, S = kv.k_pages.shape[:3]
    if kv.k_pages.dtype != torch.uint8 or kv.v_pages.dtype != torch.uint8:
        raise UnsupportedLayout("packed pages must be uint8")
    if kv.k_pages.shape != (P, Hkv, S, nb_k) or kv.v_pages.shape[:3] != (P, Hkv, S) \
            or kv.v_pages.shape[3] != nb_v:
        raise UnsupportedLayout(
            f"page shapes {tuple(kv.k_pages.shape)}/{tuple(kv.v_pages.shape)} do not "
            f"match (P, Hkv, S, NB) with NB={nb_k}/{nb_v}")
    if kv.k_norms.shape != (P, Hkv, S) or kv.v_norms.shape != (P, Hkv, S):
        raise UnsupportedLayout("norms must be (P, Hkv, S)")
    if kv.k_norms.dtype != torch.float16 or kv.v_norms.dtype != torch.float16:
        raise UnsupportedLayout("norms must be fp16")
    if Hq % Hkv:
        raise UnsupportedLayout(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if kv.page_table.dim() != 2 or kv.page_table.shape[0] != B:
        raise UnsupportedLayout("page_table must be (B, max_pages)")
    if kv.seq_lens.shape != (B,):
        raise UnsupportedLayout("seq_lens must be (B,)")
    if kv.page_table.dtype != torch.int32 or kv.seq_lens.dtype != torch.int32:
        raise UnsupportedLayout("page_table and seq_lens must be int32")
    devices = {t.device for t in (q, kv.k_pages, kv.v_pages, kv.k_norms, kv.v_norms,
                                  kv.page_table, kv.seq_lens, kv.k_quant.Pi, kv.v_quant.Pi,
                                  kv.k_quant.centroids, kv.v_quant.centroids)}
    if len(devices) != 1:
        raise UnsupportedLayout(f"all operands must share a device, got {devices}")
    if not check_ranges:
        return
    lens = kv.seq_lens_host if kv.seq_lens_host is not None else kv.seq_lens
    table = kv.page_table_host if kv.page_table_host is not None else kv.page_table
    check_page_ranges(lens, table, P, S)


def check_page_ranges(seq_lens: torch.Tensor, page_table: torch.Tensor, num_pages: int,
                      page_size: int) -> None:
    """Every length fits the table and every page id a sequence reads (those below
    cdiv(len, page_size)) lies in [0, num_pages): the scan kernels index pages with
    these ids unchecked. Copies the two small tensors to the host (host mirrors are
    read in place); the checks run in numpy, whose small-array operations cost far
    less host time than torch's."""
    lens = seq_lens.detach().to("cpu").numpy().astype(np.int64)
    table = page_table.detach().to("cpu").numpy()
    width = table.shape[1]
    if lens.size and (lens.min() < 0 or lens.max() > width * page_size):
        raise UnsupportedLayout("seq_lens out of range for the page table")
    used = (lens + page_size - 1) // page_size
    live = np.arange(width)[None, :] < used[:, None]
    bad = live & ((table < 0) | (table >= num_pages))
    if bad.any():
        b = int(np.flatnonzero(bad.any(1))[0])
        raise UnsupportedLayout(f"sequence {b} references a page outside [0, {num_pages})")


def _pow2(x: int) -> bool:
    return x >= 16 and (x & (x - 1)) == 0


def check_kernel_contract(q: torch.Tensor, kv: PackedKV, *, check_ranges: bool = True) -> None:
    """check_contract plus what the HIP kernel needs (packed_attention_triton.py:166-177)."""
    check_contract(q, kv, check_ranges=check_ranges)
    if q.shape[2] != 1:
        raise UnsupportedLayout("the HIP kernel serves decode (one query token) only")
    if not _lib.is_hip(q):
        raise UnsupportedLayout("the HIP kernel needs tensors on a HIP device")
    if not _pow2(kv.page_size) or not _pow2(kv.head_dim):
        raise UnsupportedLayout("page_size and head_dim must be powers of two >= 16")
    if kv.head_dim not in SUPPORTED_HEAD_DIMS:
        raise UnsupportedLayout(f"head_dim {kv.head_dim} is not compiled {SUPPORTED_HEAD_DIMS}")
    if q.dtype not in _lib.DTYPE_CODE or q.stride(-1) != 1:
        raise UnsupportedLayout("q must be fp32/fp16/bf16 with a contiguous head_dim")
    for pages in (kv.k_pages, kv.v_pages):
        if pages.stride(-1) != 1 or pages.stride(-2) != pages.shape[-1]:
            raise UnsupportedLayout("pages need contiguous (S, NB) rows")
        align = 16 if pages.shape[-1] % 16 == 0 else 8
        if pages.data_ptr() % align or pages.stride(0) % align or pages.stride(1) % align:
            raise UnsupportedLayout(f"page base and strides must be {align}-byte aligned")
        # the scans form a page block's address from page id x page stride in 32 x 32 bits
        if not 0 <= pages.stride(0) < 2 ** 32:
            raise UnsupportedLayout("page strides of 2^32 bytes or more")
    for norms in (kv.k_norms, kv.v_norms):
        if norms.stride(-1) != 1:
            raise UnsupportedLayout("norms need a contiguous slot axis")
        # the scans form norm offsets in 32-bit pieces (page id x page stride, head x
        # head stride + slot)
        if not (0 <= norms.stride(0) < 2 ** 31 and 0 <= norms.stride(1)
                and norms.shape[1] * norms.stride(1) + kv.page_size <= 2 ** 31):
            raise UnsupportedLayout("norm strides of 2^31 elements or more")
    for quant in (kv.k_quant, kv.v_quant):
        if not quant.Pi.is_contiguous() or not quant.centroids.is_contiguous():
            raise UnsupportedLayout("rotations and codebooks must be contiguous")
    if kv.page_table.stride(-1) != 1 or not kv.seq_lens.is_contiguous():
        raise UnsupportedLayout("page_table rows and seq_lens must be contiguous")


def decode_plan(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, page_size: int,
                bits_k: int, bits_v: int, max_pages: int, num_splits: int | None = None,
                allow_tf32: bool = False):
    """(pages_per_split, num_splits) the HIP decode uses for this shape (wn_decode_plan,
    or wn_decode_plan_tf32 for the allow_tf32 decode, whose scan may keep more waves).

    pages_per_split == 0 is a balanced plan: num_splits persistent waves share
    the batch's 64-token chunks equally.
    """
    pps, ns = ctypes.c_int(0), ctypes.c_int(0)
    _lib.call("wn_decode_plan_tf32" if allow_tf32 else "wn_decode_plan", batch, num_q_heads, num_kv_heads,
              head_dim, page_size, bits_k, bits_v, max_pages, int(num_splits or 0), ctypes.byref(pps),
              ctypes.byref(ns))
    return pps.value, ns.value


@functools.lru_cache(maxsize=1024)
def workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                    pages_per_split: int, num_splits: int) -> int:
    return int(_lib.lib().wn_decode_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim,
                                                    pages_per_split, num_splits))


# The library's plan depends only on the shape and on the device (its occupancy), so a
# decode step, which asks for the same shape layer after layer, looks it up once.
@functools.lru_cache(maxsize=1024)
def _device_plan(device_index: int, *shape_and_options) -> tuple[int, int]:
    with torch.cuda.device(device_index):
        return decode_plan(*shape_and_options)


def plan_for(q: torch.Tensor, kv: PackedKV, num_splits: int | None = None, allow_tf32: bool = False):
    """decode_plan for a query and a PackedKV handle, on the query's device."""
    B, Hq, _, D = q.shape
    return _device_plan(q.get_device(), B, Hq, kv.num_kv_heads, D, kv.page_size, kv.k_quant.bit_width,
                        kv.v_quant.bit_width, kv.page_table.shape[1], num_splits, allow_tf32)


def packed_decode_attention(q: torch.Tensor, kv: PackedKV, scale: float, *,
                            num_splits: int | None = None, allow_tf32: bool = False,
                            num_warps: int = 4, num_stages: int = 2, pages_per_iter: int = 1,
                            out_dtype: torch.dtype | None = None,
                            workspace: torch.Tensor | None = None,
                            check_ranges: bool = True,
                            timing_events=None, plan: tuple[int, int] | None = None) -> torch.Tensor:
    """q (B, Hq, 1, D) -> (B, Hq, 1, D) in q.dtype (packed_attention_triton.py:180-187).

    ``num_splits=None`` lets the library plan the split: persistent waves that
    share the batch's chunks equally where the row scan applies, else splits
    sized to fill the GPU; an integer asks for exactly that many splits over the page-table
    width, as the reference does. ``allow_tf32=True`` asks, as in the reference
    (whose kernel hands it to both ``tl.dot`` products), for TF32-class products:
    ``wn_decode_attention_tf32`` runs 4 and 6-bit K and V (alike or mixed) on the row
    scan on single fp16 operands (11 significant bits) with fp32 accumulation, and
    every other shape on the fp32-exact scan. ``num_warps`` and ``num_stages`` are
    Triton schedule knobs, accepted for call compatibility and ignored;
    ``pages_per_iter`` must still be a power of two. ``out_dtype=torch.float32``
    returns the fp32 result before the cast (for parity checks). ``workspace``
    is an optional caller-owned uint8 buffer of at least ``workspace_bytes``.
    ``timing_events`` is an optional pair of raw ``hipEvent_t`` handles recorded
    around the page-scan kernel. ``plan`` = ``(pages_per_split, num_splits)`` replaces
    the library's plan: ``(0, w)`` is a balanced plan over ``w`` waves (each wave then
    scans several chunks when the batch has more than ``w``), ``(p, n)`` with
    ``p * n >= max_pages`` fixed splits.
    """
    del num_warps, num_stages
    if pages_per_iter < 1 or pages_per_iter & (pages_per_iter - 1):
        raise UnsupportedLayout("pages_per_iter must be a power of two >= 1")
    check_kernel_contract(q, kv, check_ranges=check_ranges)
    B, Hq, _, D = q.shape
    Hkv = kv.num_kv_heads
    pps, ns = plan if plan is not None else plan_for(q, kv, num_splits, allow_tf32)
    out_dtype = out_dtype or q.dtype
    if out_dtype not in _lib.DTYPE_CODE:
        raise UnsupportedLayout(f"output dtype {out_dtype} is not supported")
    out = torch.empty(B, Hq, 1, D, dtype=out_dtype, device=q.device)
    need = workspace_bytes(B, Hq, Hkv, D, pps, ns)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != q.device:
        raise UnsupportedLayout(f"workspace needs {need} bytes on {q.device}")
    ev0, ev1 = timing_events or (None, None)
    with torch.cuda.device(q.device):
        entry = "wn_decode_attention_tf32" if allow_tf32 else "wn_decode_attention"
        _lib.call(entry, *_operands(q, kv), _lib.ptr(out), _lib.DTYPE_CODE[out_dtype],
                  _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
                  *_sizes(q, kv), float(scale), pps, ns, _lib.stream_of(q.device), ev0, ev1)
    return out


def _operands(q: torch.Tensor, kv: PackedKV) -> tuple:
    """The C-ABI arguments of a decode from q through seq_lens."""
    qv = q[:, :, 0]
    return (_lib.ptr(qv), _lib.DTYPE_CODE[q.dtype], qv.stride(0), qv.stride(1),
            _lib.ptr(kv.k_quant.Pi), _lib.ptr(kv.v_quant.Pi),
            _lib.ptr(kv.k_quant.centroids), _lib.ptr(kv.v_quant.centroids),
            _lib.ptr(kv.k_pages), kv.k_pages.stride(0), kv.k_pages.stride(1),
            _lib.ptr(kv.v_pages), kv.v_pages.stride(0), kv.v_pages.stride(1),
            _lib.ptr(kv.k_norms), kv.k_norms.stride(0), kv.k_norms.stride(1),
            _lib.ptr(kv.v_norms), kv.v_norms.stride(0), kv.v_norms.stride(1),
            _lib.ptr(kv.page_table), kv.page_table.stride(0), _lib.ptr(kv.seq_lens))


def _sizes(q: torch.Tensor, kv: PackedKV) -> tuple:
    B, Hq, _, D = q.shape
    return (B, Hq, kv.num_kv_heads, D, kv.page_size, kv.k_quant.bit_width, kv.v_quant.bit_width,
            kv.page_table.shape[1])


def packed_decode_attention_noalloc(q: torch.Tensor, kv: PackedKV, scale: float, out: torch.Tensor, *,
                                    num_splits: int | None = None, plan: tuple[int, int] | None = None,
                                    check_ranges: bool = True, timing_events=None) -> torch.Tensor:
    """``packed_decode_attention`` into a caller-owned ``out`` (B, Hq, 1, D), contiguous,
    fp32/fp16/bf16, with no device allocation at all: the scratch is the library's
    static per-GPU array (``wn_decode_attention_noalloc``, 32 MiB). For callers that
    cannot allocate (graph capture, allocation-free serving loops). A shape and plan
    needing more scratch than that raises ``UnsupportedLayout`` before any launch.
    Calls that overlap on one GPU (other streams or threads) share the array and race.
    """
    check_kernel_contract(q, kv, check_ranges=check_ranges)
    B, Hq, _, D = q.shape
    if out.shape != (B, Hq, 1, D) or out.dtype not in _lib.DTYPE_CODE or not out.is_contiguous() \
            or out.device != q.device:
        raise UnsupportedLayout(f"out must be a contiguous ({B}, {Hq}, 1, {D}) fp32/fp16/bf16 tensor on {q.device}")
    pps, ns = plan if plan is not None else plan_for(q, kv, num_splits)
    need = workspace_bytes(B, Hq, kv.num_kv_heads, D, pps, ns)
    if need > _lib.NOALLOC_SCRATCH_BYTES:
        raise UnsupportedLayout(f"this shape and plan need {need} bytes of scratch, more than the "
                                f"{_lib.NOALLOC_SCRATCH_BYTES}-byte static scratch")
    ev0, ev1 = timing_events or (None, None)
    with torch.cuda.device(q.device):
        _lib.call("wn_decode_attention_noalloc", *_operands(q, kv), _lib.ptr(out), _lib.DTYPE_CODE[out.dtype],
                  *_sizes(q, kv), float(scale), pps, ns, _lib.stream_of(q.device), ev0, ev1)
    return out


PREFILL_WIDTHS = (4, 6)


def prefill_supported(q: torch.Tensor, kv: PackedKV) -> bool:
    """Whether ``packed_prefill_attention`` compiles this shape: head_dim 128, page size a
    power of two >= 16, 4 and 6-bit K and V (alike or mixed), a fp32/fp16/bf16 query on
    a HIP device with a contiguous head_dim, norms whose rows the scan reads four at a
    time (bases 8-byte aligned, strides multiples of 4 elements)."""
    if q.dim() != 4 or q.shape[-1] != 128 or kv.head_dim != 128 or not _lib.is_hip(q):
        return False
    if kv.k_quant.bit_width not in PREFILL_WIDTHS or kv.v_quant.bit_width not in PREFILL_WIDTHS:
        return False
    if not _pow2(kv.page_size) or q.dtype not in _lib.DTYPE_CODE or q.stride(-1) != 1:
        return False
    for quant in (kv.k_quant, kv.v_quant):
        if not quant.Pi.is_contiguous() or quant.Pi.data_ptr() % 16 or not quant.centroids.is_contiguous():
            return False
    if kv.page_table.stride(-1) != 1 or not kv.seq_lens.is_contiguous():
        return False
    for n in (kv.k_norms, kv.v_norms):
        if n.stride(-1) != 1 or n.data_ptr() % 8 or n.stride(0) % 4 or n.stride(1) % 4:
            return False
    for pages, align in ((kv.k_pages, 16 if kv.k_quant.bit_width == 4 else 8), (kv.v_pages, 4)):
        if pages.stride(-1) != 1 or pages.stride(-2) != pages.shape[-1] or pages.data_ptr() % align \
                or pages.stride(0) % align or pages.stride(1) % align:
            return False
    return True


def prefill_plan_for(q: torch.Tensor, kv: PackedKV) -> int:
    """Split count of the fused prefill for this query and handle (wn_prefill_plan)."""
    B, Hq, Q, D = q.shape
    lens = kv.seq_lens_host if kv.seq_lens_host is not None else kv.seq_lens.cpu()
    max_len = int(lens.max()) if lens.numel() else 0
    ns = ctypes.c_int(0)
    with torch.cuda.device(q.device):
        _lib.call("wn_prefill_plan", B, Hq, kv.num_kv_heads, Q, D, kv.page_size, kv.k_quant.bit_width,
                  kv.v_quant.bit_width, max_len, ctypes.byref(ns))
    return ns.value


def prefill_workspace_bytes(batch: int, num_q_heads: int, num_kv_heads: int, q_len: int, head_dim: int,
                            num_splits: int) -> int:
    return int(_lib.lib().wn_prefill_workspace_bytes(batch, num_q_heads, num_kv_heads, q_len, head_dim,
                                                     num_splits))


def packed_prefill_attention(q: torch.Tensor, kv: PackedKV, scale: float, *,
                             num_splits: int | None = None, out_dtype: torch.dtype | None = None,
                             workspace: torch.Tensor | None = None, check_ranges: bool = True,
                             timing_events=None) -> torch.Tensor:
    """q (B, Hq, Q, D) -> (B, Hq, Q, D) in q.dtype, read from the packed pages
    (``wn_prefill_attention``): the reference's Q > 1 route (packed_backend.py:211-226,
    dequantize the history and run SDPA with the offset causal mask of
    packed_attention.py:198-206) without writing the history to HBM. Query i of a
    sequence of length L (the cache already holds the Q new tokens) sees keys
    j <= L - Q + i; a query that sees none gives 0.

    Both products take single fp16 operands (11 significant bits, rounded to nearest)
    and accumulate in fp32. ``num_splits`` replaces the library's split count;
    ``out_dtype=torch.float32`` returns the fp32 result before the cast;
    ``workspace`` is an optional caller-owned uint8 buffer of at least
    ``prefill_workspace_bytes``; ``timing_events`` a pair of raw ``hipEvent_t``
    handles recorded around the scan kernel. Raises ``UnsupportedLayout`` where
    ``prefill_supported`` is false."""
    check_contract(q, kv, check_ranges=check_ranges)
    if not prefill_supported(q, kv):
        raise UnsupportedLayout("the fused prefill needs head_dim 128, 4 or 6-bit K and V, page size a power "
                                "of two >= 16, a HIP device and 4-aligned norm rows")
    B, Hq, Q, D = q.shape
    Hkv = kv.num_kv_heads
    ns = int(num_splits) if num_splits else prefill_plan_for(q, kv)
    out_dtype = out_dtype or q.dtype
    if out_dtype not in _lib.DTYPE_CODE:
        raise UnsupportedLayout(f"output dtype {out_dtype} is not supported")
    out = torch.empty(B, Hq, Q, D, dtype=out_dtype, device=q.device)
    need = prefill_workspace_bytes(B, Hq, Hkv, Q, D, ns)
    if need < 0:
        raise UnsupportedLayout(f"bad prefill sizes B={B} Hq={Hq} Hkv={Hkv} Q={Q} splits={ns}")
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != q.device:
        raise UnsupportedLayout(f"workspace needs {need} bytes on {q.device}")
    ev0, ev1 = timing_events or (None, None)
    with torch.cuda.device(q.device):
        _lib.call("wn_prefill_attention", _lib.ptr(q), _lib.DTYPE_CODE[q.dtype], q.stride(0), q.stride(1),
                  q.stride(2), *_operands(q, kv)[4:], _lib.ptr(out), _lib.DTYPE_CODE[out_dtype],
                  _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
                  B, Hq, Hkv, Q, D, kv.page_size, kv.k_quant.bit_width, kv.v_quant.bit_width,
                  float(scale), ns, _lib.stream_of(q.device), ev0, ev1)
    return out


DENSE_PAGE_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def dense_supported(q: torch.Tensor, kv: DenseKV) -> bool:
    """Whether ``dense_decode_attention`` compiles this shape (head_dim 16 .. 256, page
    size >= 16 and a power of two, bf16/fp16/fp32 pages with contiguous rows, one query
    token)."""
    D = q.shape[-1]
    return (q.dim() == 4 and q.shape[2] == 1 and D in SUPPORTED_HEAD_DIMS and kv.head_dim == D
            and kv.k_pages.dtype in DENSE_PAGE_DTYPES and kv.v_pages.dtype == kv.k_pages.dtype
            and kv.page_size >= 16 and _pow2(kv.page_size) and kv.k_pages.stride(-1) == 1
            and kv.k_pages.stride(-2) == D and kv.v_pages.stride() == kv.k_pages.stride()
            and q.shape[1] % kv.num_kv_heads == 0)


def dense_plan_for(q: torch.Tensor, kv: DenseKV, num_splits: int | None = None):
    """(pages_per_split, num_splits) of the dense decode for this query and handle
    (wn_dense_decode_plan): a balanced plan of persistent waves unless ``num_splits``."""
    B, Hq, _, D = q.shape
    pps, ns = ctypes.c_int(0), ctypes.c_int(0)
    with torch.cuda.device(q.device):
        _lib.call("wn_dense_decode_plan", B, Hq, kv.num_kv_heads, D, kv.page_size,
                  _lib.DTYPE_CODE[kv.k_pages.dtype], kv.page_table.shape[1], int(num_splits or 0),
                  ctypes.byref(pps), ctypes.byref(ns))
    return pps.value, ns.value


def dense_decode_attention(q: torch.Tensor, kv: DenseKV, scale: float, *,
                           num_splits: int | None = None, allow_tf32: bool = False,
                           num_warps: int = 4, num_stages: int = 2, pages_per_iter: int = 1,
                           out_dtype: torch.dtype | None = None,
                           workspace: torch.Tensor | None = None,
                           check_ranges: bool = True,
                           timing_events=None, plan: tuple[int, int] | None = None) -> torch.Tensor:
    """Unquantized paged decode on the packed decode's schedule, the matched baseline
    (packed_attention_triton.py:190-201): q (B, Hq, 1, D) -> (B, Hq, 1, D) in q.dtype.

    Pages (P, Hkv, S, D) bf16 or fp16 (matrix-core scan at head_dim 64 and 128) or
    fp32 and the other head dims (vector-ALU scan on fixed splits). Errors before any
    launch, as the reference's (``UnsupportedLayout``): a query of more than one token
    or off the GPU, a page size or head dim that is not a power of two, non-unit element
    stride, K and V strides that differ; and what this build does not compile (head_dim
    above 256, page size below 16). A length
    beyond the table or a live page id outside the pool is rejected too (a host copy
    of the metadata; ``check_ranges=False`` skips it for callers that own the
    metadata). The schedule keywords and ``plan`` behave as in ``packed_decode_attention``.
    """
    del allow_tf32, num_warps, num_stages
    if pages_per_iter < 1 or pages_per_iter & (pages_per_iter - 1):
        raise UnsupportedLayout("pages_per_iter must be a power of two >= 1")
    if q.dim() != 4 or q.shape[2] != 1 or not _lib.is_hip(q):
        raise UnsupportedLayout("dense kernel: HIP decode only (one query token, tensors on the GPU)")
    if not _pow2(kv.page_size) or not _pow2(kv.head_dim) or kv.k_pages.stride(-1) != 1 \
            or kv.v_pages.stride() != kv.k_pages.stride():
        raise UnsupportedLayout("dense kernel: unsupported page layout")
    B, Hq, _, D = q.shape
    Hkv = kv.num_kv_heads
    if D not in SUPPORTED_HEAD_DIMS or kv.head_dim != D or kv.k_pages.shape[-1] != D:
        raise UnsupportedLayout(f"dense kernel: head_dim {D} (compiled: {SUPPORTED_HEAD_DIMS})")
    if Hq % Hkv:
        raise UnsupportedLayout(f"dense kernel: {Hq} query heads over {Hkv} kv heads")
    if kv.page_size < 16:
        raise UnsupportedLayout(f"dense kernel: page size {kv.page_size} (>= 16 compiled)")
    if kv.k_pages.dtype not in DENSE_PAGE_DTYPES or kv.v_pages.dtype != kv.k_pages.dtype:
        raise UnsupportedLayout(f"dense kernel: pages {kv.k_pages.dtype}/{kv.v_pages.dtype} (bf16, fp16 or fp32)")
    if kv.k_pages.stride(-2) != D:
        raise UnsupportedLayout("dense kernel: the rows of a (page, head) block must be contiguous")
    if kv.page_table.dtype != torch.int32 or kv.seq_lens.dtype != torch.int32 \
            or kv.page_table.stride(-1) != 1 or not kv.seq_lens.is_contiguous():
        raise UnsupportedLayout("dense kernel: page_table and seq_lens must be contiguous int32")
    for t in (kv.k_pages, kv.v_pages, kv.page_table, kv.seq_lens):
        if t.device != q.device:
            raise UnsupportedLayout(f"dense kernel: operand on {t.device}, query on {q.device}")
    if kv.page_table.dim() != 2 or kv.page_table.shape[0] != B or kv.seq_lens.shape != (B,):
        raise UnsupportedLayout("dense kernel: page_table must be (B, max_pages) and seq_lens (B,)")
    if kv.v_pages.shape != kv.k_pages.shape:
        raise UnsupportedLayout("dense kernel: K and V pages differ in shape")
    if check_ranges:
        check_page_ranges(kv.seq_lens if kv.seq_lens_host is None else kv.seq_lens_host,
                          kv.page_table if kv.page_table_host is None else kv.page_table_host,
                          kv.k_pages.shape[0], kv.page_size)
    max_pages = kv.page_table.shape[1]
    pps, ns = plan if plan is not None else dense_plan_for(q, kv, num_splits)
    out_dtype = out_dtype or q.dtype
    if out_dtype not in _lib.DTYPE_CODE:
        raise UnsupportedLayout(f"output dtype {out_dtype} is not supported")
    out = torch.empty(B, Hq, 1, D, dtype=out_dtype, device=q.device)
    need = workspace_bytes(B, Hq, Hkv, D, pps, ns)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    elif workspace.numel() * workspace.element_size() < need or workspace.device != q.device:
        raise UnsupportedLayout(f"workspace needs {need} bytes on {q.device}")
    ev0, ev1 = timing_events or (None, None)
    qv = q[:, :, 0]
    es = kv.k_pages.element_size()
    with torch.cuda.device(q.device):
        _lib.call(
            "wn_dense_decode_attention",
            _lib.ptr(qv), _lib.DTYPE_CODE[q.dtype], qv.stride(0), qv.stride(1),
            _lib.ptr(kv.k_pages), kv.k_pages.stride(0) * es, kv.k_pages.stride(1) * es,
            _lib.ptr(kv.v_pages), kv.v_pages.stride(0) * es, kv.v_pages.stride(1) * es,
            _lib.DTYPE_CODE[kv.k_pages.dtype],
            _lib.ptr(kv.page_table), kv.page_table.stride(0), _lib.ptr(kv.seq_lens),
            _lib.ptr(out), _lib.DTYPE_CODE[out_dtype],
            _lib.ptr(workspace), workspace.numel() * workspace.element_size(),
            B, Hq, Hkv, D, kv.page_size, max_pages, float(scale), pps, ns,
            _lib.stream_of(q.device), ev0, ev1)
    return out
