"""The contiguous packed KV cache: a drop-in for ``TQPackedLayer`` / ``TQPackedCache``
(``turboquant_kv/cache.py:154-419``), the reference's first packed cache and the
quantized reference its model tests compare the paged path with
(``test_packed_model.py:44-61``).

Each layer keeps, per K and V, packed codes ``(B, H, max_cache_len, NB)`` uint8 and
fp16 norms ``(B, H, max_cache_len)``, optionally split into regular channels and a
few high-RMS outlier channels quantized at a higher width (``num_outlier_channels``,
``outlier_bits``; the channels are the top RMS channels of the first keys stored).
``update`` appends the new tokens and hands attention the whole history
dequantized, as ``DynamicLayer.update`` does with plain tensors.

On MI355X:

* the append is one ``wn_append_kv`` launch for K and V together (quantize, pack
  and write into the contiguous rows: the buffer is addressed as B pages of one
  power-of-two page each, page b = sequence b) when there are no outlier channels
  and the rows allow it; otherwise ``wn_quantize`` + ``wn_pack`` per channel group
  (any group width up to 256);
* the history comes back through ``wn_tq_dequant`` (the fused kernel, read in place
  from the ``max_cache_len`` buffer) at head_dim 128 without outlier channels, else
  through ``wn_unpack`` + ``wn_dequantize`` in chunks of ``chunk`` positions.

``kernel_backend`` keeps the reference's names: ``"triton_fp32"`` and
``"native_cuda_fp32"`` select the fused kernel at fp32 accuracy, ``"triton_tf32"``
the fused kernel's fast mode (one fp16 product per term), ``"torch_fp32"`` the
chunked standalone kernels, and ``"auto"`` the fused kernel where it applies (fast
when ``allow_tf32``) and the chunked path elsewhere. The reference's dispatcher
(``dispatch.py``) is not used: ``native_kernel`` and ``dispatcher`` are accepted
and ignored, and ``last_dispatch_decision`` records the path taken.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
from transformers.cache_utils import DynamicCache, DynamicLayer

from winnow_amd import _lib
from winnow_amd.kernel import tq_dequant
from winnow_amd.packing import pack, packed_bytes, unpack
from winnow_amd.quantizer import get_quantizer

KERNEL_BACKENDS = ("auto", "torch_fp32", "triton_fp32", "triton_tf32", "native_cuda_fp32")
_FUSED_HEAD_DIM = 128   # wn_tq_dequant's head_dim
_APPEND_HEAD_DIMS = (16, 32, 64, 128, 256)


@dataclass
class DequantChoice:
    """The history path one ``update`` took (the reference keeps its dispatcher's decision)."""
    backend: str          # "fused" or "chunked"
    fast: bool            # the fused kernel's fast mode
    reason: str


@dataclass
class _Group:
    """Packed codes and fp16 norms of one channel group of one side (K or V)."""
    codes: torch.Tensor   # (B, H, max, NB) uint8
    norms: torch.Tensor   # (B, H, max) fp16

    def nbytes(self) -> int:
        return self.codes.numel() + 2 * self.norms.numel()


class TQPackedLayer(DynamicLayer):
    """Per-layer packed KV storage; shapes (batch, kv_heads, seq, head_dim)."""

    def __init__(self, head_dim: int, bit_width: int, device, max_cache_len: int,
                 num_outlier_channels: int = 0, outlier_bits: int = 0, chunk: int = 1024,
                 use_kernel: bool = True, allow_tf32: bool = True, kernel_backend: str = "auto",
                 native_kernel=None, dispatcher=None):
        super().__init__()
        del native_kernel, dispatcher  # planner objects of the reference, not used here
        backend = kernel_backend if use_kernel else "torch_fp32"
        if backend not in KERNEL_BACKENDS:
            raise ValueError(f"unknown kernel_backend={kernel_backend!r}")
        self.use_kernel, self.allow_tf32, self.kernel_backend = use_kernel, allow_tf32, backend
        self.last_dispatch_decision: DequantChoice | None = None
        self._head_dim, self._bits, self._capacity, self._span = head_dim, bit_width, max_cache_len, chunk
        split = num_outlier_channels > 0 and outlier_bits > bit_width
        self._n_outlier = num_outlier_channels if split else 0
        self._n_regular = head_dim - self._n_outlier
        self._outlier_bits = outlier_bits
        # K and V share each group's quantizer (seed 42 regular, 43 outlier), as the reference's
        self._quant = get_quantizer(bit_width, self._n_regular, device)
        self._quant_outlier = get_quantizer(outlier_bits, self._n_outlier, device, seed=43) if split else None
        self._row_bytes = packed_bytes(self._n_regular, bit_width)
        self._outlier_row_bytes = packed_bytes(self._n_outlier, outlier_bits) if split else 0
        self._tokens = 0
        self._outlier_channels = None          # (head_dim,) bool: the outlier channels
        self._k_groups = self._v_groups = None   # lists of _Group: regular, then outlier
        self._append_table = self._append_start = None   # fused append's (B, 1) table, start positions
        self.is_initialized = False

    # ---------------------------------------------------------------- storage
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        B, H, _, D = key_states.shape
        if D != self._head_dim:
            raise ValueError(f"TQPackedLayer: head_dim {D} != {self._head_dim}")
        self.dtype, self.device = key_states.dtype, key_states.device
        dev = key_states.device

        def group(nb):
            return _Group(torch.empty(B, H, self._capacity, nb, dtype=torch.uint8, device=dev),
                          torch.empty(B, H, self._capacity, dtype=torch.float16, device=dev))
        widths = [self._row_bytes] + ([self._outlier_row_bytes] if self._n_outlier else [])
        self._k_groups = [group(nb) for nb in widths]
        self._v_groups = [group(nb) for nb in widths]
        if self._n_outlier:
            rms = key_states.float().pow(2).mean(dim=(0, 1, 2)).sqrt()
            self._outlier_channels = torch.zeros(D, dtype=torch.bool, device=dev)
            self._outlier_channels[rms.topk(min(self._n_outlier, D)).indices] = True
        self._dims = (B, H, D)
        self.is_initialized = True

    def _fused_append_ok(self, x: torch.Tensor) -> bool:
        """One wn_append_kv launch writes both sides: no outlier split, a compiled
        head_dim, rows whose byte strides keep the kernel's 8-byte alignment."""
        g = self._k_groups[0]
        return (not self._n_outlier and self._head_dim in _APPEND_HEAD_DIMS and x.dtype in _lib.DTYPE_CODE
                and (self._capacity * self._row_bytes) % 8 == 0 and g.codes.data_ptr() % 8 == 0
                and self._v_groups[0].codes.data_ptr() % 8 == 0)

    @torch.no_grad()
    def _append_fused(self, k: torch.Tensor, v: torch.Tensor, pos: int) -> None:
        B, H, n, D = k.shape
        k = k if k.stride(-1) == 1 else k.contiguous()
        v = v if (v.stride(-1) == 1 and v.dtype == k.dtype) else v.to(k.dtype).contiguous()
        S = 1 << max(self._capacity - 1, 1).bit_length()   # one power-of-two page holds a whole row
        dev = k.device
        if self._append_table is None or self._append_table.shape[0] != B:
            # row b of the cache is "page" b: a (B, 1) identity table, and the start
            # position of every row, kept on the layer (the steady-state append then
            # costs the fill of B integers and the append launch)
            self._append_table = torch.arange(B, dtype=torch.int32, device=dev).view(B, 1)
            self._append_start = torch.empty(B, dtype=torch.int32, device=dev)
        table, start = self._append_table, self._append_start
        start.fill_(pos)
        kg, vg, q = self._k_groups[0], self._v_groups[0], self._quant
        with torch.cuda.device(dev):
            _lib.call("wn_append_kv",
                      _lib.ptr(k), *k.stride()[:3], _lib.ptr(v), *v.stride()[:3], _lib.DTYPE_CODE[k.dtype],
                      _lib.ptr(q.Pi), _lib.ptr(q.boundaries), self._bits, _lib.ptr(q.Pi), _lib.ptr(q.boundaries), self._bits,
                      _lib.ptr(table), 1, _lib.ptr(start),
                      _lib.ptr(kg.codes), kg.codes.stride(0), kg.codes.stride(1),
                      _lib.ptr(vg.codes), vg.codes.stride(0), vg.codes.stride(1),
                      _lib.ptr(kg.norms), kg.norms.stride(0), kg.norms.stride(1),
                      _lib.ptr(vg.norms), vg.norms.stride(0), vg.norms.stride(1),
                      B, H, n, D, S, B, 1, _lib.stream_of(dev), None, None)

    @torch.no_grad()
    def _append_groups(self, x: torch.Tensor, groups, pos: int) -> None:
        """wn_quantize + wn_pack per channel group, written into [pos, pos + n)."""
        n = x.shape[-2]
        if self._n_outlier:
            xf = x.float()
            parts = [(xf[..., ~self._outlier_channels], self._quant, self._bits), (xf[..., self._outlier_channels], self._quant_outlier, self._outlier_bits)]
        else:
            parts = [(x, self._quant, self._bits)]
        for (xp, q, bw), g in zip(parts, groups):
            idx, nrm = q.quantize(xp)
            g.codes[:, :, pos:pos + n] = pack(idx, bw)
            g.norms[:, :, pos:pos + n] = nrm.to(torch.float16)

    # ---------------------------------------------------------------- history
    def _choose(self) -> DequantChoice:
        b = self.kernel_backend
        if b == "torch_fp32":
            return DequantChoice("chunked", False, "kernel_backend torch_fp32")
        if self._n_outlier:
            # the reference uses its kernels only without outlier channels and otherwise
            # takes the chunked path whatever kernel_backend asked for (cache.py:245-246)
            return DequantChoice("chunked", False, f"{b}: outlier channels take the chunked path")
        fused_ok = self._head_dim == _FUSED_HEAD_DIM
        if b == "auto":
            if fused_ok:
                return DequantChoice("fused", self.allow_tf32, "auto: fused kernel (head_dim 128, no outliers)")
            return DequantChoice("chunked", False, "auto: the fused kernel needs head_dim 128")
        if not fused_ok:
            raise RuntimeError(f"requested {b}, but the fused dequant serves head_dim 128")
        return DequantChoice("fused", b == "triton_tf32", f"kernel_backend {b}")

    @torch.no_grad()
    def _history(self, groups, length: int) -> torch.Tensor:
        B, H, D = self._dims
        out = torch.empty(B, H, length, D, dtype=self.dtype, device=self.device)
        choice = self._choose()
        self.last_dispatch_decision = choice
        if length == 0:
            return out
        if choice.backend == "fused":
            g = groups[0]
            tq_dequant(g.codes[:, :, :length], g.norms[:, :, :length], self._quant.centroids, self._quant.Pi,
                       self._bits, D, out=out, allow_tf32=choice.fast)
            return out
        quants = [(self._quant, self._bits, self._n_regular)] + \
            ([(self._quant_outlier, self._outlier_bits, self._n_outlier)] if self._n_outlier else [])
        for s in range(0, length, self._span):
            e = min(s + self._span, length)
            pieces = []
            for g, (q, bw, dim) in zip(groups, quants):
                part = torch.empty(B, H, e - s, dim, dtype=self.dtype, device=self.device)
                q.dequantize_into(unpack(g.codes[:, :, s:e].contiguous(), bw, dim), g.norms[:, :, s:e], part)
                pieces.append(part)
            if self._n_outlier:
                sl = out[:, :, s:e]
                sl[..., ~self._outlier_channels] = pieces[0]
                sl[..., self._outlier_channels] = pieces[1]
            else:
                out[:, :, s:e] = pieces[0]
        return out

    # ---------------------------------------------------------------- cache protocol
    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        n = key_states.shape[-2]
        if self._tokens + n > self._capacity:
            raise RuntimeError(f"TQPackedLayer overflow: {self._tokens}+{n} > max_cache_len={self._capacity}. "
                               f"Raise max_cache_len.")
        if self._fused_append_ok(key_states):
            self._append_fused(key_states, value_states, self._tokens)
        else:
            self._append_groups(key_states, self._k_groups, self._tokens)
            self._append_groups(value_states, self._v_groups, self._tokens)
        self._tokens += n
        return self._history(self._k_groups, self._tokens), self._history(self._v_groups, self._tokens)

    def get_seq_length(self, *a, **k) -> int:
        return self._tokens

    def get_mask_sizes(self, query_length: int, *a, **k):
        # asked before the layer stores the query's tokens (transformers' mask preparation)
        return self._tokens + query_length, 0

    def get_max_length(self, *a, **k) -> int:
        return self._capacity

    def get_max_cache_shape(self, *a, **k) -> int:
        return self.get_max_length()

    def reset(self) -> None:
        self._tokens = 0

    # ---------------------------------------------------------------- accounting
    def persistent_bytes(self) -> int:
        """Bytes this layer holds between steps (what limits concurrency)."""
        if not self.is_initialized:
            return 0
        return sum(g.nbytes() for g in self._k_groups + self._v_groups)

    def persistent_bytes_used(self) -> int:
        """The same, counting only the positions written so far."""
        if not self.is_initialized or self._capacity == 0:
            return 0
        return int(self.persistent_bytes() * self._tokens / self._capacity)

    def transient_bytes(self) -> int:
        """Bytes of the dequantized K and V handed to attention each step."""
        if not self.is_initialized:
            return 0
        B, H, D = self._dims
        return 2 * B * H * self._tokens * D * torch.empty((), dtype=self.dtype).element_size()


class TQPackedCache(DynamicCache):
    """``past_key_values`` of ``TQPackedLayer``s, one per decoder layer (cache.py:356-419)."""

    def __init__(self, config, bit_width: int, max_cache_len: int, device="cuda",
                 num_outlier_channels: int = 0, outlier_bits: int = 0, chunk: int = 1024,
                 use_kernel: bool = True, allow_tf32: bool = True, kernel_backend: str = "auto",
                 native_kernel=None, dispatcher=None):
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // config.num_attention_heads
        super().__init__()
        self.layers = [TQPackedLayer(head_dim, bit_width, device, max_cache_len, num_outlier_channels,
                                     outlier_bits, chunk, use_kernel, allow_tf32, kernel_backend,
                                     native_kernel, dispatcher)
                       for _ in range(config.num_hidden_layers)]
        self.layer_class_to_replicate = None   # the layers are fixed, not grown on demand
        self.bit_width, self.head_dim = bit_width, head_dim

    def persistent_bytes(self) -> int:
        return sum(l.persistent_bytes() for l in self.layers)

    def persistent_bytes_used(self) -> int:
        return sum(l.persistent_bytes_used() for l in self.layers)

    def transient_bytes(self) -> int:
        return max((l.transient_bytes() for l in self.layers), default=0)

    def effective_bits(self) -> float:
        """Stored bits per KV element, norms included."""
        l = self.layers[0]
        if not l.is_initialized:
            return float("nan")
        bits = 8 * (l._row_bytes + l._outlier_row_bytes) + 16 * (2 if l._n_outlier else 1)
        return bits / self.head_dim

    def get_seq_length(self, layer_idx: int = 0, *a, **k) -> int:
        return self.layers[layer_idx].get_seq_length()
