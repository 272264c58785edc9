"""winnow_amd -- MI355X-native TurboQuant compressed-domain KV decode path.

Three drop-in pieces behind the reference's Python API (lgoyal6/winnow
``turboquant_kv``), each running hand-written gfx950 HIP kernels through the
C ABI in ``include/winnow_hip.h`` (``libwinnow_hip.so``):

* append:    ``packing`` (pack/unpack), ``quantizer.TurboQuantMSE`` (quantize),
             ``packed_backend.PagedPackedCache.update`` (fused quantize+pack+scatter)
* layout:    ``page_pool.PagePool`` (paged packed pool, fenced reclamation)
* attention: ``packed_attention.packed_decode_attention``

Around them: ``cache.TQPackedCache`` (the contiguous packed cache, imported on its
own: it pulls in transformers), ``packed_backend`` (the HF attention backend),
``engine`` (continuous batching) and ``kernel.tq_dequant`` (fused dequantization).
"""
from winnow_amd.packed_attention import (  # noqa: F401
    DenseKV, PackedKV, Quantizer, UnsupportedLayout, check_contract, default_scale,
    packed_decode_attention,
)
from winnow_amd.packing import SUPPORTED, pack, packed_bytes, unpack  # noqa: F401
from winnow_amd.page_pool import PagePool, PageRef, PoolExhausted, StalePage  # noqa: F401
from winnow_amd.quantizer import TurboQuantMSE, get_quantizer  # noqa: F401

__all__ = [
    "DenseKV", "PackedKV", "Quantizer", "UnsupportedLayout", "check_contract", "default_scale",
    "packed_decode_attention", "SUPPORTED", "pack", "packed_bytes", "unpack", "PagePool", "PageRef",
    "PoolExhausted", "StalePage", "TurboQuantMSE", "get_quantizer",
]
