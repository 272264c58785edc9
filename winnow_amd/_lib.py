"""ctypes binding of ``libwinnow_hip.so`` (the C ABI declared in include/winnow_hip.h).

The library is loaded lazily on first use and never rebuilt here: a missing
library raises ``HipLibraryMissing``, so no product path can silently fall back
to host code. Build it with ``python -m winnow_amd.build``.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libwinnow_hip.so"
ABI_VERSION = 9

WN_F32, WN_F16, WN_BF16 = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 32 << 20          # WN_NOALLOC_SCRATCH_BYTES
DTYPE_CODE = {torch.float32: WN_F32, torch.float16: WN_F16, torch.bfloat16: WN_BF16}

_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_f = ctypes.c_float
_c_p = ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/winnow_hip.h one to one.
SIGNATURES = {
    "wn_abi_version": (_c_i, []),
    "wn_last_error": (ctypes.c_char_p, []),
    "wn_decode_plan": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
                              ctypes.POINTER(_c_i), ctypes.POINTER(_c_i)]),
    "wn_decode_plan_tf32": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
                                   ctypes.POINTER(_c_i), ctypes.POINTER(_c_i)]),
    "wn_decode_workspace_bytes": (_c_i64, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i]),
    "wn_decode_attention": (_c_i, [
        _c_p, _c_i, _c_i64, _c_i64,                 # q, dtype, strides
        _c_p, _c_p, _c_p, _c_p,                     # pi_k, pi_v, codebooks
        _c_p, _c_i64, _c_i64,                       # k pages
        _c_p, _c_i64, _c_i64,                       # v pages
        _c_p, _c_i64, _c_i64,                       # k norms
        _c_p, _c_i64, _c_i64,                       # v norms
        _c_p, _c_i64, _c_p,                         # table, stride, seq_lens
        _c_p, _c_i, _c_p, _c_i64,                   # out, out dtype, workspace
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,   # B Hq Hkv D S bwk bwv max_pages
        _c_f, _c_i, _c_i,                           # scale, pages_per_split, num_splits
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
    "wn_decode_attention_tf32": (_c_i, [
        _c_p, _c_i, _c_i64, _c_i64,                 # q, dtype, strides
        _c_p, _c_p, _c_p, _c_p,                     # pi_k, pi_v, codebooks
        _c_p, _c_i64, _c_i64,                       # k pages
        _c_p, _c_i64, _c_i64,                       # v pages
        _c_p, _c_i64, _c_i64,                       # k norms
        _c_p, _c_i64, _c_i64,                       # v norms
        _c_p, _c_i64, _c_p,                         # table, stride, seq_lens
        _c_p, _c_i, _c_p, _c_i64,                   # out, out dtype, workspace
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,   # B Hq Hkv D S bwk bwv max_pages
        _c_f, _c_i, _c_i,                           # scale, pages_per_split, num_splits
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
    "wn_decode_attention_noalloc": (_c_i, [
        _c_p, _c_i, _c_i64, _c_i64,                 # q, dtype, strides
        _c_p, _c_p, _c_p, _c_p,                     # pi_k, pi_v, codebooks
        _c_p, _c_i64, _c_i64,                       # k pages
        _c_p, _c_i64, _c_i64,                       # v pages
        _c_p, _c_i64, _c_i64,                       # k norms
        _c_p, _c_i64, _c_i64,                       # v norms
        _c_p, _c_i64, _c_p,                         # table, stride, seq_lens
        _c_p, _c_i,                                 # out, out dtype
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,   # B Hq Hkv D S bwk bwv max_pages
        _c_f, _c_i, _c_i,                           # scale, pages_per_split, num_splits
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
    "wn_append_kv": (_c_i, [
        _c_p, _c_i64, _c_i64, _c_i64,
        _c_p, _c_i64, _c_i64, _c_i64, _c_i,
        _c_p, _c_p, _c_i,
        _c_p, _c_p, _c_i,
        _c_p, _c_i64, _c_p,
        _c_p, _c_i64, _c_i64,
        _c_p, _c_i64, _c_i64,
        _c_p, _c_i64, _c_i64,
        _c_p, _c_i64, _c_i64,
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
    "wn_quantize": (_c_i, [_c_p, _c_i, _c_i64, _c_i64, _c_p, _c_p, _c_i, _c_i, _c_p, _c_p, _c_p]),
    "wn_pack": (_c_i, [_c_p, _c_i64, _c_i, _c_i, _c_p, _c_p]),
    "wn_unpack": (_c_i, [_c_p, _c_i64, _c_i, _c_i, _c_p, _c_p]),
    "wn_dequantize": (_c_i, [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i, _c_i, _c_p, _c_i, _c_p]),
    "wn_tq_dequant": (_c_i, [_c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_i, _c_i, _c_p, _c_i, _c_i, _c_p]),
    "wn_dense_decode_plan": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
                                    ctypes.POINTER(_c_i), ctypes.POINTER(_c_i)]),
    "wn_dense_decode_attention": (_c_i, [
        _c_p, _c_i, _c_i64, _c_i64,                 # q, dtype, strides
        _c_p, _c_i64, _c_i64,                       # k pages, strides (bytes)
        _c_p, _c_i64, _c_i64, _c_i,                 # v pages, strides, page dtype
        _c_p, _c_i64, _c_p,                         # table, stride, seq_lens
        _c_p, _c_i, _c_p, _c_i64,                   # out, out dtype, workspace
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,         # B Hq Hkv D S max_pages
        _c_f, _c_i, _c_i,                           # scale, pages_per_split, num_splits
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
    "wn_dequantize_history": (_c_i, [
        _c_p, _c_i64, _c_i64,                       # pages, page stride, head stride
        _c_p, _c_i64, _c_i64,                       # norms, page stride, head stride
        _c_p, _c_i, _c_i, _c_i,                     # table row, L, Hkv, S
        _c_p, _c_p, _c_i, _c_i,                     # centroids, Pi, bw, D
        _c_p, _c_i, _c_i, _c_p]),                   # out, out dtype, fast, stream
    "wn_prefill_plan": (_c_i, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, ctypes.POINTER(_c_i)]),
    "wn_prefill_workspace_bytes": (_c_i64, [_c_i, _c_i, _c_i, _c_i, _c_i, _c_i]),
    "wn_prefill_attention": (_c_i, [
        _c_p, _c_i, _c_i64, _c_i64, _c_i64,         # q, dtype, strides (b, h, q)
        _c_p, _c_p, _c_p, _c_p,                     # pi_k, pi_v, codebooks
        _c_p, _c_i64, _c_i64,                       # k pages
        _c_p, _c_i64, _c_i64,                       # v pages
        _c_p, _c_i64, _c_i64,                       # k norms
        _c_p, _c_i64, _c_i64,                       # v norms
        _c_p, _c_i64, _c_p,                         # table, stride, seq_lens
        _c_p, _c_i, _c_p, _c_i64,                   # out, out dtype, workspace
        _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,   # B Hq Hkv Q D S bwk bwv
        _c_f, _c_i,                                 # scale, num_splits
        _c_p, _c_p, _c_p]),                         # stream, ev_begin, ev_end
}

# bench.py's measurement probes (include/winnow_probe.h): libwinnow_probe.so beside
# the product library, loaded only by probe_call
PROBE_SIGNATURES = {
    "wn_probe_last_error": (ctypes.c_char_p, []),
    "wn_probe_lds_lookup_rate": (_c_i, [_c_i, _c_i, ctypes.POINTER(ctypes.c_double)]),
}


class HipLibraryMissing(RuntimeError):
    """libwinnow_hip.so is not built (or not loadable); there is no fallback."""


class WinnowHipError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed ({code}): {message}")
        self.code = code


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipLibraryMissing(
                    f"{LIB_PATH} is missing: build it with `python -m winnow_amd.build`")
            try:
                handle = ctypes.CDLL(str(LIB_PATH))
            except OSError as e:
                raise HipLibraryMissing(f"cannot load {LIB_PATH}: {e}") from e
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            if handle.wn_abi_version() != ABI_VERSION:
                raise HipLibraryMissing(
                    f"{LIB_PATH} has ABI {handle.wn_abi_version()}, expected {ABI_VERSION}; rebuild it")
            _lib = handle
    return _lib


_probe = None


def probe_path() -> Path:
    return LIB_PATH.with_name("libwinnow_probe.so")


def probe_lib() -> ctypes.CDLL:
    global _probe
    with _lock:
        if _probe is None:
            path = probe_path()
            if not path.exists():
                raise HipLibraryMissing(f"{path} is missing: build it with `python -m winnow_amd.build`")
            handle = ctypes.CDLL(str(path))
            for name, (res, args) in PROBE_SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype, fn.argtypes = res, args
            _probe = handle
    return _probe


def probe_call(name: str, *args) -> None:
    """Invoke a measurement probe; raise ``WinnowHipError`` with its message on failure."""
    handle = probe_lib()
    rc = getattr(handle, name)(*args)
    if rc != 0:
        raise WinnowHipError(name, rc, handle.wn_probe_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    """Invoke an entry point; raise ``WinnowHipError`` with wn_last_error() on failure."""
    handle = lib()
    rc = getattr(handle, name)(*args)
    if rc != 0:
        raise WinnowHipError(name, rc, handle.wn_last_error().decode(errors="replace"))


def ptr(t: torch.Tensor | None):
    """A tensor's device address for a ``void*`` argument (a plain integer: ctypes
    converts it faster than a c_void_p object built in Python)."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def is_hip(t: torch.Tensor) -> bool:
    return t.device.type == "cuda" and torch.version.hip is not None
