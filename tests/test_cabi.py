"""The C-ABI library loads on the host and exports exactly what include/winnow_hip.h declares.

No compute call is made here (there is no GPU in the CPU suite); only host-side
entry points that touch no device (version, error string, split planning,
workspace sizing, argument validation) are exercised.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "winnow_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(wn_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from winnow_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} is not built: run `python -m winnow_amd.build`")
    return _lib.lib()


def test_header_declares_the_expected_entry_points():
    names = declared_symbols()
    for must in ("wn_abi_version", "wn_last_error", "wn_decode_plan", "wn_decode_workspace_bytes",
                 "wn_decode_attention", "wn_append_kv", "wn_quantize", "wn_pack", "wn_unpack",
                 "wn_dequantize", "wn_tq_dequant", "wn_dequantize_history", "wn_dense_decode_plan",
                 "wn_dense_decode_attention"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    from winnow_amd import _lib
    for name in declared_symbols():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_probe_library_is_separate(lib):
    """The measurement probe lives in libwinnow_probe.so (include/winnow_probe.h), not
    in the product library or its header."""
    from winnow_amd import _lib
    assert not hasattr(lib, "wn_probe_lds_lookup_rate")
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "winnow_probe.h").read_text(), flags=re.S)
    names = sorted(set(re.findall(r"\b(wn_[a-z_0-9]+)\s*\(", text)))
    assert names == sorted(_lib.PROBE_SIGNATURES)
    probe = _lib.probe_lib()
    for name in names:
        assert hasattr(probe, name), f"{name} declared in winnow_probe.h but not exported"
    assert probe.wn_probe_last_error() == b""


def test_abi_version_and_error_string(lib):
    assert lib.wn_abi_version() == 9
    assert isinstance(lib.wn_last_error(), bytes)


def test_plan_reference_semantics(lib):
    from winnow_amd.packed_attention import decode_plan
    # explicit splits: clamp to [1, max_pages], cdiv(max_pages, splits) pages each
    assert decode_plan(2, 8, 4, 128, 16, 4, 4, 10, 3) == (4, 3)
    assert decode_plan(2, 8, 4, 128, 16, 4, 4, 10, 50) == (1, 10)
    assert decode_plan(2, 8, 4, 128, 16, 4, 4, 0, 1) == (1, 1)
    # automatic plans for shapes the vector-ALU scan serves (no device query): fixed
    # splits covering the table
    # (odd n_rep above 8 and head_dim 64; even n_rep up to 16 runs on the row scan)
    for B, Hq, Hkv, D, mp in ((16, 72, 8, 128, 2048), (4, 88, 8, 128, 8192), (64, 8, 8, 64, 4096),
                              (1, 16, 1, 64, 64), (1, 1, 1, 64, 1)):
        pps, ns = decode_plan(B, Hq, Hkv, D, 16, 4, 4, mp)
        assert pps * ns >= mp and pps >= 1 and ns >= 1
        assert (ns - 1) * pps < max(mp, 1)
        # the allow_tf32 plan: the same scan serves these shapes, so the same plan
        assert decode_plan(B, Hq, Hkv, D, 16, 4, 4, mp, allow_tf32=True) == (pps, ns)
    # explicit splits mean the same under allow_tf32
    assert decode_plan(2, 8, 4, 128, 16, 4, 4, 10, 3, allow_tf32=True) == (4, 3)
    assert decode_plan(2, 8, 4, 128, 16, 4, 4, 10, 50, allow_tf32=True) == (1, 10)


def test_workspace_bytes(lib):
    from winnow_amd.packed_attention import workspace_bytes
    w1 = workspace_bytes(16, 32, 8, 128, 64, 32)
    w2 = workspace_bytes(16, 32, 8, 128, 32, 64)
    assert w2 > w1 > 16 * 32 * 32 * 128 * 4
    # balanced plan: num_splits + B*Hkv partial rows of every real query head
    wb = workspace_bytes(16, 32, 8, 128, 0, 3072)
    assert wb >= (3072 + 128) * 4 * 130 * 4
    assert lib.wn_decode_workspace_bytes(16, 30, 8, 128, 4, 4) == -1     # Hq % Hkv


def test_argument_errors_are_reported_not_fatal(lib):
    from winnow_amd import _lib
    with pytest.raises(_lib.WinnowHipError, match="bit width"):
        _lib.call("wn_pack", None, 1, 128, 7, None, None)
    assert b"bit width" in lib.wn_last_error()
    with pytest.raises(_lib.WinnowHipError, match="head_dim"):
        _lib.call("wn_quantize", None, 0, 1, 128, None, None, 4, 300, None, None, None)
    # empty work is a successful no-op and clears the error
    _lib.call("wn_pack", None, 0, 128, 4, None, None)
    assert lib.wn_last_error() == b""


def test_head_dims_compiled_and_refused(lib):
    """The decode entry points take the powers of two 16 .. 256 and refuse 8, 96 and
    512 with the compiled list; bf16 dense pages at a head_dim without the matrix-core
    scan need fixed splits. wn_quantize / wn_dequantize take any head_dim up to 256 (the
    legacy cache's regular and outlier channel splits), so 8 and 96 pass their head_dim
    check (the next check, a null operand, reports) and 512 is refused."""
    from winnow_amd import _lib
    for D in (8, 16, 96, 128, 256):
        with pytest.raises(_lib.WinnowHipError, match="null operand"):
            _lib.call("wn_quantize", None, 0, 1, D, None, None, 4, D, None, None, None)
    with pytest.raises(_lib.WinnowHipError, match="head_dim 512"):
        _lib.call("wn_quantize", None, 0, 1, 512, None, None, 4, 512, None, None, None)
    dense = ("wn_dense_decode_attention", None, 2, 0, 0, None, 0, 0, None, 0, 0)
    with pytest.raises(_lib.WinnowHipError, match="fixed splits"):
        _lib.call(*dense, 2, None, 0, None, None, 0, None, 0, 1, 4, 1, 256, 16, 1, 1.0, 0, 1, None, None, None)
    for D in (8, 96, 512):
        with pytest.raises(_lib.WinnowHipError, match="16, 32, 64, 128, 256"):
            _lib.call(*dense, 2, None, 0, None, None, 0, None, 0, 1, 4, 1, D, 16, 1, 1.0, 0, 1, None, None, None)


def test_dequant_and_dense_entry_points_reject_before_any_launch(lib):
    """Argument errors of the newer entry points come back as codes with a message,
    before anything touches a device (no GPU here)."""
    from winnow_amd import _lib
    with pytest.raises(_lib.WinnowHipError, match="head_dim"):          # 64 is not compiled
        _lib.call("wn_tq_dequant", None, None, 1, 4, 4, None, None, 4, 64, None, 0, 0, None)
    with pytest.raises(_lib.WinnowHipError, match="bad sizes"):         # plane_rows < L
        _lib.call("wn_tq_dequant", None, None, 1, 4, 3, None, None, 4, 128, None, 0, 0, None)
    with pytest.raises(_lib.WinnowHipError, match="output dtype"):
        _lib.call("wn_tq_dequant", None, None, 1, 4, 4, None, None, 4, 128, None, 9, 0, None)
    with pytest.raises(_lib.WinnowHipError, match="null pointer"):
        _lib.call("wn_tq_dequant", None, None, 1, 4, 4, None, None, 4, 128, None, 0, 0, None)
    with pytest.raises(_lib.WinnowHipError, match="S=12"):              # S must be a power of two
        _lib.call("wn_dequantize_history", None, 0, 0, None, 0, 0, None, 5, 2, 12, None, None, 4, 128,
                  None, 0, 0, None)
    dense = ("wn_dense_decode_attention", None, _lib.WN_BF16 if hasattr(_lib, "WN_BF16") else 2, 0, 0,
             None, 0, 0, None, 0, 0)
    with pytest.raises(_lib.WinnowHipError, match="head_dim"):          # head_dim 96 is not compiled
        _lib.call(*dense, 2, None, 0, None, None, 0, None, 0, 1, 4, 1, 96, 16, 1, 1.0, 0, 1, None, None, None)
    with pytest.raises(_lib.WinnowHipError, match="fixed splits"):      # fp32 pages on a balanced plan
        _lib.call(*dense, 0, None, 0, None, None, 0, None, 0, 1, 4, 1, 128, 16, 1, 1.0, 0, 1, None, None, None)
    with pytest.raises(_lib.WinnowHipError, match="page dtype"):        # no such dtype code
        _lib.call(*dense, 7, None, 0, None, None, 0, None, 0, 1, 4, 1, 128, 16, 1, 1.0, 0, 1, None, None, None)
    with pytest.raises(_lib.WinnowHipError, match="page size"):
        _lib.call(*dense, 2, None, 0, None, None, 0, None, 0, 1, 4, 1, 128, 8, 1, 1.0, 0, 1, None, None, None)
    # no sequences: a successful no-op
    _lib.call(*dense, 2, None, 0, None, None, 0, None, 0, 0, 4, 1, 128, 16, 1, 1.0, 0, 1, None, None, None)
    assert lib.wn_last_error() == b""


def test_decode_rejects_norm_strides_past_32_bits(lib):
    """Norm strides of 2^31 elements or more come back as an error before any launch
    (fake, aligned, never dereferenced device pointers; no GPU here)."""
    from winnow_amd import _lib
    P = 1 << 20
    B, Hq, Hkv, D, S, NB, max_pages = 1, 8, 8, 128, 16, 64, 4

    def call(kn_p, kn_h):
        _lib.call("wn_decode_attention", P, _lib.WN_F32, Hq * D, D, P, P, P, P,
                  P, Hkv * S * NB, S * NB, P, Hkv * S * NB, S * NB,
                  P, kn_p, kn_h, P, Hkv * S, S,
                  P, max_pages, P, P, _lib.WN_F32, P, 1 << 30,
                  B, Hq, Hkv, D, S, 4, 4, max_pages, 1.0, 0, 4, None, None, None)

    with pytest.raises(_lib.WinnowHipError, match="norm strides"):
        call(1 << 31, S)
    with pytest.raises(_lib.WinnowHipError, match="norm strides"):
        call(Hkv * S, 1 << 28)



def test_decode_rejects_page_strides_past_32_bits(lib):
    """Page strides of 2^32 bytes or more come back as an error before any launch: the
    row scans form a page block's address from page id x page stride in 32 x 32 bits
    (fake, aligned, never dereferenced device pointers; no GPU here)."""
    from winnow_amd import _lib
    P = 1 << 20
    B, Hq, Hkv, D, S, NB, max_pages = 1, 8, 8, 128, 16, 64, 4

    def call(k_p, v_p):
        _lib.call("wn_decode_attention", P, _lib.WN_F32, Hq * D, D, P, P, P, P,
                  P, k_p, S * NB, P, v_p, S * NB,
                  P, Hkv * S, S, P, Hkv * S, S,
                  P, max_pages, P, P, _lib.WN_F32, P, 1 << 30,
                  B, Hq, Hkv, D, S, 4, 4, max_pages, 1.0, 0, 4, None, None, None)

    with pytest.raises(_lib.WinnowHipError, match="page strides"):
        call(1 << 32, Hkv * S * NB)
    with pytest.raises(_lib.WinnowHipError, match="page strides"):
        call(Hkv * S * NB, 1 << 32)
