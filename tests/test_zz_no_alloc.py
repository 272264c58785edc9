"""The allocation-free decode entry point, ``wn_decode_attention_noalloc`` (no counterpart
in the reference; for callers that cannot allocate device memory).

Two calls in a row through the C ABI, the second with a smaller batch, other widths
and another head grouping, each against ``wn_decode_attention`` with a workspace on
the same inputs and plan: the kernels and the plan are the same, so the outputs must
be bit-identical; both are also held to the CPU oracle at 2e-3 / 1e-3. No torch
allocation happens across a call, and a plan needing more than the static scratch is
refused before any launch, by the Python wrapper and by the C entry point itself.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from cases import build, to_device
from oracle import attention as oa

pytestmark = pytest.mark.gpu
DEV = "cuda"

# (seed, B, Hq, Hkv, lens, bits K, bits V): the second call is smaller
CALLS = [(901, 6, 32, 8, (3000, 0, 129, 2048, 64, 777), 4, 4),
         (902, 2, 64, 8, (500, 7), 4, 6)]


def _pa():
    from winnow_amd import packed_attention as pa
    return pa


@pytest.mark.parametrize("plan", [None, (0, 5)])
def test_noalloc_equals_the_workspace_entry_point_on_consecutive_calls(plan):
    pa = _pa()
    for seed, B, Hq, Hkv, lens, bwk, bwv in CALLS:
        print(f"no-alloc decode: B={B} Hq={Hq} Hkv={Hkv} bits {bwk}/{bwv} plan {plan}", flush=True)
        q, kv = build(seed, B, Hq, Hkv, 128, lens, 16, bwk, bw_v=bwv)
        dkv, qd = to_device(kv, DEV), q.to(DEV)
        scale = oa.default_scale(128)
        want = pa.packed_decode_attention(qd, dkv, scale, out_dtype=torch.float32, plan=plan)
        out = torch.full_like(want, float("nan"))
        torch.cuda.synchronize()
        before = torch.cuda.memory_stats().get("allocation.all.allocated", 0)
        got = pa.packed_decode_attention_noalloc(qd, dkv, scale, out, plan=plan)
        torch.cuda.synchronize()
        assert torch.cuda.memory_stats().get("allocation.all.allocated", 0) == before, "a torch allocation"
        assert got is out
        assert torch.equal(got, want), (got - want).abs().max()
        ref = oa.tiled_compressed_attention(q, kv, scale)
        assert torch.allclose(got.cpu(), ref, atol=2e-3, rtol=1e-3), (got.cpu() - ref).abs().max()
        for b, L in enumerate(lens):
            if L == 0:
                assert (got[b] == 0).all()


def test_noalloc_refuses_plans_beyond_its_scratch():
    from winnow_amd import _lib
    pa = _pa()
    seed, B, Hq, Hkv, lens, bwk, bwv = CALLS[1]
    q, kv = build(seed, B, Hq, Hkv, 128, lens, 16, bwk, bw_v=bwv)
    dkv, qd = to_device(kv, DEV), q.to(DEV)
    out = torch.zeros(B, Hq, 1, 128, device=DEV)
    big = (0, 100000)                         # 100000 waves: ~400 MB of partials
    assert pa.workspace_bytes(B, Hq, Hkv, 128, *big) > _lib.NOALLOC_SCRATCH_BYTES
    with pytest.raises(pa.UnsupportedLayout, match="static scratch"):
        pa.packed_decode_attention_noalloc(qd, dkv, 0.1, out, plan=big)
    # the C entry point checks the size itself, before any launch
    lib = _lib.lib()
    with torch.cuda.device(qd.device):
        rc = lib.wn_decode_attention_noalloc(*pa._operands(qd, dkv), _lib.ptr(out), _lib.WN_F32,
                                             *pa._sizes(qd, dkv), ctypes.c_float(0.1), *big,
                                             _lib.stream_of(qd.device), None, None)
    assert rc == -3 and b"static scratch" in lib.wn_last_error()
    torch.cuda.synchronize()
    assert (out == 0).all()
