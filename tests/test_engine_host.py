"""Engine admission on the host (no forward runs): the refusals of
turboquant_kv/engine.py:93-113 and cancellation of a request that never ran."""
from __future__ import annotations

import pytest
import torch

from winnow_amd.engine import Engine, EngineConfig, Refused, Request
from winnow_amd.page_pool import PagePool


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.w = torch.nn.Parameter(torch.zeros(1))


def _engine(**cfg):
    pool = PagePool(num_layers=1, num_pages=8, num_kv_heads=1, page_size=16, nb_k=64, nb_v=64, device="cpu",
                    max_pages_per_request=3)
    return Engine(_Model(), pool, None, None, 128, config=EngineConfig(**cfg))


def test_refusals_carry_their_reason():
    eng = _engine(max_queue=1, max_prompt_tokens=40, max_new_tokens_cap=16)
    for req, why in ((Request("a", [], 4), "empty_prompt"), (Request("b", [1] * 41, 4), "prompt_too_long"),
                     (Request("c", [1], 0), "bad_max_new_tokens"), (Request("d", [1] * 40, 16), "exceeds_request_cap")):
        with pytest.raises(Refused) as ei:
            eng.submit(req)
        assert ei.value.reason == why
    eng.submit(Request("e", [1, 2], 4))
    for req, why in ((Request("e", [1], 4), "duplicate_request_id"), (Request("f", [1], 4), "queue_full")):
        with pytest.raises(Refused) as ei:
            eng.submit(req)
        assert ei.value.reason == why


def test_cancel_of_a_queued_request_releases_without_a_forward():
    eng = _engine()
    r = eng.submit(Request("q", [1, 2, 3], 4))
    assert eng.cancel("q") and not eng.cancel("nope")
    assert not eng.step()                          # ends it without running the model
    assert r.status == "cancelled" and r.done.is_set() and eng.idle()
    assert not eng.cancel("q")
