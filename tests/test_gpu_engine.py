"""The continuous-batching engine (``winnow_amd.engine``) on the GPU, the reference's
request-lifecycle tests (test_packed_model.py:83-275) on a tiny seeded Qwen2 with
head_dim 128 (``tiny_qwen``). Decoding is greedy, so:

* one request through the engine (prefill in chunks of 7, HIP decode) equals the
  same prompt through the reconstruct path, token for token (8-bit codes, logits
  within 1e-3 of their scale as in test_gpu_model);
* requests of mixed lengths run concurrently (more than the batch holds) each equal
  the request run alone;
* EOS, length, cancellation, deadlines, shutdown and admission refusals end or
  refuse requests with their reason, and every page returns to the pool.
"""
from __future__ import annotations

import pytest
import torch

DEV = "cuda"
BW = 8
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    from tiny_qwen import tiny_qwen
    return tiny_qwen(DEV)


def make_engine(model, pages=64, page_size=16, cap=None, eos=(), clock=None, **cfg):
    from winnow_amd import packed_backend as pb
    from winnow_amd.engine import Engine, EngineConfig
    model.config._attn_implementation = pb.ATTN_NAME
    pool = pb.make_pool(model.config, bit_width=BW, num_pages=pages, page_size=page_size, device=DEV,
                        max_pages_per_request=cap)
    kq, vq = pb.quantizers_for(model.config, BW, DEV)
    kw = {"clock": clock} if clock is not None else {}
    return Engine(model, pool, kq, vq, pb.head_dim_of(model.config), eos_ids=eos, config=EngineConfig(**cfg), **kw)


def run(engine, reqs):
    for r in reqs:
        engine.submit(r)
    engine.run_until_idle()
    return reqs


def alone(model, prompt, n, **cfg):
    from winnow_amd.engine import Request
    (r,) = run(make_engine(model, **cfg), [Request("solo", prompt, n)])
    return r.generated


def all_pages_back(engine):
    engine.pool.reclaim()
    torch.cuda.synchronize()
    engine.pool.reclaim()
    st = engine.pool.stats()
    return st["owned"] == 0 and st["free"] == st["total"]


def test_single_request_matches_the_reconstruct_path(model):
    from tiny_qwen import prompts
    from winnow_amd import packed_backend as pb
    from winnow_amd.engine import Request
    prompt = prompts(1, seed=3, lo=20, hi=21)[0]
    ref = make_engine(model, decode_backend="reconstruct_sdpa", prefill_chunk=512)
    ref_logits = []
    ref.on_logits = lambda reqs, lg: ref_logits.append(lg[0].clone())
    (rr,) = run(ref, [Request("r", prompt, 12)])
    eng = make_engine(model, prefill_chunk=7)
    got = []
    eng.on_logits = lambda reqs, lg: got.append(lg[0].clone())
    pb.BACKEND_COUNTS.clear()
    (r,) = run(eng, [Request("a", prompt, 12)])
    assert r.status == "length" and r.generated == rr.generated
    # the chunks before the last produce logits the one-chunk reference never sees
    scale = max(1.0, max(x.abs().max().item() for x in ref_logits))
    for a, b in zip(got[-len(ref_logits):], ref_logits):
        assert (a - b).abs().max().item() < 1e-3 * scale
    assert pb.BACKEND_COUNTS["hip_packed"] > 0
    assert pb.BACKEND_COUNTS["prefill_reconstruct_sdpa"] >= 3
    assert pb.BACKEND_COUNTS["native_sdpa"] == 0
    assert all_pages_back(eng)


def test_concurrent_mixed_lengths_equal_isolated(model):
    from tiny_qwen import prompts
    from winnow_amd.engine import Request
    ps = prompts(5, seed=7)
    eng = make_engine(model, max_batch=3, prefill_chunk=32)
    reqs = run(eng, [Request(f"q{i}", p, 9) for i, p in enumerate(ps)])
    for r, p in zip(reqs, ps):
        assert r.status == "length"
        assert r.generated == alone(model, p, 9, prefill_chunk=32), r.request_id
    assert all_pages_back(eng)


def test_eos_stops_and_frees(model):
    from tiny_qwen import prompts
    from winnow_amd.engine import Request
    p = prompts(1, seed=11)[0]
    full = alone(model, p, 10)
    eos = full[3]
    eng = make_engine(model, eos=(eos,))
    (r,) = run(eng, [Request("e", p, 10)])
    assert r.status == "eos" and r.generated == full[:full.index(eos) + 1]
    (r2,) = run(eng, [Request("e2", p, 10, ignore_eos=True)])
    assert r2.status == "length" and r2.generated == full
    assert all_pages_back(eng)


def test_admission_refusals(model):
    from winnow_amd.engine import Refused, Request
    eng = make_engine(model, pages=8, cap=3, max_queue=2, max_prompt_tokens=40, max_new_tokens_cap=16)
    cases = [(Request("a", [], 4), "empty_prompt"), (Request("b", [1] * 41, 4), "prompt_too_long"),
             (Request("c", [1] * 5, 0), "bad_max_new_tokens"), (Request("d", [1] * 5, 17), "bad_max_new_tokens"),
             (Request("e", [1] * 40, 16), "exceeds_request_cap")]
    for req, why in cases:
        with pytest.raises(Refused) as ei:
            eng.submit(req)
        assert ei.value.reason == why
    eng.submit(Request("f", [1, 2, 3], 4))
    with pytest.raises(Refused) as ei:
        eng.submit(Request("f", [1, 2, 3], 4))
    assert ei.value.reason == "duplicate_request_id"
    eng.submit(Request("g", [1, 2, 3], 4))
    with pytest.raises(Refused) as ei:
        eng.submit(Request("h", [1, 2, 3], 4))
    assert ei.value.reason == "queue_full"
    eng.run_until_idle()
    eng.shutdown()
    with pytest.raises(Refused) as ei:
        eng.submit(Request("i", [1, 2, 3], 4))
    assert ei.value.reason == "shutting_down"


def test_pool_exhaustion_queues_then_admits(model):
    from tiny_qwen import prompts
    from winnow_amd.engine import Request
    ps = prompts(2, seed=13, lo=40, hi=60)
    eng = make_engine(model, pages=5, cap=5, max_batch=4)    # one request's worst case at a time
    reqs = [Request("x", ps[0], 8), Request("y", ps[1], 8)]
    for r in reqs:
        eng.submit(r)
    eng.step()
    assert reqs[0].state != "queued" and reqs[1].state == "queued"
    eng.run_until_idle()
    for r, p in zip(reqs, ps):
        assert r.status == "length" and r.generated == alone(model, p, 8)
    assert all_pages_back(eng)


def test_cancel_deadline_and_shutdown(model):
    from tiny_qwen import prompts
    from winnow_amd.engine import Request
    ps = prompts(3, seed=17)
    now = [0.0]
    eng = make_engine(model, clock=lambda: now[0])
    events = []
    a = Request("a", ps[0], 30, on_event=lambda r, e: events.append((r.request_id, e["kind"])))
    b = Request("b", ps[1], 30, deadline=5.0)
    c = Request("c", ps[2], 30)
    for r in (a, b, c):
        eng.submit(r)
    for _ in range(6):
        eng.step()
    assert eng.cancel("a")
    now[0] = 6.0                                                # past b's deadline
    eng.step()
    assert a.status == "cancelled" and b.status == "deadline"
    assert ("a", "final") in events and ("a", "token") in events
    assert 0 < len(a.generated) < 30
    eng.shutdown()
    assert c.status == "cancelled" and c.detail == "server shutting down"
    assert not eng.cancel("c")
    assert all_pages_back(eng)
