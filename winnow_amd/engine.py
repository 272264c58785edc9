"""Continuous-batching greedy decode over the paged packed cache, on one GPU.

The API is that of ``turboquant_kv/engine.py:34-278``: ``Refused`` (with a
machine-readable ``reason``), ``Request``, ``EngineConfig``, and ``Engine`` with
``submit``, ``cancel``, ``idle``, ``shutdown``, ``step``, ``run_until_idle`` and the
``on_logits`` diagnostic hook. Its behaviour is the reference's:

* a request is admitted, first come first served, only once the pool can reserve its
  worst case (prompt plus ``max_new_tokens``), so a running request never meets an
  allocation failure; one that can never fit is refused at ``submit``;
* each step ends cancelled and expired requests, admits, runs one prefill chunk of
  one request, then one batched decode forward of every request past its prefill;
* decoding is greedy, so a request's tokens depend on its prompt alone and a batched
  run equals the request run by itself.

Structure (this module's own):

* Running requests sit in ``max_batch`` fixed batch slots; a finished request frees
  its slot for the next admission. The decode batch is the slots in order.
* Admission checks are an ordered table of rules (``_RULES``); the first that fails
  gives the refusal reason.
* Prefill chunks and decode steps go through one forward helper: each row of the
  batch appends the same number of tokens at its own position, through a
  ``PagedPackedCache`` that uploads the page metadata once per forward; the
  attention is ``packed_backend.winnow_packed_attention`` (HIP decode operator,
  GPU dequantization + SDPA for prefill chunks).
* Pages of an ended request are released behind one fence recorded after the last
  forward that read them, so the pool recycles them only when the GPU is done.
"""
from __future__ import annotations

import itertools
import threading
import time
from collections import deque
from dataclasses import dataclass, field

import torch

from winnow_amd.packed_backend import PagedPackedCache
from winnow_amd.page_pool import PoolExhausted, default_fence


class Refused(RuntimeError):
    """A submission the engine will not queue; ``reason`` is machine-readable (engine.py:34-40)."""

    def __init__(self, reason: str, detail: str = ""):
        super().__init__(f"{reason}: {detail}" if detail else reason)
        self.reason = reason


@dataclass
class Request:
    """A generation request; the fields after ``ignore_eos`` are the engine's record of it
    (engine.py:43-62)."""

    request_id: str
    prompt_ids: list[int]
    max_new_tokens: int
    deadline: float | None = None            # in the engine clock's seconds
    on_event: object = None                  # callable(request, event: dict)
    ignore_eos: bool = False
    state: str = "queued"                    # queued -> prefill -> decode -> done
    status: str = ""                         # ok, eos, length, cancelled, deadline, error
    detail: str = ""
    generated: list[int] = field(default_factory=list)
    stored: int = 0                          # tokens of this request in the cache
    submitted_at: float = 0.0
    first_token_at: float | None = None
    token_times: list[float] = field(default_factory=list)
    finished_at: float | None = None
    cancel_requested: bool = False
    done: threading.Event = field(default_factory=threading.Event)


@dataclass
class EngineConfig:
    """Batching and admission limits (engine.py:65-71)."""

    max_batch: int = 8
    max_queue: int = 64
    prefill_chunk: int = 512
    max_prompt_tokens: int = 8192
    max_new_tokens_cap: int = 512
    decode_backend: str = "auto"
    allow_tf32: bool = False       # TF32-class products in the packed decode operator


# Admission rules in the order they are checked: (reason, refused?, detail).
_RULES = (
    ("shutting_down", lambda e, r: e.closed, lambda e, r: ""),
    ("empty_prompt", lambda e, r: not r.prompt_ids, lambda e, r: ""),
    ("prompt_too_long", lambda e, r: len(r.prompt_ids) > e.cfg.max_prompt_tokens,
     lambda e, r: f"{len(r.prompt_ids)} > {e.cfg.max_prompt_tokens}"),
    ("bad_max_new_tokens", lambda e, r: not 1 <= r.max_new_tokens <= e.cfg.max_new_tokens_cap,
     lambda e, r: f"must be 1..{e.cfg.max_new_tokens_cap}"),
    ("exceeds_request_cap", lambda e, r: e._worst_pages(r) > e.pool.max_pages_per_request,
     lambda e, r: f"{e._worst_pages(r)} pages > {e.pool.max_pages_per_request}"),
)


class Engine:
    """One scheduler (whoever calls ``step``) and any number of submitting or cancelling threads."""

    def __init__(self, model, pool, k_quant, v_quant, head_dim: int, eos_ids=(),
                 config: EngineConfig | None = None, clock=time.monotonic):
        self.model, self.pool = model, pool
        self.kq, self.vq, self.head_dim = k_quant, v_quant, head_dim
        self.eos = frozenset(int(t) for t in eos_ids)
        self.cfg = config or EngineConfig()
        self.clock = clock
        self.device = next(model.parameters()).device
        self.closed = False
        self.steps = 0
        self.on_logits = None                 # callable(requests, fp32 logits (B, vocab))
        self._slots: list[Request | None] = [None] * self.cfg.max_batch
        self._admitted_at: dict[str, int] = {}
        self._ticket = itertools.count()
        self._waiting: deque[Request] = deque()
        self._live: dict[str, Request] = {}   # every request not yet done, by id
        self._mu = threading.Lock()           # waiting queue, id map, cancel flags
        self._sched = threading.Lock()        # one step at a time

    def _worst_pages(self, req: Request) -> int:
        return self.pool.pages_for(len(req.prompt_ids) + req.max_new_tokens)

    # ---- client side ------------------------------------------------------
    def submit(self, req: Request) -> Request:
        """Queue ``req`` or raise ``Refused`` with the reason it can never be served."""
        for reason, refused, detail in _RULES:
            if refused(self, req):
                raise Refused(reason, detail(self, req))
        with self._mu:
            if req.request_id in self._live:
                raise Refused("duplicate_request_id")
            if len(self._waiting) >= self.cfg.max_queue:
                raise Refused("queue_full", f"{self.cfg.max_queue} queued")
            req.submitted_at = self.clock()
            self._live[req.request_id] = req
            self._waiting.append(req)
        return req

    def cancel(self, request_id: str) -> bool:
        """Ask for a request to end at the next step; False if it is unknown or done."""
        with self._mu:
            req = self._live.get(request_id)
            if req is None or req.state == "done":
                return False
            req.cancel_requested = True
            return True

    def idle(self) -> bool:
        with self._mu:
            return not self._waiting and all(s is None for s in self._slots)

    def shutdown(self) -> None:
        """Refuse new work and end everything outstanding as cancelled."""
        with self._mu:
            self.closed = True
            for req in self._live.values():
                req.cancel_requested = True
                req.detail = "server shutting down"
        self.step()

    def step(self) -> bool:
        """One scheduling iteration; False when there was nothing to run."""
        with self._sched:
            return self._step()

    def run_until_idle(self, max_steps: int = 100000) -> None:
        for _ in range(max_steps):
            if self.idle():
                return
            self.step()
        raise RuntimeError("engine did not drain")

    # ---- scheduler side ---------------------------------------------------
    def _running(self) -> list[Request]:
        return [r for r in self._slots if r is not None]

    def _notify(self, req: Request, **event) -> None:
        if req.on_event is not None:
            req.on_event(req, event)

    def _retire(self, req: Request, status: str, detail: str = "", fence=None) -> None:
        """End ``req``: free its slot, release its pages behind ``fence`` (default: an event
        recorded now), report the final event."""
        req.state, req.status = "done", status
        req.detail = req.detail or detail
        req.finished_at = self.clock()
        if req in self._slots:
            self._slots[self._slots.index(req)] = None
        self._admitted_at.pop(req.request_id, None)
        self.pool.release(req.request_id, fence)
        with self._mu:
            self._live.pop(req.request_id, None)
        self._notify(req, kind="final", status=status, detail=req.detail)
        req.done.set()

    def _expire(self) -> None:
        """End requests that were cancelled or are past their deadline."""
        now = self.clock()
        with self._mu:
            candidates = list(self._waiting) + self._running()
        for req in candidates:
            why = "cancelled" if req.cancel_requested else (
                "deadline" if req.deadline is not None and now > req.deadline else None)
            if why is None:
                continue
            with self._mu:
                if req in self._waiting:
                    self._waiting.remove(req)
            self._retire(req, why)

    def _fill_slots(self) -> None:
        """Admit from the head of the queue while a slot is free and the pool can reserve
        the head's worst case; nobody overtakes a head that does not fit."""
        while None in self._slots:
            with self._mu:
                if not self._waiting:
                    return
                head = self._waiting[0]
            try:
                self.pool.ensure(head.request_id, len(head.prompt_ids) + head.max_new_tokens)
            except PoolExhausted:
                return
            with self._mu:
                self._waiting.popleft()
            head.state = "prefill"
            self._admitted_at[head.request_id] = next(self._ticket)
            self._slots[self._slots.index(None)] = head

    def _forward(self, reqs: list[Request], tokens: list[list[int]]) -> torch.Tensor:
        """One forward appending ``tokens[b]`` (all the same length) to request b at its own
        position; the fp32 logits of each row's last token."""
        n = len(tokens[0])
        ids = torch.tensor(tokens, dtype=torch.long, device=self.device)
        start = torch.tensor([r.stored for r in reqs], dtype=torch.long, device=self.device)
        positions = start[:, None] + torch.arange(n, device=self.device)[None, :]
        cache = PagedPackedCache(self.pool, [r.request_id for r in reqs], [r.stored for r in reqs],
                                 k_quant=self.kq, v_quant=self.vq, head_dim=self.head_dim,
                                 decode_backend=self.cfg.decode_backend, allow_tf32=self.cfg.allow_tf32)
        out = self.model(input_ids=ids, position_ids=positions, past_key_values=cache, use_cache=True,
                         logits_to_keep=1)
        for r, stored in zip(reqs, cache.lengths):
            r.stored = stored
        logits = out.logits[:, -1].float()
        if self.on_logits is not None:
            self.on_logits(reqs, logits)
        return logits

    def _take_token(self, req: Request, token: int, now: float) -> str | None:
        """Record a generated token; the reason the request stops, if it does."""
        req.generated.append(token)
        req.token_times.append(now)
        if req.first_token_at is None:
            req.first_token_at = now
        self._notify(req, kind="token", index=len(req.generated) - 1, token_id=token, t=now)
        if token in self.eos and not req.ignore_eos:
            return "eos"
        return "length" if len(req.generated) >= req.max_new_tokens else None

    def _prefill_chunk(self, ended: dict) -> bool:
        """The next prompt chunk of the earliest-admitted request still in prefill."""
        pending = [r for r in self._running() if r.state == "prefill"]
        if not pending:
            return False
        req = min(pending, key=lambda r: self._admitted_at[r.request_id])
        lo = req.stored
        hi = min(lo + self.cfg.prefill_chunk, len(req.prompt_ids))
        try:
            logits = self._forward([req], [req.prompt_ids[lo:hi]])
        except Exception as exc:  # noqa: BLE001 - reported on the request
            self._retire(req, "error", f"{type(exc).__name__}: {exc}", default_fence(self.device))
            return True
        if hi == len(req.prompt_ids):
            req.state = "decode"
            why = self._take_token(req, int(logits[0].argmax()), self.clock())
            if why:
                ended[req.request_id] = (req, why)
        return True

    def _decode_batch(self, ended: dict) -> bool:
        """One token for every request past its prefill that has not just ended."""
        batch = [r for r in self._running() if r.state == "decode" and r.request_id not in ended]
        if not batch:
            return False
        try:
            tokens = self._forward(batch, [[r.generated[-1]] for r in batch]).argmax(-1).tolist()
        except Exception as exc:  # noqa: BLE001 - reported on every request of the batch
            fence = default_fence(self.device)
            for r in batch:
                self._retire(r, "error", f"{type(exc).__name__}: {exc}", fence)
            return True
        now = self.clock()
        for r, t in zip(batch, tokens):
            why = self._take_token(r, int(t), now)
            if why:
                ended[r.request_id] = (r, why)
        return True

    @torch.no_grad()
    def _step(self) -> bool:
        self.steps += 1
        self._expire()
        self._fill_slots()
        ended: dict[str, tuple[Request, str]] = {}
        ran = self._prefill_chunk(ended)
        ran = self._decode_batch(ended) or ran
        if ended:
            fence = default_fence(self.device)      # after every forward of this step
            for req, why in ended.values():
                self._retire(req, why, fence=fence)
        return ran
