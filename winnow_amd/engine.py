"""Continuous-batching greedy decode over the paged packed cache, on one GPU.

Drop-in for ``turboquant_kv/engine.py`` (``Refused``, ``Request``, ``EngineConfig``,
``Engine`` with ``submit`` / ``cancel`` / ``idle`` / ``shutdown`` / ``step`` /
``run_until_idle`` and the ``on_logits`` hook; engine.py:34-278). Requests are
admitted in arrival order once the pool can reserve their worst case (prompt plus
``max_new_tokens``), so a running request never meets an allocation failure. A
scheduling step

1. ends requests that were cancelled or passed their deadline, releasing their
   pages behind a fence recorded on the stream after the last forward that read them;
2. admits queued requests while the batch has room;
3. runs one prefill chunk of one request (B = 1; the history is dequantized on the
   GPU and read by SDPA, ``packed_backend.winnow_packed_attention``);
4. runs one batched decode forward for every request past its prefill, each at its
   own position, through the HIP compressed-domain operator.

Submissions that can never be served (empty or over-long prompts, a worst case
beyond the per-request page cap, a full queue, a duplicate id, shutdown) raise
``Refused`` with a machine-readable reason. Greedy decoding makes a request's
tokens a function of its prompt alone, so a batched run must equal the request
run by itself; the tests check exactly that.

On the device side one decode step is one forward whose page table and lengths
are uploaded once (``PagedPackedCache``), the append is one fused launch per layer
and the attention one operator call per layer; the host reads back one token id
per request per step.
"""
from __future__ import annotations

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
        super().__init__(reason if not detail else f"{reason}: {detail}")
        self.reason = reason


@dataclass
class Request:
    """One generation request and the engine's bookkeeping for it (engine.py:43-62)."""

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
    stored: int = 0                          # tokens already in the cache
    submitted_at: float = 0.0
    first_token_at: float | None = None
    token_times: list[float] = field(default_factory=list)
    finished_at: float | None = None
    cancel_requested: bool = False
    done: threading.Event = field(default_factory=threading.Event)


@dataclass
class EngineConfig:
    """Admission and batching limits (engine.py:65-71)."""

    max_batch: int = 8
    max_queue: int = 64
    prefill_chunk: int = 512
    max_prompt_tokens: int = 8192
    max_new_tokens_cap: int = 512
    decode_backend: str = "auto"


class Engine:
    """Single scheduler (``step``), any number of submitting / cancelling threads."""

    def __init__(self, model, pool, k_quant, v_quant, head_dim: int, eos_ids=(),
                 config: EngineConfig | None = None, clock=time.monotonic):
        self.model, self.pool = model, pool
        self.kq, self.vq, self.head_dim = k_quant, v_quant, head_dim
        self.eos = frozenset(int(e) for e in eos_ids)
        self.cfg = config or EngineConfig()
        self.clock = clock
        self.device = next(model.parameters()).device
        self._lock = threading.Lock()         # queue, id map, cancel flags
        self._step_lock = threading.Lock()    # one step at a time
        self._queue: deque[Request] = deque()
        self._active: list[Request] = []
        self._by_id: dict[str, Request] = {}
        self.closed = False
        self.steps = 0
        self.on_logits = None                 # diagnostic hook: (requests, fp32 logits)

    # ---- client side ----------------------------------------------------
    def submit(self, req: Request) -> Request:
        c = self.cfg
        n = len(req.prompt_ids)
        if self.closed:
            raise Refused("shutting_down")
        if n == 0:
            raise Refused("empty_prompt")
        if n > c.max_prompt_tokens:
            raise Refused("prompt_too_long", f"{n} > {c.max_prompt_tokens}")
        if not 1 <= req.max_new_tokens <= c.max_new_tokens_cap:
            raise Refused("bad_max_new_tokens", f"must be 1..{c.max_new_tokens_cap}")
        pages = self.pool.pages_for(n + req.max_new_tokens)
        if pages > self.pool.max_pages_per_request:
            raise Refused("exceeds_request_cap", f"{pages} pages > {self.pool.max_pages_per_request}")
        with self._lock:
            if req.request_id in self._by_id:
                raise Refused("duplicate_request_id")
            if len(self._queue) >= c.max_queue:
                raise Refused("queue_full", f"{c.max_queue} queued")
            req.submitted_at = self.clock()
            self._queue.append(req)
            self._by_id[req.request_id] = req
        return req

    def cancel(self, request_id: str) -> bool:
        with self._lock:
            req = self._by_id.get(request_id)
            if req is None or req.state == "done":
                return False
            req.cancel_requested = True
            return True

    def idle(self) -> bool:
        with self._lock:
            return not self._queue and not self._active

    def shutdown(self) -> None:
        """Refuse new work and end everything outstanding as cancelled."""
        with self._lock:
            self.closed = True
            for r in (*self._queue, *self._active):
                r.cancel_requested = True
                r.detail = "server shutting down"
        self.step()

    # ---- scheduler side -------------------------------------------------
    def _emit(self, req: Request, **event) -> None:
        if req.on_event is not None:
            req.on_event(req, event)

    def _finish(self, req: Request, status: str, detail: str = "", fence=None) -> None:
        req.state, req.status = "done", status
        req.detail = req.detail or detail
        req.finished_at = self.clock()
        self.pool.release(req.request_id, fence)
        with self._lock:
            self._by_id.pop(req.request_id, None)
        self._emit(req, kind="final", status=status, detail=req.detail)
        req.done.set()

    def _reap(self) -> None:
        now = self.clock()
        with self._lock:
            candidates = [*self._queue, *self._active]
        for req in candidates:
            if req.cancel_requested:
                why = "cancelled"
            elif req.deadline is not None and now > req.deadline:
                why = "deadline"
            else:
                continue
            with self._lock:
                if req in self._queue:
                    self._queue.remove(req)
            if req in self._active:
                self._active.remove(req)
            self._finish(req, why)            # the pool fences the release itself

    def _admit(self) -> None:
        while len(self._active) < self.cfg.max_batch:
            with self._lock:
                if not self._queue:
                    return
                head = self._queue[0]
            try:
                self.pool.ensure(head.request_id, len(head.prompt_ids) + head.max_new_tokens)
            except PoolExhausted:
                return                        # first in, first served: nobody overtakes
            with self._lock:
                self._queue.popleft()
            head.state = "prefill"
            self._active.append(head)

    def _forward(self, reqs: list[Request], input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        cache = PagedPackedCache(self.pool, [r.request_id for r in reqs], [r.stored for r in reqs],
                                 k_quant=self.kq, v_quant=self.vq, head_dim=self.head_dim,
                                 decode_backend=self.cfg.decode_backend)
        out = self.model(input_ids=input_ids, position_ids=positions, past_key_values=cache,
                         use_cache=True, logits_to_keep=1)
        for r, n in zip(reqs, cache.lengths):
            r.stored = n
        logits = out.logits[:, -1].float()
        if self.on_logits is not None:
            self.on_logits(reqs, logits)
        return logits

    def _accept(self, req: Request, token: int, now: float) -> str | None:
        """Record a generated token; the reason to stop, if any."""
        req.generated.append(token)
        req.token_times.append(now)
        if req.first_token_at is None:
            req.first_token_at = now
        self._emit(req, kind="token", index=len(req.generated) - 1, token_id=token, t=now)
        if token in self.eos and not req.ignore_eos:
            return "eos"
        return "length" if len(req.generated) >= req.max_new_tokens else None

    def _fence(self):
        return default_fence(self.device)

    def step(self) -> bool:
        """One scheduling iteration; False when there was nothing to run."""
        with self._step_lock:
            return self._step()

    @torch.no_grad()
    def _step(self) -> bool:
        self.steps += 1
        self._reap()
        self._admit()
        ran = False
        ended: list[tuple[Request, str]] = []

        req = next((r for r in self._active if r.state == "prefill"), None)
        if req is not None:
            ran = True
            lo = req.stored
            hi = min(lo + self.cfg.prefill_chunk, len(req.prompt_ids))
            try:
                logits = self._forward([req], torch.tensor([req.prompt_ids[lo:hi]], device=self.device),
                                       torch.arange(lo, hi, device=self.device)[None])
            except Exception as exc:  # noqa: BLE001 - reported on the request
                self._active.remove(req)
                self._finish(req, "error", f"{type(exc).__name__}: {exc}", self._fence())
                req = None
            if req is not None and hi == len(req.prompt_ids):
                req.state = "decode"
                why = self._accept(req, int(logits[0].argmax()), self.clock())
                if why:
                    ended.append((req, why))

        batch = [r for r in self._active if r.state == "decode" and all(r is not e for e, _ in ended)]
        if batch:
            ran = True
            try:
                logits = self._forward(batch, torch.tensor([[r.generated[-1]] for r in batch], device=self.device),
                                       torch.tensor([[r.stored] for r in batch], device=self.device))
                tokens = logits.argmax(-1).tolist()
                now = self.clock()
                for r, t in zip(batch, tokens):
                    why = self._accept(r, int(t), now)
                    if why:
                        ended.append((r, why))
            except Exception as exc:  # noqa: BLE001
                fence = self._fence()
                for r in batch:
                    self._active.remove(r)
                    self._finish(r, "error", f"{type(exc).__name__}: {exc}", fence)

        if ended:
            fence = self._fence()
            for r, why in ended:
                self._active.remove(r)
                self._finish(r, why, fence=fence)
        return ran

    def run_until_idle(self, max_steps: int = 100000) -> None:
        for _ in range(max_steps):
            if self.idle():
                return
            self.step()
        raise RuntimeError("engine did not drain")
