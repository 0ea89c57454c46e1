"""Continuous batching over the paged pool, after scheduler/scheduler.py of the reference.

Policy per step (the reference's ``Scheduler.loop``, scheduler.py:508-653):

* Running requests are served in admission order under a token budget
  (scheduler.py:576-627): a request whose prompt is cached (``prefilled``)
  gets 1 token (its last generated token) and one more page when its pages are
  full; a request still prefilling gets ``min(remaining budget, uncached
  tokens)`` and the pages that chunk needs.  Once the budget is spent the
  rest get nothing this step.
* When the free pages do not cover the step, the newest running requests are
  preempted (scheduler.py:629-643, 359-372): their pages and KV are dropped and
  they recompute from scratch later (prompt plus the tokens they generated).
* Free slots, lowest id first, then admit requests while budget remains
  (scheduler.py:377-433): preempted requests first (the last preempted
  first), then new ones in arrival order, each with ``min(remaining budget,
  prompt + generated)`` tokens; a request whose pages do not fit goes back and
  admission stops.  Its page count rounds a page-aligned chunk up by one page
  (``_required_pages``, scheduler.py:209-218).
* If any served request is prefilling, the step is one packed mixed step
  (the mixed module of the smallest token bucket that fits: a graph replay
  by default); otherwise a decode step (``DecodeModule`` of the smallest batch
  bucket that fits, one hipGraph replay) (scheduler.py:655-720).
* Afterwards each served request's KV length grows by its budget; a request
  whose prompt and generated tokens are all cached takes the step's token, and
  finishes on an EOS token or after ``max_new_tokens`` tokens, freeing its slot
  and pages (scheduler.py:320-357).

Slot 0 and page 0 stay reserved for the padding rows of fixed-size steps.
The steps run through a ``StepExecutor``; ``ModuleExecutor`` is the GPU one
(step modules over the HIP kernels), and tests may pass their own.
"""
from __future__ import annotations

import math
import queue
import time
from collections import Counter
from concurrent.futures import Future, InvalidStateError
from dataclasses import dataclass, field
from typing import ClassVar, Protocol


@dataclass
class Request:
    """One generation request (scheduler/models.py:6-22 of the reference)."""
    future: Future
    prompt: list[int]
    t_arrival: float
    t_first: float = 0.0
    kv_len: int = 0          # tokens of prompt + new_tokens already in the pool
    budget: int = 0          # tokens this step feeds
    new_tokens: list[int] = field(default_factory=list)
    pages: list[int] = field(default_factory=list)
    prefilled: bool = False

    def requires_page(self, page_size: int) -> bool:
        return len(self.pages) * page_size == self.kv_len

    def uncached_token_count(self) -> int:
        return len(self.prompt) + len(self.new_tokens) - self.kv_len


@dataclass
class RequestResult:
    new_tokens: list[int]
    t_arrival: float
    t_first: float
    t_end: float


@dataclass
class RunStats:
    decode_steps: Counter = field(default_factory=Counter)  # batch bucket -> steps
    mixed_steps: Counter = field(default_factory=Counter)   # token bucket -> steps
    batch_sizes: Counter = field(default_factory=Counter)   # served requests -> steps
    tokens: int = 0           # tokens fed to mixed steps
    bucket_tokens: int = 0    # their bucket sizes (padding included)
    preemptions: int = 0
    recomputed_tokens: int = 0


class StepExecutor(Protocol):
    """Runs one step on the model; returns one next token per slot."""

    def decode(self, slot_ids: list[int]) -> list[int]: ...

    def mixed(self, chunks: list[list[int]], slot_ids: list[int]) -> list[int]: ...


def _smallest_fit(sizes, value: int) -> int:
    for size in sorted(sizes):
        if size >= value:
            return size
    raise RuntimeError(f"no bucket holds {value}")


def batch_buckets(n_slots: int, buckets=(1, 2, 4, 8, 16, 32)) -> list[int]:
    """Decode batch buckets up to the first that holds every usable slot."""
    out = []
    for size in buckets:
        out.append(size)
        if size >= n_slots - 1:
            break
    return out


def token_buckets(token_budget: int, min_bucket: int = 16, full_threshold: int = 128,
                  step: int = 32) -> list[int]:
    """Mixed-step token buckets: doubling up to the threshold, then fixed steps to the budget."""
    out, size = [], min_bucket
    while size < full_threshold:
        out.append(size)
        size *= 2
    out.append(full_threshold)
    out.extend(range(full_threshold + step, token_budget + step, step))
    return out


class ModuleExecutor:
    """Steps on the GPU through the step modules.

    Every graph is captured here, before any request runs (the captures'
    warm-ups touch only the reserved slot 0 and page 0): one ``DecodeModule``
    per batch bucket and, with ``graph_mixed``, one ``FullMixedModule`` per
    token bucket at the largest batch bucket (padded sequences cost nothing,
    so one graph serves every batch size).
    Without it, mixed steps run eagerly (``MixedModule`` of the token bucket,
    made on first use).  With ``piecewise_above`` set, the token buckets above
    it use ``PiecewiseMixedModule`` instead, sharing one attention-output
    buffer, as the reference's ``PiecewiseGraphBackend`` does for buckets above
    its full-graph threshold (scheduler/graph_backend.py:64-95).
    """

    def __init__(self, model, kv_cache, batch_sizes: list[int], token_counts: list[int], pool=None,
                 graph_mixed: bool = True, piecewise_above: int | None = None):
        import torch

        from .decode_module import DecodeModule
        from .mixed_module import FullMixedModule, PiecewiseMixedModule

        self.model = model
        self.kv_cache = kv_cache
        self.token_counts = sorted(token_counts)
        self.pool = pool if pool is not None else torch.cuda.graph_pool_handle()
        self.decode_modules = {b: DecodeModule(model, kv_cache, batch_size=b, pool=self.pool)
                               for b in sorted(batch_sizes, reverse=True)}
        self.max_batch = max(batch_sizes)
        self.mixed_modules = {}
        piecewise = [t for t in self.token_counts if piecewise_above is not None and t > piecewise_above]
        if graph_mixed and piecewise:
            self.buffer = torch.zeros((1, max(piecewise), kv_cache.num_q_heads, kv_cache.head_dim),
                                      dtype=kv_cache.dtype, device=kv_cache.device)
        if graph_mixed:
            for t in sorted(self.token_counts, reverse=True):
                if t in piecewise:
                    self.mixed_modules[t] = PiecewiseMixedModule(model, kv_cache, token_count=t,
                                                                 buffer=self.buffer, pool=self.pool,
                                                                 batch_size=self.max_batch)
                else:
                    self.mixed_modules[t] = FullMixedModule(model, kv_cache, batch_size=self.max_batch,
                                                            token_count=t, pool=self.pool)

    def decode_module(self, n: int):
        return self.decode_modules[_smallest_fit(self.decode_modules, n)]

    def mixed_module(self, n_tokens: int):
        from .mixed_module import MixedModule

        bucket = _smallest_fit(self.token_counts, n_tokens)
        if bucket not in self.mixed_modules:
            self.mixed_modules[bucket] = MixedModule(self.model, self.kv_cache, token_count=bucket,
                                                     batch_size=self.max_batch)
        return self.mixed_modules[bucket]

    def decode(self, slot_ids: list[int]) -> list[int]:
        return self.decode_module(len(slot_ids)).forward(slot_ids)

    def mixed(self, chunks: list[list[int]], slot_ids: list[int]) -> list[int]:
        return self.mixed_module(sum(map(len, chunks))).forward(chunks, slot_ids)


class Scheduler:
    """Continuous-batching loop over a model with the paged-attention drop-in.

    Unlike the reference (which loads ``model_id`` from the hub and builds its
    graph backends itself, scheduler.py:25-127) this takes a ready model and
    KV storage, and a step executor (``ModuleExecutor`` by default).  Requests
    come in through ``call`` (returns a Future of ``RequestResult``);
    ``loop`` serves until ``stop`` has been called and every request is done;
    ``generate`` is the synchronous form.
    """

    DECODE_BATCH_BUCKETS: ClassVar[tuple] = (1, 2, 4, 8, 16, 32)
    MIN_TOKEN_BUCKET: ClassVar[int] = 16
    FULL_GRAPH_TOKEN_THRESHOLD: ClassVar[int] = 128
    PIECEWISE_TOKEN_STEP: ClassVar[int] = 32

    SENTINEL: ClassVar[object] = object()

    def __init__(self, model, kv_cache, eos_token_ids: set[int], max_new_tokens: int,
                 token_budget: int, executor: StepExecutor | None = None,
                 piecewise_mixed: bool = False) -> None:
        n_slots = kv_cache.n_slots
        if n_slots <= 1:
            raise ValueError("n_slots must be greater than 1.")
        if n_slots - 1 > self.DECODE_BATCH_BUCKETS[-1]:
            raise ValueError("n_slots can't be larger than largest bucket size.")
        if max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be positive.")
        if not eos_token_ids:
            raise ValueError("eos_token_ids must not be empty.")
        if token_budget <= n_slots - 1:
            raise ValueError("token_budget must be greater than n_slots - 1.")
        if token_budget <= self.FULL_GRAPH_TOKEN_THRESHOLD:
            raise ValueError("token_budget must be greater than FULL_GRAPH_TOKEN_THRESHOLD.")
        if token_budget % self.PIECEWISE_TOKEN_STEP != 0:
            raise ValueError("token_budget must be a multiple of PIECEWISE_TOKEN_STEP.")

        self.model = model
        self.kv_cache = kv_cache
        self.n_slots = n_slots
        self.page_size = kv_cache.page_size
        self.n_pages = kv_cache.n_pages
        self.max_new_tokens = max_new_tokens
        self.token_budget = token_budget
        self.eos_token_ids = frozenset(eos_token_ids)
        if self._required_pages(1, total=True) > self.n_pages - 1:
            raise ValueError(f"max_new_tokens can't need more than {self.n_pages - 1} pages.")
        self.batch_sizes = batch_buckets(n_slots, self.DECODE_BATCH_BUCKETS)
        self.token_counts = token_buckets(token_budget, self.MIN_TOKEN_BUCKET,
                                          self.FULL_GRAPH_TOKEN_THRESHOLD, self.PIECEWISE_TOKEN_STEP)
        self.executor = executor if executor is not None else ModuleExecutor(
            model, kv_cache, self.batch_sizes, self.token_counts,
            piecewise_above=self.FULL_GRAPH_TOKEN_THRESHOLD if piecewise_mixed else None)

        self.stats = RunStats()
        self.requests: queue.Queue = queue.Queue()
        self.preempted: list[Request] = []
        self.order: list[int] = []  # running slots, in admission order
        self.slots: list[Request | None] = [None] * n_slots
        self.open = True
        self._reset_occupancy()

    # ------------------------------------------------------------------ pages / slots

    def _reset_occupancy(self) -> None:
        unused = self.kv_cache.unused_idx
        # a stack: pop() hands out the lowest free page first
        self._free_pages: list[int] = [p for p in range(self.n_pages - 1, -1, -1) if p != unused]
        self._free_slots: set[int] = set(range(self.n_slots)) - {unused}
        self._busy_slots: set[int] = set()

    def _required_pages(self, n_tokens: int, total: bool) -> int:
        L = n_tokens + (self.max_new_tokens if total else 0)
        if L % self.page_size == 0:
            L += 1
        return math.ceil(L / self.page_size)

    def _palloc(self, slot_ids: list[int], page_counts: list[int]) -> None:
        if len(slot_ids) != len(page_counts):
            raise RuntimeError("Unmatching page counts.")
        if any(c < 0 or c > self.n_pages - 1 - len(self.slots[s].pages)
               for s, c in zip(slot_ids, page_counts)):
            raise RuntimeError("Invalid page counts.")
        if sum(page_counts) > len(self._free_pages):
            raise RuntimeError("No enough pages to allocate.")
        for s, count in zip(slot_ids, page_counts):
            if count == 0:
                continue
            req = self.slots[s]
            start = len(req.pages)
            new = [self._free_pages.pop() for _ in range(count)]
            self.kv_cache.block_table[s, start:start + count] = self._device_ids(new)
            req.pages.extend(new)

    def _device_ids(self, ids: list[int]):
        import torch
        return torch.tensor(ids, dtype=torch.long).to(self.kv_cache.block_table.device)

    def _release(self, slot_ids: list[int]) -> None:
        """Free the slots and their pages; the pool forgets their lengths and rows."""
        for s in slot_ids:
            req = self.slots[s]
            if req is not None:
                self._free_pages.extend(sorted(req.pages, reverse=True))
            self.slots[s] = None
            self._busy_slots.discard(s)
            self._free_slots.add(s)
            if s in self.order:
                self.order.remove(s)
        if slot_ids:
            self.kv_cache.reset(slot_ids)

    # ------------------------------------------------------------------ one step

    def _plan_running(self) -> int:
        """Budgets and pages for the running slots; preempts the newest when pages run short."""
        slot_ids, page_counts, budgets = [], [], []
        left = self.token_budget
        for s in self.order:
            req = self.slots[s]
            slot_ids.append(s)
            if left <= 0:
                budgets.append(0)
                page_counts.append(0)
                continue
            if req.prefilled:
                page_counts.append(1 if req.requires_page(self.page_size) else 0)
                budgets.append(1)
                left -= 1
            else:
                n = min(left, req.uncached_token_count())
                page_counts.append(math.ceil((req.kv_len + n) / self.page_size) - len(req.pages))
                budgets.append(n)
                left -= n

        freed, victims = 0, []
        while len(self._free_pages) + freed < sum(page_counts):
            s = slot_ids.pop()
            freed += len(self.slots[s].pages)
            victims.append(s)
            page_counts.pop()
            left += budgets.pop()
        self._preempt(victims)
        self._palloc(slot_ids, page_counts)
        for s, n in zip(slot_ids, budgets):
            self.slots[s].budget = n
        return left

    def _preempt(self, slot_ids: list[int]) -> None:
        reqs = [self.slots[s] for s in slot_ids]
        self._release(slot_ids)
        self.stats.preemptions += len(reqs)
        for req in reqs:
            self.stats.recomputed_tokens += req.kv_len
            req.prefilled = False
            req.kv_len = 0
            req.pages = []
            req.budget = 0
            self.preempted.append(req)

    def _admit(self, wait: bool, only_preempted: bool, left: int) -> None:
        slot_ids, page_counts, budgets = [], [], []
        for s in sorted(self._free_slots):
            if left <= 0:
                break
            if self.preempted:
                req = self.preempted.pop()
            elif not only_preempted:
                if wait:
                    req = self.requests.get()
                    wait = False
                else:
                    try:
                        req = self.requests.get_nowait()
                    except queue.Empty:
                        break
            else:
                break
            if req is self.SENTINEL:
                self.open = False
                break
            n = min(left, len(req.prompt) + len(req.new_tokens))
            need = self._required_pages(n, total=False)
            if need > len(self._free_pages) - sum(page_counts):
                self.preempted.append(req)  # back to the front of the line
                break
            self.order.append(s)
            self.slots[s] = req
            self._free_slots.discard(s)
            self._busy_slots.add(s)
            slot_ids.append(s)
            page_counts.append(need)
            budgets.append(n)
            left -= n
        for s, n in zip(slot_ids, budgets):
            self.slots[s].budget = n
        self._palloc(slot_ids, page_counts)

    def _run_step(self) -> None:
        served = [s for s in self.order if self.slots[s].budget > 0]
        if not served:
            return
        self.stats.batch_sizes[len(served)] += 1
        if all(self.slots[s].prefilled for s in served):
            self.stats.decode_steps[_smallest_fit(self.batch_sizes, len(served))] += 1
            tokens = self.executor.decode(served)
        else:
            chunks = []
            for s in served:
                req = self.slots[s]
                full = req.prompt + req.new_tokens
                chunks.append(full[req.kv_len:req.kv_len + req.budget])
            n = sum(map(len, chunks))
            self.stats.mixed_steps[_smallest_fit(self.token_counts, n)] += 1
            self.stats.tokens += n
            self.stats.bucket_tokens += _smallest_fit(self.token_counts, n)
            tokens = self.executor.mixed(chunks, served)
        self._refresh(served, tokens)

    def _refresh(self, slot_ids: list[int], next_tokens: list[int]) -> None:
        done = []
        now = time.perf_counter()
        for s, token in zip(slot_ids, next_tokens):
            req = self.slots[s]
            req.kv_len += req.budget
            if not req.prefilled and req.kv_len == len(req.prompt) + len(req.new_tokens):
                req.prefilled = True
            if not req.prefilled:
                continue
            if token in self.eos_token_ids or len(req.new_tokens) == self.max_new_tokens - 1:
                _complete(req.future, RequestResult(new_tokens=req.new_tokens + [token],
                                                    t_arrival=req.t_arrival,
                                                    t_first=req.t_first or now, t_end=now))
                done.append(s)
            else:
                if not req.new_tokens:
                    req.t_first = now
                req.new_tokens.append(token)
        self._release(done)

    # ------------------------------------------------------------------ public surface

    def call(self, prompt: list[int]) -> Future:
        fut: Future = Future()
        if not self.open:
            fut.set_exception(RuntimeError("Loop is not open."))
        elif len(prompt) == 0:
            fut.set_exception(ValueError("Empty prompts are not allowed."))
        elif self._required_pages(len(prompt), total=True) > self.n_pages - 1:
            fut.set_exception(ValueError("Possible amount of tokens exceeds available pages."))
        else:
            self.requests.put(Request(future=fut, prompt=list(prompt), t_arrival=time.perf_counter()))
        return fut

    def stop(self) -> None:
        self.requests.put(self.SENTINEL)

    def step(self) -> bool:
        """One scheduling round; False once the loop has nothing left to do."""
        if self.open:
            if self._busy_slots:
                self._admit(wait=False, only_preempted=False, left=self._plan_running())
            else:
                self._admit(wait=True, only_preempted=False, left=self.token_budget)
            self._run_step()
            return True
        if self._busy_slots or self.preempted:
            self._admit(wait=False, only_preempted=True, left=self._plan_running())
            self._run_step()
            return True
        return False

    def loop(self) -> None:
        try:
            while self.step():
                pass
            self._end(RuntimeError("Loop has been terminated."))
        except Exception as exc:  # fail every pending request, then surface the error
            self._end(exc)
            raise

    def generate(self, prompts: list[list[int]]) -> list[RequestResult]:
        """Serve ``prompts`` to completion in this thread; results in prompt order."""
        futures = [self.call(p) for p in prompts]
        self.stop()
        self.loop()
        return [f.result() for f in futures]

    def _end(self, exc: Exception) -> None:
        for s in list(self._busy_slots):
            _fail(self.slots[s].future, exc)
        while True:
            try:
                req = self.requests.get_nowait()
            except queue.Empty:
                break
            if req is self.SENTINEL:
                self.open = False
            else:
                _fail(req.future, exc)
        while self.preempted:
            _fail(self.preempted.pop().future, exc)
        self._release(sorted(self._busy_slots))
        self.order.clear()
        self._reset_occupancy()


def _complete(future: Future, result: RequestResult) -> None:
    try:
        future.set_result(result)
    except InvalidStateError:
        pass


def _fail(future: Future, exc: Exception) -> None:
    try:
        future.set_exception(exc)
    except InvalidStateError:
        pass
