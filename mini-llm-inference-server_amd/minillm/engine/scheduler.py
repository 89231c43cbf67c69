"""Iteration-level scheduler over the paged pool (reference src/minillm/engine/scheduler.py:77-187).

Each step is either a prefill step (admit waiting requests FCFS, without skipping, while the batch,
the token budget and the pool allow, keeping one block in reserve for every request whose next token
starts a new block) or a decode step for every running request (a request at a block boundary gets
one more block; when none is free the newest request is preempted and requeued at the front, to be
recomputed).  With a prefix cache, an admitted request reuses the cached blocks of its longest named
prefix and only the rest is prefilled.  Bookkeeping only: block ids, no tensors.

With `chunked_prefill` a step mixes both kinds (the reference's planned M7:
docs/decisions/09-scheduler-policy.md, "Mixed prefill + decode steps"): every decoding request gets
its one token, then requests still inside their prompt get their next chunk (oldest first), then
waiting requests are admitted FCFS into what is left of the token budget, each with a first chunk.
A chunk that stops before a request's last uncached token samples nothing; the prompt continues on top
of its own cached tokens next step (reference tests/test_paged.py:142-146).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from ..cache.prefix import extend_chain
from .block_manager import BlockManager


@dataclass(eq=False)
class Request:
    req_id: str
    prompt: list[int]
    max_tokens: int
    stop_ids: frozenset
    timeline: dict
    output: list[int] = field(default_factory=list)
    block_ids: list[int] = field(default_factory=list)
    num_cached: int = 0  # tokens whose k/v are in the pool
    num_preemptions: int = 0
    root: bytes = b""
    block_hashes: list[bytes] = field(default_factory=list)
    num_named: int = 0  # leading blocks already named in the prefix cache
    num_cached_tokens: int | None = None  # prompt tokens served from the cache at first admission

    @property
    def num_tokens(self) -> int:
        return len(self.prompt) + len(self.output)

    def uncached(self) -> list[int]:
        return (self.prompt + self.output)[self.num_cached:]


@dataclass
class SchedulerOutput:
    prefill: list[Request]
    decode: list[Request]
    preempted: list[Request] = field(default_factory=list)
    chunks: dict = field(default_factory=dict)  # request -> new tokens this step (every scheduled row)

    def rows(self) -> list[tuple[Request, int]]:
        """(request, number of new tokens) for every row of the step, decode rows first."""
        return [(r, self.chunks[r]) for r in self.decode + self.prefill]


class Scheduler:
    def __init__(self, max_num_seqs: int, max_num_batched_tokens: int, blocks: BlockManager, prefix=None,
                 chunked_prefill: bool = False) -> None:
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.blocks = blocks
        self.prefix = prefix
        self.chunked_prefill = chunked_prefill
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []  # admission order, newest last
        self.num_preemptions = 0

    def add(self, req: Request) -> None:
        self.waiting.append(req)

    def schedule(self) -> SchedulerOutput:
        if self.chunked_prefill:
            return self._schedule_mixed()
        admitted = self._admit()
        if admitted:
            return SchedulerOutput(prefill=admitted, decode=[], chunks={r: len(r.uncached()) for r in admitted})
        preempted = self._grow_running()
        return SchedulerOutput(prefill=[], decode=list(self.running), preempted=preempted,
                               chunks={r: 1 for r in self.running})

    def _at_boundary(self, req: Request) -> bool:
        return req.num_cached >= len(req.block_ids) * self.blocks.block_size

    def _decoding(self, req: Request) -> bool:
        """Past its prompt: one uncached token, the last sampled one."""
        return req.num_tokens - req.num_cached == 1 and bool(req.output)

    def _admit(self) -> list[Request]:
        reserve = sum(1 for r in self.running if self._at_boundary(r))
        admitted: list[Request] = []
        budget_used = 0
        for req in list(self.waiting):
            if len(self.running) == self.max_num_seqs:
                break
            taken = self._take(req, reserve, None if not admitted else self.max_num_batched_tokens - budget_used)
            if taken is None:
                break
            to_compute, spare = taken
            reserve += spare
            budget_used += to_compute
            admitted.append(req)
        for req in admitted:
            self.waiting.remove(req)
        return admitted

    def _take(self, req: Request, reserve: int, budget: int | None) -> tuple[int, int] | None:
        """Admits `req` into the running set when its tokens fit `budget` (None: no limit) and the pool
        has blocks for all its tokens plus `reserve`; returns (tokens to compute, spare blocks it reserves)."""
        bs = self.blocks.block_size
        n = req.num_tokens
        hits = self._lookup(req)
        to_compute = n - len(hits) * bs
        if budget is not None and to_compute > budget:
            return None
        total = self.blocks.blocks_for(n)
        need = total - len(hits)
        revive = sum(1 for b in hits if self.blocks.is_cached_unheld(b))
        spare = 1 if n == total * bs else 0  # its first decode token will start a new block
        if need + revive + spare + reserve > self.blocks.num_free:
            return None
        self.blocks.acquire(hits)
        req.block_ids = hits + self.blocks.allocate(need)
        req.num_cached = len(hits) * bs
        req.num_named = len(hits)
        if self.prefix is not None:
            self.prefix.queries += n
            self.prefix.hits += len(hits) * bs
        if req.num_cached_tokens is None:
            req.num_cached_tokens = len(hits) * bs
        self.running.append(req)
        return to_compute, spare

    def _schedule_mixed(self) -> SchedulerOutput:
        preempted = self._grow_running()
        budget = self.max_num_batched_tokens
        decode = [r for r in self.running if self._decoding(r)][:budget]
        chunks = {r: 1 for r in decode}
        budget -= len(decode)
        prefill = []
        for r in self.running:  # prompts already under way, oldest first
            if r in chunks or budget == 0:
                continue
            n = min(budget, len(r.uncached()))
            chunks[r], budget = n, budget - n
            prefill.append(r)
        # FCFS admission into the rest of the budget; one block of reserve for every running request
        # whose next sampled token starts a new block
        bs = self.blocks.block_size
        reserve = sum(1 for r in self.running if len(r.block_ids) * bs <= r.num_tokens)
        while self.waiting and budget > 0 and len(self.running) < self.max_num_seqs:
            req = self.waiting[0]
            taken = self._take(req, reserve, None)
            if taken is None:
                break
            self.waiting.popleft()
            n = min(budget, len(req.uncached()))
            chunks[req], budget = n, budget - n
            reserve += taken[1]
            prefill.append(req)
        return SchedulerOutput(prefill=prefill, decode=decode, preempted=preempted, chunks=chunks)

    def _lookup(self, req: Request) -> list[int]:
        """Cached blocks of the request's first (num_tokens - 1) tokens: the last token is always
        computed, so the step has logits to sample."""
        if self.prefix is None:
            return []
        bs = self.blocks.block_size
        k = (req.num_tokens - 1) // bs
        if k == 0:
            return []
        extend_chain(req.block_hashes, req.root, req.prompt + req.output, k, bs)
        return self.prefix.lookup(req.block_hashes[:k])

    def name_full_blocks(self, reqs: list[Request]) -> None:
        if self.prefix is None:
            return
        bs = self.blocks.block_size
        for req in reqs:
            full = req.num_cached // bs
            if full <= req.num_named:
                continue
            extend_chain(req.block_hashes, req.root, req.prompt + req.output, full, bs)
            for j in range(req.num_named, full):
                self.prefix.insert(req.block_hashes[j], req.block_ids[j])
            req.num_named = full

    def _grow_running(self) -> list[Request]:
        preempted: list[Request] = []
        for req in list(self.running):  # oldest first
            if req not in self.running or not self._at_boundary(req):
                continue
            while self.blocks.num_free == 0:
                victim = self.running[-1]
                self._preempt(victim)
                preempted.append(victim)
                if victim is req:
                    break
            if req in self.running:
                req.block_ids += self.blocks.allocate(1)
        return preempted

    def _preempt(self, req: Request) -> None:
        self.running.remove(req)
        self.blocks.free(req.block_ids)
        req.num_cached = req.num_named = 0
        req.num_preemptions += 1
        self.num_preemptions += 1
        self.waiting.appendleft(req)

    def finish(self, reqs: list[Request]) -> None:
        for req in reqs:
            self.running.remove(req)
            self.blocks.free(req.block_ids)

    def remove_waiting(self, req_id: str) -> Request | None:
        for req in self.waiting:
            if req.req_id == req_id:
                self.waiting.remove(req)
                return req
        return None
