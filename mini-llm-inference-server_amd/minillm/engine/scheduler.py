"""Iteration-level scheduler over the paged pool: which requests run in a step, and with how many new
tokens each.  Bookkeeping only (block ids, counters), no tensors.

Rules (reference src/minillm/engine/scheduler.py:77-187 and docs/decisions/09-scheduler-policy.md state
them; the code is this build's own):
- a step is a prefill step while waiting requests can be admitted, else a decode step of every running
  request;
- admission is first come, first served, without skipping: it stops at the first waiting request that
  does not fit.  A request fits when fewer than `max_num_seqs` run, its tokens to compute fit the step's
  budget (the first request of a step always does), and the pool can give it every block its tokens
  need plus one spare block for each running or admitted request whose next token opens a new block;
- a prefix-cache hit shares the named blocks of the request's longest named prefix (its last token is
  always computed, so the step has logits to sample);
- a decode step first gives every running request at a block boundary one more block, oldest first;
  when the pool is empty the newest running request is preempted (its blocks released, its progress
  dropped) and put back at the front of the queue, to be recomputed when readmitted.

With `chunked_prefill` a step mixes both kinds (the reference's planned M7: docs/decisions/09-scheduler-
policy.md, "Mixed prefill + decode steps"): every decoding request gets its one token, then requests
still inside their prompt get their next chunk (oldest first), then waiting requests are admitted FCFS
into what is left of the token budget, each with a first chunk.  A chunk that stops short of a request's
last uncached token samples nothing; the prompt continues on top of its own cached tokens next step
(reference tests/test_paged.py:142-146).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

from ..cache.prefix import extend_chain
from .block_manager import BlockManager


@dataclass(eq=False)  # requests are compared by identity
class Request:
    req_id: str
    prompt: list[int]
    max_tokens: int
    stop_ids: frozenset
    timeline: dict
    output: list[int] = field(default_factory=list)
    block_ids: list[int] = field(default_factory=list)  # the block table, while it holds K/V
    num_cached: int = 0  # leading tokens whose K/V are in the pool
    num_preemptions: int = 0
    root: bytes = b""  # salted root of its prefix-hash chain
    block_hashes: list[bytes] = field(default_factory=list)  # names of its leading full blocks, as computed
    num_named: int = 0  # leading blocks of its table already named in the prefix cache
    num_cached_tokens: int | None = None  # prompt tokens served from the cache at its first admission

    @property
    def num_tokens(self) -> int:
        return len(self.prompt) + len(self.output)

    def uncached(self) -> list[int]:
        """The tokens whose K/V are not in the pool yet (prompt and output alike)."""
        n = len(self.prompt)
        c = self.num_cached
        return self.prompt[c:] + self.output if c <= n else self.output[c - n:]


@dataclass
class SchedulerOutput:
    prefill: list[Request]
    decode: list[Request]
    preempted: list[Request] = field(default_factory=list)
    chunks: dict = field(default_factory=dict)  # request -> new tokens this step (every scheduled row)

    def rows(self) -> list[tuple[Request, int]]:
        """(request, number of new tokens) for every row of the step, decode rows first."""
        return [(r, self.chunks[r]) for r in self.decode + self.prefill]


@dataclass
class _Claim:
    """What admitting one request takes: the named blocks it shares and what else the pool must give."""

    req: Request
    shared: list[int]  # blocks of its longest named prefix
    compute: int  # tokens to run through the model
    new_blocks: int  # blocks to allocate for the rest
    revived: int  # shared blocks nobody holds (they leave the pool's free count)
    spare: int  # 1 when its first sampled token opens a new block

    @property
    def pool_cost(self) -> int:
        return self.new_blocks + self.revived + self.spare


class Scheduler:
    def __init__(self, max_num_seqs: int, max_num_batched_tokens: int, blocks: BlockManager, prefix=None,
                 chunked_prefill: bool = False) -> None:
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.blocks = blocks
        self.prefix = prefix
        self.chunked_prefill = chunked_prefill
        self.waiting: deque[Request] = deque()
        self.running: list[Request] = []  # admission order: the newest is last
        self.num_preemptions = 0

    def add(self, req: Request) -> None:
        self.waiting.append(req)

    def schedule(self) -> SchedulerOutput:
        if self.chunked_prefill:
            return self._mixed_step()
        admitted = self._admit_prefills()
        if admitted:
            return SchedulerOutput(admitted, [], chunks={r: r.num_tokens - r.num_cached for r in admitted})
        preempted = self._make_room()
        return SchedulerOutput([], list(self.running), preempted, {r: 1 for r in self.running})

    # ------------------------------------------------------------------ admission

    def _claim(self, req: Request) -> _Claim:
        bs = self.blocks.block_size
        shared = self._longest_named_prefix(req)
        total = self.blocks.blocks_for(req.num_tokens)
        return _Claim(req, shared, compute=req.num_tokens - len(shared) * bs, new_blocks=total - len(shared),
                      revived=sum(1 for b in shared if self.blocks.is_cached_unheld(b)),
                      spare=int(req.num_tokens == total * bs))

    def _grant(self, claim: _Claim) -> None:
        """Moves the claimed request into the running set with its block table."""
        req, bs = claim.req, self.blocks.block_size
        self.blocks.acquire(claim.shared)  # first, so that the allocation below cannot evict them
        req.block_ids = claim.shared + self.blocks.allocate(claim.new_blocks)
        req.num_cached = len(claim.shared) * bs
        req.num_named = len(claim.shared)
        if req.num_cached_tokens is None:
            req.num_cached_tokens = req.num_cached
        if self.prefix is not None:
            self.prefix.queries += req.num_tokens
            self.prefix.hits += req.num_cached
        self.running.append(req)

    def _open_block_count(self) -> int:
        """Running requests whose next token, as of the last step, opens a new block."""
        bs = self.blocks.block_size
        return sum(1 for r in self.running if r.num_cached >= len(r.block_ids) * bs)

    def _admit_prefills(self) -> list[Request]:
        reserve = self._open_block_count()
        tokens = 0
        admitted: list[Request] = []
        while self.waiting and len(self.running) < self.max_num_seqs:
            claim = self._claim(self.waiting[0])
            over_budget = admitted and tokens + claim.compute > self.max_num_batched_tokens
            if over_budget or claim.pool_cost + reserve > self.blocks.num_free:
                break  # FCFS: nothing behind the head of the queue goes first
            self._grant(claim)
            admitted.append(self.waiting.popleft())
            reserve += claim.spare
            tokens += claim.compute
        return admitted

    def _mixed_step(self) -> SchedulerOutput:
        preempted = self._make_room()
        budget = self.max_num_batched_tokens
        decode = [r for r in self.running if r.output and r.num_tokens - r.num_cached == 1][:budget]
        chunks = {r: 1 for r in decode}
        budget -= len(decode)
        prefill = []
        for r in self.running:  # prompts already under way, oldest first
            if r in chunks or budget == 0:
                continue
            n = min(budget, r.num_tokens - r.num_cached)
            chunks[r], budget = n, budget - n
            prefill.append(r)
        # FCFS admission into the rest of the budget, with one spare block for every running request
        # whose next sampled token opens a new block
        bs = self.blocks.block_size
        reserve = sum(1 for r in self.running if len(r.block_ids) * bs <= r.num_tokens)
        while self.waiting and budget > 0 and len(self.running) < self.max_num_seqs:
            claim = self._claim(self.waiting[0])
            if claim.pool_cost + reserve > self.blocks.num_free:
                break
            self._grant(claim)
            req = self.waiting.popleft()
            n = min(budget, claim.compute)
            chunks[req], budget = n, budget - n
            reserve += claim.spare
            prefill.append(req)
        return SchedulerOutput(prefill, decode, preempted, chunks)

    # ------------------------------------------------------------------ prefix cache

    def _longest_named_prefix(self, req: Request) -> list[int]:
        """Named blocks covering the request's first num_tokens - 1 tokens, as far as the cache knows them."""
        if self.prefix is None:
            return []
        bs = self.blocks.block_size
        k = (req.num_tokens - 1) // bs
        if k <= 0:
            return []
        extend_chain(req.block_hashes, req.root, req.prompt + req.output, k, bs)
        return self.prefix.lookup(req.block_hashes[:k])

    def name_full_blocks(self, reqs: list[Request]) -> None:
        """After a step: names every block of `reqs` that its K/V filled since it was last named."""
        if self.prefix is None:
            return
        bs = self.blocks.block_size
        for req in reqs:
            full = req.num_cached // bs
            if full > req.num_named:
                extend_chain(req.block_hashes, req.root, req.prompt + req.output, full, bs)
                for j in range(req.num_named, full):
                    self.prefix.insert(req.block_hashes[j], req.block_ids[j])
                req.num_named = full

    # ------------------------------------------------------------------ growth and preemption

    def _make_room(self) -> list[Request]:
        """One more block for every running request at a block boundary, oldest first, preempting from the
        newest end while the pool is empty; returns the preempted requests, newest first."""
        bs = self.blocks.block_size
        preempted: list[Request] = []
        i = 0
        while i < len(self.running):
            req = self.running[i]
            if req.num_cached >= len(req.block_ids) * bs:
                while self.blocks.num_free == 0 and i < len(self.running):
                    preempted.append(self._requeue_newest())
                if i >= len(self.running):  # `req` itself went back to the queue, and all newer ones
                    break
                req.block_ids.extend(self.blocks.allocate(1))
            i += 1
        return preempted

    def _requeue_newest(self) -> Request:
        victim = self.running.pop()
        self.blocks.free(victim.block_ids)  # named blocks stay named: a readmission may find them again
        victim.num_cached = 0
        victim.num_named = 0
        victim.num_preemptions += 1
        self.num_preemptions += 1
        self.waiting.appendleft(victim)
        return victim

    # ------------------------------------------------------------------ leaving

    def finish(self, reqs: list[Request]) -> None:
        """Finished or aborted running requests leave the running set and release their blocks."""
        gone = set(map(id, reqs))
        self.running = [r for r in self.running if id(r) not in gone]
        for req in reqs:
            self.blocks.free(req.block_ids)

    def remove_waiting(self, req_id: str) -> Request | None:
        for i, req in enumerate(self.waiting):
            if req.req_id == req_id:
                del self.waiting[i]
                return req
        return None
