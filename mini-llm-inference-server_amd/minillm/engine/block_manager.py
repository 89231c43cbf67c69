"""Pool block accounting for the paged KV cache (reference src/minillm/engine/block_manager.py:21-96 states
the rules; this is an independent design).

Rules the engine relies on:
- a block is held (by as many block tables as list it), idle-blank (no KV worth keeping) or idle-named
  (no holder, but the prefix cache names it, so its KV may be revived);
- allocation takes idle-blank blocks first, oldest release first (the pool starts as 0 .. n-1), and only
  then evicts idle-named blocks, least recently released first, dropping their names;
- a released table is walked from its last block to its first, so a chain's tail is evicted before its
  head (a lookup stops at the first unnamed block, so an evicted head would strand the rest).

Design: per-block holder counts in an int32 array, and one reclaim heap of (tier, ticket, block) for the
idle blocks, tier 0 blank and tier 1 named, tickets increasing with every release.  Popping the heap
yields exactly the order above.  Re-acquiring an idle block voids its entry by setting the block's ticket
to -1 (a stale entry is dropped when it surfaces), so nothing is searched or moved on a prefix hit.
"""

from __future__ import annotations

import heapq
from collections import Counter

import numpy as np

BLANK, NAMED = 0, 1


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, prefix=None) -> None:
        self.num_blocks = int(num_blocks)
        self.block_size = int(block_size)
        self.prefix = prefix
        self._holders = np.zeros(self.num_blocks, dtype=np.int32)
        self._ticket = np.arange(self.num_blocks, dtype=np.int64)  # ticket of a block's live heap entry, -1 if none
        self._heap: list[tuple[int, int, int]] = [(BLANK, b, b) for b in range(self.num_blocks)]  # already a heap
        self._next_ticket = self.num_blocks
        self._idle = self.num_blocks  # blocks without a holder
        self._idle_named = 0

    # ------------------------------------------------------------------ queries

    @property
    def num_free(self) -> int:
        """Blocks an allocation may take: idle-blank ones plus idle-named ones it would evict."""
        return self._idle

    @property
    def num_cached(self) -> int:
        """Idle blocks the prefix cache still names."""
        return self._idle_named

    def blocks_for(self, num_tokens: int) -> int:
        return -(-int(num_tokens) // self.block_size)

    def is_cached_unheld(self, block: int) -> bool:
        return self._holders[block] == 0 and self._named(block)

    # ------------------------------------------------------------------ transitions

    def allocate(self, n: int) -> list[int]:
        """`n` blocks, each with one holder: idle-blank blocks first, then evictions of idle-named ones."""
        if n > self._idle:
            raise RuntimeError(f"cannot allocate {n} KV blocks: only {self._idle} are free or evictable")
        out = []
        while len(out) < n:
            tier, ticket, b = heapq.heappop(self._heap)
            if self._ticket[b] != ticket:
                continue  # voided when the block was re-acquired, or superseded
            self._ticket[b] = -1
            if tier == NAMED:
                self._idle_named -= 1
                if self._named(b):
                    self.prefix.forget(b)
            self._holders[b] = 1
            self._idle -= 1
            out.append(b)
        return out

    def acquire(self, blocks: list[int]) -> None:
        """One more holder for each block (prefix-cache hits); an idle block leaves the reclaim heap."""
        for b in blocks:
            if self._holders[b] == 0:
                self._idle -= 1
                if self._named(b):
                    self._idle_named -= 1
                self._ticket[b] = -1
            self._holders[b] += 1
        if len(self._heap) > 2 * self.num_blocks + 64:  # stale entries of revived blocks: compact
            self._heap = [(tier, t, b) for t, (tier, b) in self._live()]
            heapq.heapify(self._heap)

    def free(self, blocks: list[int]) -> None:
        """Drops one holder of every block of a table, tail first; empties the list."""
        while blocks:
            b = blocks.pop()
            self._holders[b] -= 1
            if self._holders[b] == 0:
                self._park(b, NAMED if self._named(b) else BLANK)

    def clear_cache(self) -> None:
        """Every idle-named block becomes blank (its name dropped), in eviction order."""
        named = sorted((t, b) for t, (tier, b) in self._live() if tier == NAMED)
        for _, b in named:
            self.prefix.forget(b)
            self._idle_named -= 1
            self._idle -= 1  # _park counts it again
            self._park(b, BLANK)

    def check(self, tables: list[list[int]]) -> None:
        """Raises AssertionError unless every block's holder count equals the number of tables listing it
        and every block is in exactly one state (held, idle-blank, idle-named)."""
        held = Counter(b for t in tables for b in t)
        want = np.zeros(self.num_blocks, dtype=np.int64)
        if held:
            idx = np.fromiter(held.keys(), dtype=np.int64, count=len(held))
            want[idx] = np.fromiter(held.values(), dtype=np.int64, count=len(held))
        wrong = np.flatnonzero(want != self._holders)
        if wrong.size:
            raise AssertionError(f"block refcounts disagree with the block tables at blocks {wrong[:10].tolist()}")
        live = self._live()
        idle = [b for _, (_, b) in live]
        no_holder = np.flatnonzero(self._holders == 0).tolist()
        named = sum(1 for _, (tier, _) in live if tier == NAMED)
        if sorted(idle) != no_holder or len(idle) != self._idle or named != self._idle_named:
            raise AssertionError(f"idle-block bookkeeping is inconsistent: {len(idle)} parked, {len(no_holder)} "
                                 f"without a holder, counter {self._idle}; {named} named vs {self._idle_named}")

    # ------------------------------------------------------------------ internals

    def _named(self, block: int) -> bool:
        return self.prefix is not None and self.prefix.is_cached(block)

    def _park(self, b: int, tier: int) -> None:
        t = self._next_ticket
        self._next_ticket += 1
        self._ticket[b] = t
        heapq.heappush(self._heap, (tier, t, b))
        self._idle += 1
        if tier == NAMED:
            self._idle_named += 1

    def _live(self) -> list[tuple[int, tuple[int, int]]]:
        """(ticket, (tier, block)) of every live heap entry."""
        return [(t, (tier, b)) for tier, t, b in self._heap if self._ticket[b] == t]
