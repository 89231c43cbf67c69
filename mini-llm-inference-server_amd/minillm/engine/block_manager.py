"""Pool block accounting (reference src/minillm/engine/block_manager.py:21-96).

A block is free, held (refcount = number of block tables listing it) or cached (refcount 0 but named
in the prefix cache, evicted least-recently-used when nothing is free).  Tables come out as arbitrary
permutations of the pool after churn, which is what the kernels see through kv_indices.
"""

from __future__ import annotations

import math
from collections import Counter, OrderedDict, deque


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, prefix=None) -> None:
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.prefix = prefix
        self._free: deque[int] = deque(range(num_blocks))
        self._lru: OrderedDict[int, None] = OrderedDict()  # cached, unheld; oldest first
        self._refs = [0] * num_blocks

    @property
    def num_free(self) -> int:
        """Blocks available to allocate: free ones plus cached ones that would be evicted."""
        return len(self._free) + len(self._lru)

    @property
    def num_cached(self) -> int:
        return len(self._lru)

    def blocks_for(self, num_tokens: int) -> int:
        return math.ceil(num_tokens / self.block_size)

    def is_cached_unheld(self, block: int) -> bool:
        return block in self._lru

    def allocate(self, n: int) -> list[int]:
        if n > self.num_free:
            raise RuntimeError(f"asked for {n} blocks, {self.num_free} free")
        got = []
        for _ in range(n):
            if self._free:
                b = self._free.popleft()
            else:
                b, _ = self._lru.popitem(last=False)
                self.prefix.forget(b)
            self._refs[b] = 1
            got.append(b)
        return got

    def acquire(self, blocks: list[int]) -> None:
        """One more reference on each block (prefix-cache hits)."""
        for b in blocks:
            if self._refs[b] == 0:
                self._lru.pop(b)
            self._refs[b] += 1

    def free(self, blocks: list[int]) -> None:
        """Drop a reference on each block, last block first (so a row's tail is evicted before its
        head, whose hash the rest of the chain depends on); empties the list."""
        for b in reversed(blocks):
            self._refs[b] -= 1
            if self._refs[b] == 0:
                if self.prefix is not None and self.prefix.is_cached(b):
                    self._lru[b] = None
                else:
                    self._free.append(b)
        blocks.clear()

    def clear_cache(self) -> None:
        while self._lru:
            b, _ = self._lru.popitem(last=False)
            self.prefix.forget(b)
            self._free.append(b)

    def check(self, tables: list[list[int]]) -> None:
        """Every block in exactly one state; held refcounts equal the tables' occurrences."""
        owners = Counter(b for t in tables for b in t)
        bad = [b for b in range(self.num_blocks) if self._refs[b] != owners.get(b, 0)]
        if bad:
            raise AssertionError(f"refcounts don't match block tables for blocks {bad[:10]}")
        seen = list(owners) + list(self._free) + list(self._lru)
        if len(seen) != self.num_blocks or len(set(seen)) != self.num_blocks:
            raise AssertionError(f"block accounting broken: {len(owners)} held + {len(self._free)} free + "
                                 f"{len(self._lru)} cached vs {self.num_blocks}")
