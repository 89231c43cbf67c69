"""Prefix cache: full pool blocks named by a chained SHA-256 of their tokens, so requests with the same
leading tokens share those blocks' K/V (the shared-prefix pages the prefill kernel reads from many block
tables).

The names are a published byte format (reference docs/decisions/08-block-hash-spec.md; reference
src/minillm/cache/prefix.py:21-35), kept bit for bit:
  root  = SHA-256("minillm-kv-v1" || 0x00 || canonical JSON of the salt keys)
  block = SHA-256(parent || the block's tokens as little-endian uint32)

The index is this build's own: a dict from name to block id, and the reverse as a list indexed by block
id (block ids are dense, 0 .. pool size - 1).  The first block to carry a name keeps it; a second block
computed with the same contents at the same time stays private to its request.  Holders and eviction
order belong to the block manager, which drops a block's name when it reuses the block.
"""

from __future__ import annotations

import hashlib
import json
import struct

HASH_VERSION = "minillm-kv-v1"


def root_hash(extra_keys: dict) -> bytes:
    canonical = json.dumps(extra_keys, sort_keys=True, separators=(",", ":"), ensure_ascii=False)
    return hashlib.sha256(HASH_VERSION.encode() + b"\x00" + canonical.encode()).digest()


def block_hash(parent: bytes, tokens: list[int]) -> bytes:
    return hashlib.sha256(parent + struct.pack(f"<{len(tokens)}I", *tokens)).digest()


def extend_chain(chain: list[bytes], root: bytes, tokens: list[int], num_blocks: int, block_size: int) -> None:
    """Grows `chain` in place until it names the first `num_blocks` full blocks of `tokens`."""
    parent = chain[-1] if chain else root
    for i in range(len(chain), num_blocks):
        parent = block_hash(parent, tokens[i * block_size:(i + 1) * block_size])
        chain.append(parent)


class PrefixCache:
    def __init__(self) -> None:
        self._block_by_name: dict[bytes, int] = {}
        self._name_by_block: list[bytes | None] = []
        # token accounting the engine reports (hit rate = hits / queries)
        self.queries = 0  # prompt tokens looked up at admission
        self.hits = 0  # of those, tokens whose K/V came from named blocks

    def __len__(self) -> int:
        return len(self._block_by_name)

    def lookup(self, chain: list[bytes]) -> list[int]:
        """Blocks named by the longest leading run of `chain` that the index knows."""
        blocks: list[int] = []
        get = self._block_by_name.get
        for name in chain:
            b = get(name)
            if b is None:
                return blocks
            blocks.append(b)
        return blocks

    def insert(self, name: bytes, block: int) -> None:
        """Names a block that just filled, unless the name or the block is taken already."""
        if name in self._block_by_name or self.is_cached(block):
            return
        if block >= len(self._name_by_block):
            self._name_by_block.extend([None] * (block + 1 - len(self._name_by_block)))
        self._name_by_block[block] = name
        self._block_by_name[name] = block

    def is_cached(self, block: int) -> bool:
        return block < len(self._name_by_block) and self._name_by_block[block] is not None

    def forget(self, block: int) -> None:
        """Drops the block's name (it is about to hold other K/V)."""
        if self.is_cached(block):
            del self._block_by_name[self._name_by_block[block]]
            self._name_by_block[block] = None

    def clear(self) -> None:
        """Drops every name.  Only for a cache no block manager is using: a manager keeps counts of the idle
        blocks it parked as named (an engine clears through BlockManager.clear_cache, which drops the names
        of idle blocks only)."""
        self._block_by_name.clear()
        self._name_by_block.clear()
