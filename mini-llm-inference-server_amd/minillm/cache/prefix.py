"""Prefix-cache index: full pool blocks named by a chained SHA-256 of their tokens
(reference src/minillm/cache/prefix.py:21-76; byte layout fixed by docs/decisions/08-block-hash-spec.md).

  root  = SHA-256("minillm-kv-v1" || 0x00 || canonical JSON of the salt keys)
  block = SHA-256(parent || the block's tokens as little-endian uint32)

Requests whose leading blocks hash alike share those blocks (the shared-prefix pages the prefill
kernel reads from many block tables).  Ownership and eviction order belong to the block manager.
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
    """Append hashes to `chain` until it names the first `num_blocks` full blocks of `tokens`."""
    while len(chain) < num_blocks:
        i = len(chain)
        parent = chain[-1] if chain else root
        chain.append(block_hash(parent, tokens[i * block_size:(i + 1) * block_size]))


class PrefixCache:
    def __init__(self) -> None:
        self._by_hash: dict[bytes, int] = {}
        self._by_block: dict[int, bytes] = {}
        self.queries = 0  # prompt tokens looked up
        self.hits = 0  # of those, tokens served from cached blocks

    def __len__(self) -> int:
        return len(self._by_hash)

    def lookup(self, hashes: list[bytes]) -> list[int]:
        """Blocks of the longest cached prefix of `hashes`."""
        found = []
        for h in hashes:
            b = self._by_hash.get(h)
            if b is None:
                break
            found.append(b)
        return found

    def insert(self, h: bytes, block: int) -> None:
        """Name a block that just filled; the first block to hold a prefix stays its cached copy."""
        if h in self._by_hash or block in self._by_block:
            return
        self._by_hash[h] = block
        self._by_block[block] = h

    def is_cached(self, block: int) -> bool:
        return block in self._by_block

    def forget(self, block: int) -> None:
        h = self._by_block.pop(block, None)
        if h is not None:
            del self._by_hash[h]

    def clear(self) -> None:
        self._by_hash.clear()
        self._by_block.clear()
