"""The attention-backend interface (reference src/minillm/attention/base.py:16-45).

- `prefill`: attention over contiguous k/v (no cache, contiguous caches, padded batches).
- `forward`: the engine's path: ragged new tokens, k/v in the paged pool, described by `AttentionMetadata`.
"""

from __future__ import annotations

from abc import ABC, abstractmethod

import torch


class AttentionBackend(ABC):
    name: str = "base"

    @abstractmethod
    def prefill(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                key_valid: torch.Tensor | None = None, **kwargs) -> torch.Tensor:
        """Causal attention of the new tokens over everything so far.

        q [B, H, Tq, Dh]; k, v [B, Hkv, Tk, Dh] with Tk >= Tq and H a multiple of Hkv.  Query i sits at
        position Tk - Tq + i and sees keys 0 .. Tk - Tq + i.  key_valid [B, Tk] (bool, optional) marks
        real keys; a query with no real key may see its own position.  Returns [B, H, Tq, Dh], scale
        1/sqrt(Dh).
        """

    @abstractmethod
    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor,
                v_cache: torch.Tensor, meta) -> torch.Tensor:
        """One layer of one engine step on paged KV.

        q [N, H, Dh], k, v [N, Hkv, Dh]: the step's new tokens, all sequences concatenated.  k_cache,
        v_cache [num_blocks, block_size, Hkv, Dh]: the layer's pool.  Writes k, v into the pool at
        `meta.slot_mapping`, then returns each new token's causal attention over its sequence's
        context, [N, H, Dh].
        """
