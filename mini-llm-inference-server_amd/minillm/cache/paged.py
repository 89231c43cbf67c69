"""Paged KV pool (reference src/minillm/cache/paged.py:21-69).

Per layer, separate K and V tensors [num_blocks, block_size, Hkv, Dh] (NHD: token-major inside a
block), zero-initialised and allocated once; a block id names the same slot range in every layer.
Token p of a sequence lives at block_ids[p // block_size], offset p % block_size.  On an MI355X the
pool is sized from the 288 GB of HBM: one 16-token block of Llama-3.1-8B is 64 KB per layer, 2 MB
across its 32 layers.

A pool of dtype torch.float8_e4m3fn (the reference's planned fp8 KV cache, M9b in
docs/distributed_inference_plan.md:310) stores e4m3fn(x / scale) with one scale per tensor: `k_scale[l]`
and `v_scale[l]` for layer l, which the model passes to the backend with the layer's pools.  One block of
Llama-3.1-8B is then 32 KB per layer, so the same HBM holds twice the tokens.

`PagedStep` is the pool as one forward pass sees it: the pool plus that step's metadata.
"""

from __future__ import annotations

import torch

BLOCK_SIZE = 16


class PagedKVCache:
    def __init__(self, config, num_blocks: int, device: torch.device | str, dtype: torch.dtype,
                 block_size: int = BLOCK_SIZE, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        shape = (num_blocks, block_size, config.num_key_value_heads, config.head_dim)
        self.k = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(config.num_hidden_layers)]
        self.v = [torch.zeros(shape, device=device, dtype=dtype) for _ in range(config.num_hidden_layers)]
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.quantized = dtype == torch.float8_e4m3fn
        if not self.quantized and (k_scale != 1.0 or v_scale != 1.0):
            raise ValueError("k_scale / v_scale apply to fp8 pools only")
        self.k_scale = [float(k_scale)] * config.num_hidden_layers
        self.v_scale = [float(v_scale)] * config.num_hidden_layers

    def scales(self, layer: int) -> dict:
        """Keyword arguments of the backend call for `layer`: its scales for an fp8 pool, none otherwise."""
        return {"k_scale": self.k_scale[layer], "v_scale": self.v_scale[layer]} if self.quantized else {}

    @staticmethod
    def bytes_per_block(config, dtype: torch.dtype, block_size: int = BLOCK_SIZE) -> int:
        """K and V, every layer: 2 x layers x block_size x KV heads x head_dim x bytes per element."""
        elem = torch.tensor([], dtype=dtype).element_size()
        return 2 * config.num_hidden_layers * block_size * config.num_key_value_heads * config.head_dim * elem

    @classmethod
    def blocks_for_bytes(cls, config, dtype: torch.dtype, num_bytes: int, block_size: int = BLOCK_SIZE) -> int:
        return num_bytes // cls.bytes_per_block(config, dtype, block_size)

    def step(self, meta) -> PagedStep:
        return PagedStep(self, meta)


class PagedStep:
    """What a model's forward pass calls on its KV cache for one ragged step.  The backend's `forward`
    reads and writes the pool itself, so there is nothing to mark or advance."""

    ragged = True

    def __init__(self, cache: PagedKVCache, meta) -> None:
        self.cache, self.meta = cache, meta

    def positions(self, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None) -> torch.Tensor:
        return self.meta.positions[None, :]

    def mark(self, attention_mask: torch.Tensor | None, num_tokens: int) -> None:
        if attention_mask is not None:
            raise ValueError("a ragged step has no padding, so no attention mask")

    def key_valid(self, num_new: int) -> None:
        return None

    def advance(self, num_tokens: int) -> None:
        pass
