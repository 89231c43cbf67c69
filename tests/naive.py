"""Textbook attention, written out with loops over heads in float64.

Independent of torch SDPA: softmax(q k^T / sqrt(d) + mask) v for each query head h, reading KV head
h // (H / Hkv) (reference tests/test_attention.py:11-19, `repeat_interleave` semantics).  The mask is
built from the definition of a ragged step: new token i of a row with `length` keys sits at position
length - n + i and sees keys 0 .. length - n + i.
"""

from __future__ import annotations

import math

import torch


def naive_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, allowed: torch.Tensor) -> torch.Tensor:
    """q [H, n, d], k/v [Hkv, L, d], allowed [n, L] bool -> [H, n, d] float64."""
    h_q, n, d = q.shape
    group = h_q // k.shape[0]
    out = torch.empty(h_q, n, d, dtype=torch.float64)
    for h in range(h_q):
        kv = h // group
        scores = q[h].double() @ k[kv].double().T / math.sqrt(d)
        scores = scores.masked_fill(~allowed, float("-inf"))
        p = torch.softmax(scores, dim=-1)
        out[h] = p @ v[kv].double()
    return out


def causal_allowed(n: int, length: int) -> torch.Tensor:
    """[n, length]: new token i (position length - n + i) may see key j iff j <= length - n + i."""
    i = torch.arange(n)[:, None]
    j = torch.arange(length)[None, :]
    return j <= (length - n + i)


def dense_context(pool: torch.Tensor, blocks: list[int], length: int) -> torch.Tensor:
    """A sequence's first `length` tokens read slot by slot from the pool: [Hkv, length, d]."""
    bs = pool.shape[1]
    rows = [pool[blocks[p // bs], p % bs] for p in range(length)]
    return torch.stack(rows, dim=0).transpose(0, 1)
