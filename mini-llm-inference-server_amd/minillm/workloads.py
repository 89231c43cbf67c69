"""Synthetic one-layer workloads of the paged hot path, with their algorithmic work.

Llama-3.1-8B head layout throughout (32 query heads, 8 KV heads, head_dim 128, 16-token blocks,
bf16).  Every tensor is drawn on the CPU from `torch.Generator().manual_seed(seed)` so any device (or
the CPU) sees identical bytes; page assignment is a seeded `randperm` of the pool.

- `decode_4`      4 rows with cached contexts 37/128/211/500 and one new token; a 128-page pool.
- `decode_256`    256 rows, cached context uniform in [128, 4096], one new token; pool = 2x the pages.
- `mixed_128`     8 prefill rows (new tokens lognormal, median 512, sigma 0.5, capped at 2048, on top of
                  0-1024 cached) + 120 decode rows (context uniform in [256, 8192]), seeded row order.
- `prefix_64`     64 rows sharing one 2048-token prefix (128 pages present in every block table) with
                  a private suffix of 64-512 new tokens each.
- `decode_uniform_<rows>x<pages>`  rows of exactly `pages` pages each (a load-balance bound for decode).

Work per layer (the denominators of the reported rates):
  bytes  B = sum_s L_s*Hkv*Dh*2*2 (context K+V, appended token included) + N*H*Dh*2*2 (q in, o out)
           + N*Hkv*Dh*2*2*2 (append: read k, v, write the pool) + 4*sum_s ceil(L_s/16) + 4*(3S+1)
  flops  F = sum_s 4*H*Dh*(n_s*c_s + n_s*(n_s+1)/2)   (causal, unmasked pairs only)
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

H, HKV, DH, BS = 32, 8, 128, 16


@dataclass
class Workload:
    name: str
    seqs: list[tuple[int, int, list[int]]]  # (num_cached, num_new, block_ids)
    num_blocks: int
    q: torch.Tensor  # [N, H, Dh]
    k: torch.Tensor  # [N, Hkv, Dh]
    v: torch.Tensor
    pool_k: torch.Tensor  # [num_blocks, BS, Hkv, Dh]
    pool_v: torch.Tensor
    h: int = H
    hkv: int = HKV
    dh: int = DH
    block_size: int = BS
    notes: dict = field(default_factory=dict)

    @property
    def num_tokens(self) -> int:
        return sum(n for _, n, _ in self.seqs)

    @property
    def lens(self) -> list[int]:
        return [c + n for c, n, _ in self.seqs]

    def kv_bytes(self, rows=None, kv_elem: int = 2) -> int:
        """Context K+V bytes of the given rows (all rows by default); kv_elem = pool bytes per element
        (2 for bf16 / fp16, 1 for fp8)."""
        rows = range(len(self.seqs)) if rows is None else rows
        return sum((self.seqs[i][0] + self.seqs[i][1]) * self.hkv * self.dh * kv_elem * 2 for i in rows)

    def algorithmic_bytes(self, kv_elem: int = 2) -> int:
        """Context K+V once, q in and o out (16-bit), the append's k/v read (16-bit) and pool write, page
        ids and per-row indices."""
        n, s = self.num_tokens, len(self.seqs)
        pages = sum(-(-length // self.block_size) for length in self.lens)
        return (self.kv_bytes(kv_elem=kv_elem) + n * self.h * self.dh * 2 * 2
                + n * self.hkv * self.dh * 2 * (2 + kv_elem) + 4 * pages + 4 * (3 * s + 1))

    def decode_kernel_bytes(self, kv_elem: int = 2) -> int:
        """Algorithmic bytes of the decode launch alone: its rows' context K+V, their q and o, page ids."""
        rows = [i for i, (_, n, _) in enumerate(self.seqs) if n == 1]
        pages = sum(-(-self.lens[i] // self.block_size) for i in rows)
        return (self.kv_bytes(rows, kv_elem) + len(rows) * self.h * self.dh * 2 * 2 + 4 * pages
                + 4 * (3 * len(rows) + 1))

    def prefill_flops(self) -> int:
        return sum(4 * self.h * self.dh * (n * c + n * (n + 1) // 2) for c, n, _ in self.seqs if n > 1)

    def flops(self) -> int:
        return sum(4 * self.h * self.dh * (n * c + n * (n + 1) // 2) for c, n, _ in self.seqs)


def _randn(g: torch.Generator, shape, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def _assign(g: torch.Generator, lens: list[int], pool: int) -> list[list[int]]:
    perm = torch.randperm(pool, generator=g).tolist()
    out, o = [], 0
    for length in lens:
        need = -(-length // BS)
        out.append(perm[o:o + need])
        o += need
    return out


def _finish(name, g, steps, tables, pool, notes=None, dtype=torch.bfloat16) -> Workload:
    n = sum(new for _, new in steps)
    pool_k = _randn(g, (pool, BS, HKV, DH), dtype)
    pool_v = _randn(g, (pool, BS, HKV, DH), dtype)
    q = _randn(g, (n, H, DH), dtype)
    k = _randn(g, (n, HKV, DH), dtype)
    v = _randn(g, (n, HKV, DH), dtype)
    seqs = [(c, new, t) for (c, new), t in zip(steps, tables)]
    return Workload(name, seqs, pool, q, k, v, pool_k, pool_v, notes=notes or {})


def decode_4(seed: int = 0, dtype=torch.bfloat16) -> Workload:
    g = torch.Generator().manual_seed(seed)
    cached = [37, 128, 211, 500]
    steps = [(c, 1) for c in cached]
    tables = _assign(g, [c + 1 for c in cached], 128)
    return _finish("decode_4", g, steps, tables, 128, dtype=dtype)


def decode_256(seed: int = 0, num_seqs: int = 256, dtype=torch.bfloat16) -> Workload:
    g = torch.Generator().manual_seed(seed)
    cached = torch.randint(128, 4097, (num_seqs,), generator=g).tolist()
    steps = [(c, 1) for c in cached]
    lens = [c + 1 for c in cached]
    pool = 2 * sum(-(-length // BS) for length in lens)
    tables = _assign(g, lens, pool)
    return _finish("decode_256", g, steps, tables, pool, dtype=dtype)


def mixed_128(seed: int = 0, sigma: float = 0.5, dtype=torch.bfloat16) -> Workload:
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(8, generator=g, dtype=torch.float64)
    n_pf = [min(2048, max(2, round(math.exp(math.log(512) + sigma * float(x))))) for x in z]
    c_pf = torch.randint(0, 1025, (8,), generator=g).tolist()
    c_dec = torch.randint(256, 8193, (120,), generator=g).tolist()
    steps = [(c, n) for c, n in zip(c_pf, n_pf)] + [(c, 1) for c in c_dec]
    order = torch.randperm(len(steps), generator=g).tolist()
    steps = [steps[i] for i in order]
    lens = [c + n for c, n in steps]
    pool = 2 * sum(-(-length // BS) for length in lens)
    tables = _assign(g, lens, pool)
    return _finish("mixed_128", g, steps, tables, pool, notes={"sigma": sigma}, dtype=dtype)


def prefix_64(seed: int = 0, dtype=torch.bfloat16) -> Workload:
    g = torch.Generator().manual_seed(seed)
    prefix_pages = 2048 // BS
    suffix = torch.randint(64, 513, (64,), generator=g).tolist()
    private = [-(-(2048 + n) // BS) - prefix_pages for n in suffix]
    pool = 2 * (prefix_pages + sum(private))
    perm = torch.randperm(pool, generator=g).tolist()
    shared, o = perm[:prefix_pages], prefix_pages
    tables = []
    for p in private:
        tables.append(shared + perm[o:o + p])
        o += p
    steps = [(2048, n) for n in suffix]
    return _finish("prefix_64", g, steps, tables, pool, notes={"shared_pages": prefix_pages}, dtype=dtype)


def decode_uniform(rows: int, pages: int, seed: int = 0, dtype=torch.bfloat16) -> Workload:
    """`rows` decode rows of exactly `pages` full pages each (the appended token fills the last one), pool
    and page assignment as decode_256's.  When the split size comes out at `pages` (or a divisor), every
    row and KV head is one equal item: a launch with no tail.  At 384 x 89 it holds decode_256's bytes
    within 0.3%, the load-balance bound of that workload."""
    g = torch.Generator().manual_seed(seed)
    steps = [(pages * BS - 1, 1)] * rows
    lens = [pages * BS] * rows
    pool = 2 * rows * pages
    return _finish(f"decode_uniform_{rows}x{pages}", g, steps, _assign(g, lens, pool), pool,
                   notes={"rows": rows, "pages": pages}, dtype=dtype)


WORKLOADS = {"decode_4": decode_4, "decode_256": decode_256, "mixed_128": mixed_128, "prefix_64": prefix_64}


def by_name(name: str) -> Workload:
    """A workload of WORKLOADS, or `decode_uniform_<rows>x<pages>`."""
    if name in WORKLOADS:
        return WORKLOADS[name]()
    if name.startswith("decode_uniform_"):
        rows, _, pages = name.removeprefix("decode_uniform_").partition("x")
        if rows.isdigit() and pages.isdigit() and int(rows) > 0 and int(pages) > 0:
            return decode_uniform(int(rows), int(pages))
    raise ValueError(f"unknown workload {name!r}: one of {sorted(WORKLOADS)} or decode_uniform_<rows>x<pages>")
