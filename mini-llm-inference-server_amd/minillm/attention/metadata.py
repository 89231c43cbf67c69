"""Per-step attention metadata for paged KV, built on the GPU.

Same dataclass, field names, dtypes and meanings as the reference
(src/minillm/attention/metadata.py:27-103):

    query_start_loc = [0, 1, 6]        # host list: seq 0's new tokens are [0, 1), seq 1's are [1, 6)
    seq_lens        = [4, 5]           # host list: context length per sequence, this step included
    positions       = [3, 0, 1, 2, 3, 4]                     # int64 [N]
    slot_mapping    = [b0*bs + 3, b1*bs + 0, ...]            # int64 [N], block * block_size + offset
    block_tables    = [[b0, 0], [b1, b2]]                    # int64 [S, W], padded with block 0
    logits_index    = [0, 5]                                 # int64 [S]
    qo_indptr, seq_lens_i32, block_tables_i32, kv_indptr, kv_indices, kv_last_page_len   # int32

`build` does only O(S) work on the host (the two host lists and the table-length check, which raises
ValueError like the reference, metadata.py:75-76).  The block tables go to the device as one packed
int32 upload and `mllm_build_metadata` expands them into every tensor field in two launches; the
result is bit-identical to the reference's host loops.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import chain

import numpy as np
import torch

from .. import _native


@dataclass
class SeqStep:
    """One sequence in a step: `num_cached` tokens already in the pool, `num_new` added now."""

    num_cached: int
    num_new: int
    block_ids: list[int]  # covers num_cached + num_new tokens


@dataclass
class AttentionMetadata:
    block_size: int
    query_start_loc: list[int]
    seq_lens: list[int]
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    block_tables: torch.Tensor
    logits_index: torch.Tensor
    qo_indptr: torch.Tensor
    seq_lens_i32: torch.Tensor
    block_tables_i32: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    kv_last_page_len: torch.Tensor

    @property
    def max_query_len(self) -> int:
        return max(self.num_new)

    @property
    def max_seq_len(self) -> int:
        return max(self.seq_lens)

    @property
    def num_seqs(self) -> int:
        return len(self.seq_lens)

    @property
    def num_new(self) -> list[int]:
        q = self.query_start_loc
        return [q[i + 1] - q[i] for i in range(len(q) - 1)]

    @classmethod
    def build(cls, seqs: list[SeqStep], block_size: int, device: torch.device | str) -> AttentionMetadata:
        if not seqs:
            raise ValueError("a step needs at least one sequence")
        bs = int(block_size)
        starts, lens = [0], []
        for s in seqs:
            end = s.num_cached + s.num_new
            if len(s.block_ids) * bs < end:
                raise ValueError(f"{len(s.block_ids)} blocks can't hold {end} tokens")
            starts.append(starts[-1] + s.num_new)
            lens.append(end)
        device = torch.device(device)
        if device.type != "cuda":
            raise RuntimeError(f"the HIP metadata build needs a GPU device, got {device}")
        n_seq = len(seqs)
        nblk = [len(s.block_ids) for s in seqs]
        width = max(nblk)
        n_ids = sum(nblk)
        n_tok = starts[-1]
        n_pages = sum(-(-n // bs) for n in lens)

        host = pack_steps(seqs, np.empty(3 * n_seq + 1 + n_ids, dtype=np.int32))
        packed = torch.from_numpy(host).to(device)
        meta = cls._arenas(bs, starts, lens, n_tok, width, n_pages, device)
        meta._launch_build(packed, width)
        meta._upload = packed  # keeps the input alive until the launches that read it have run
        return meta

    @classmethod
    def _arenas(cls, bs: int, starts: list[int], lens: list[int], n_tok: int, width: int, n_pages: int,
                device) -> AttentionMetadata:
        """The metadata object over two fresh device arenas (int64 and int32 fields), not yet filled."""
        n_seq = len(lens)
        i64 = torch.empty(2 * n_tok + n_seq * width + n_seq, dtype=torch.long, device=device)
        i32 = torch.empty(2 * (n_seq + 1) + 2 * n_seq + n_seq * width + n_pages, dtype=torch.int32, device=device)
        o = 0
        positions = i64[o:o + n_tok]; o += n_tok
        slots = i64[o:o + n_tok]; o += n_tok
        tables = i64[o:o + n_seq * width].view(n_seq, width); o += n_seq * width
        logits_index = i64[o:o + n_seq]
        o = 0
        qo_indptr = i32[o:o + n_seq + 1]; o += n_seq + 1
        seq_lens_i32 = i32[o:o + n_seq]; o += n_seq
        tables_i32 = i32[o:o + n_seq * width].view(n_seq, width); o += n_seq * width
        kv_indptr = i32[o:o + n_seq + 1]; o += n_seq + 1
        kv_indices = i32[o:o + n_pages]; o += n_pages
        last_len = i32[o:o + n_seq]
        return cls(block_size=bs, query_start_loc=starts, seq_lens=lens, positions=positions, slot_mapping=slots,
                   block_tables=tables, logits_index=logits_index, qo_indptr=qo_indptr, seq_lens_i32=seq_lens_i32,
                   block_tables_i32=tables_i32, kv_indptr=kv_indptr, kv_indices=kv_indices,
                   kv_last_page_len=last_len)

    def _launch_build(self, packed: torch.Tensor, width: int) -> None:
        """mllm_build_metadata from a packed device upload (see pack_steps) into this object's arenas."""
        n_seq = self.num_seqs
        base = packed.data_ptr()
        _native.lib().call(
            "mllm_build_metadata", base, base + 4 * n_seq, base + 8 * n_seq, base + 4 * (3 * n_seq + 1), n_seq,
            self.block_size, width, self.positions.data_ptr(), self.slot_mapping.data_ptr(),
            self.block_tables.data_ptr(), self.logits_index.data_ptr(), self.qo_indptr.data_ptr(),
            self.seq_lens_i32.data_ptr(), self.block_tables_i32.data_ptr(), self.kv_indptr.data_ptr(),
            self.kv_indices.data_ptr(), self.kv_last_page_len.data_ptr(), _native.stream_ptr(packed.device))


def pack_steps(seqs: list[SeqStep], out: np.ndarray) -> np.ndarray:
    """The packed int32 upload of a step: num_cached[S] | num_new[S] | table_indptr[S+1] | table_ids[...],
    written into the front of `out`."""
    n_seq = len(seqs)
    nblk = [len(s.block_ids) for s in seqs]
    n_ids = sum(nblk)
    out[:n_seq] = [s.num_cached for s in seqs]
    out[n_seq:2 * n_seq] = [s.num_new for s in seqs]
    out[2 * n_seq] = 0
    np.cumsum(nblk, out=out[2 * n_seq + 1:3 * n_seq + 1])
    out[3 * n_seq + 1:3 * n_seq + 1 + n_ids] = np.fromiter(chain.from_iterable(s.block_ids for s in seqs),
                                                          dtype=np.int32, count=n_ids)
    return out[:3 * n_seq + 1 + n_ids]


class StaticDecodeMetadata:
    """Metadata of a decode step of exactly `num_rows` rows (one new token each) in fixed device buffers,
    for HIP graph capture: the arenas, the packed upload buffer and its pinned host twin never move, so
    a captured `build()` reads whatever `load()` last put there.

    Rows past the step's own are padding: one cached-less token whose only block id is -1, so its slot is
    negative (the append skips it) and its page reads are clamped inside the pool.  The host lists hold
    the worst case (every row at `max_blocks` blocks), which is what a plan built from them must cover.
    The step's split-KV size is staged too (`meta.split_dev`, at least `meta.split_min` pages), so the
    captured plan splits each replayed step as an eager step of the same rows would."""

    SPLIT_MIN = 8  # the smallest split the host heuristic picks: the plan's capacities are sized for it

    def __init__(self, num_rows: int, max_blocks: int, block_size: int, device) -> None:
        self.num_rows, self.max_blocks, self.block_size = num_rows, max_blocks, block_size
        cap = 3 * num_rows + 1 + num_rows * max_blocks
        self.pinned = torch.empty(cap + 1, dtype=torch.int32, pin_memory=True)  # + the split size
        self.packed = torch.zeros(cap + 1, dtype=torch.int32, device=device)
        self.meta = AttentionMetadata._arenas(block_size, list(range(num_rows + 1)),
                                              [max_blocks * block_size] * num_rows, num_rows, max_blocks,
                                              num_rows * max_blocks, device)
        self.meta.split_dev = self.packed[cap:]
        self.meta.split_min = self.SPLIT_MIN
        self._cap = cap
        self._pad = SeqStep(0, 1, [-1])

    def load(self, seqs: list[SeqStep], pages_per_split: int = SPLIT_MIN) -> None:
        """Stages a decode step (len(seqs) <= num_rows) and its split size for the next build: host
        packing plus one non-blocking copy on the current stream."""
        if len(seqs) > self.num_rows:
            raise ValueError(f"{len(seqs)} rows do not fit a {self.num_rows}-row decode graph")
        bs = self.block_size
        for s in seqs:
            if s.num_new != 1:
                raise ValueError("a decode graph takes rows with one new token")
            end = s.num_cached + 1
            if len(s.block_ids) * bs < end:
                raise ValueError(f"{len(s.block_ids)} blocks can't hold {end} tokens")
            if -(-end // bs) > self.max_blocks:
                raise ValueError(f"a row of {end} tokens exceeds the graph's {self.max_blocks} blocks")
        rows = [SeqStep(s.num_cached, 1, s.block_ids[:-(-(s.num_cached + 1) // bs)]) for s in seqs]
        rows += [self._pad] * (self.num_rows - len(seqs))
        host = self.pinned.numpy()
        n = len(pack_steps(rows, host))
        host[self._cap] = max(self.SPLIT_MIN, min(128, int(pages_per_split)))
        self.packed[:n].copy_(self.pinned[:n], non_blocking=True)
        self.packed[self._cap:].copy_(self.pinned[self._cap:], non_blocking=True)

    def build(self) -> None:
        """mllm_build_metadata over the staged step (capturable: fixed pointers and launch shapes)."""
        self.meta._launch_build(self.packed, self.max_blocks)
