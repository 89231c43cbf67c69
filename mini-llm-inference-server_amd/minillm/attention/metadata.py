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

    def _launch_build_rows(self, packed: torch.Tensor, tables: DeviceBlockTables, width: int) -> None:
        """mllm_build_metadata_rows from num_cached | num_new | rows | num_blocks at the front of `packed`."""
        n_seq = self.num_seqs
        base = packed.data_ptr()
        _native.lib().call(
            "mllm_build_metadata_rows", base, base + 4 * n_seq, base + 8 * n_seq, base + 12 * n_seq,
            tables.tables.data_ptr(), tables.max_blocks, n_seq, self.block_size, width, self.positions.data_ptr(),
            self.slot_mapping.data_ptr(), self.block_tables.data_ptr(), self.logits_index.data_ptr(),
            self.qo_indptr.data_ptr(), self.seq_lens_i32.data_ptr(), self.block_tables_i32.data_ptr(),
            self.kv_indptr.data_ptr(), self.kv_indices.data_ptr(), self.kv_last_page_len.data_ptr(),
            _native.stream_ptr(packed.device))

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


class DeviceBlockTables:
    """A device-resident mirror of the block manager's tables: one row of `max_blocks` int32 block ids per
    request (keyed by any hashable, the engine's Request objects), so a step uploads only the ids each
    request gained since its last step instead of every table (the reference's build flattens and uploads
    all of them, metadata.py:82-83,101).  A request's list of block ids only grows while it runs; a new
    list object (re-admission after preemption) is uploaded whole.  Row `max_rows` is reserved for
    padding rows: its only block id is -1."""

    def __init__(self, max_rows: int, max_blocks: int, device) -> None:
        self.max_rows, self.max_blocks = int(max_rows), int(max_blocks)
        self.device = torch.device(device)
        self.pad_row = self.max_rows
        self.tables = torch.zeros((self.max_rows + 1) * self.max_blocks, dtype=torch.int32, device=self.device)
        self.tables[self.pad_row * self.max_blocks] = -1
        self._free = list(range(self.max_rows - 1, -1, -1))
        self._row: dict = {}
        self._synced: dict = {}  # key -> (the block-id list object, entries already on the device)

    def release(self, key) -> None:
        row = self._row.pop(key, None)
        if row is not None:
            self._free.append(row)
            self._synced.pop(key, None)

    def sync(self, keys, seqs: list[SeqStep]) -> tuple[list[int], list[int]]:
        """Rows of the step's sequences and the flat (index, id) updates that bring them up to date."""
        rows, updates = [], []
        for key, s in zip(keys, seqs):
            ids = s.block_ids
            if len(ids) > self.max_blocks:
                raise ValueError(f"{len(ids)} blocks exceed the resident table's {self.max_blocks} per row")
            row = self._row.get(key)
            if row is None:
                if not self._free:
                    raise ValueError(f"more than {self.max_rows} requests hold resident table rows")
                row = self._row[key] = self._free.pop()
            prev = self._synced.get(key)
            start = prev[1] if prev is not None and prev[0] is ids and prev[1] <= len(ids) else 0
            base = row * self.max_blocks
            for j in range(start, len(ids)):
                updates += (base + j, ids[j])
            self._synced[key] = (ids, len(ids))
            rows.append(row)
        return rows, updates

    def build(self, keys, seqs: list[SeqStep], block_size: int) -> AttentionMetadata:
        """AttentionMetadata of a step (same fields, bit-identical) from the resident tables: one upload of
        num_cached | num_new | rows | num_blocks | updates, a table update and the two build launches."""
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
        rows, updates = self.sync(keys, seqs)
        n_seq = len(seqs)
        nblk = [len(s.block_ids) for s in seqs]
        host = np.empty(4 * n_seq + len(updates), dtype=np.int32)
        host[:n_seq] = [s.num_cached for s in seqs]
        host[n_seq:2 * n_seq] = [s.num_new for s in seqs]
        host[2 * n_seq:3 * n_seq] = rows
        host[3 * n_seq:4 * n_seq] = nblk
        host[4 * n_seq:] = updates
        packed = torch.from_numpy(host).to(self.device)
        width = max(nblk)
        meta = AttentionMetadata._arenas(bs, starts, lens, starts[-1], width, sum(-(-n // bs) for n in lens),
                                         self.device)
        self.apply(packed, 4 * n_seq, len(updates) // 2)
        meta._launch_build_rows(packed, self, width)
        meta._upload = packed
        return meta

    def apply(self, packed: torch.Tensor, offset: int, num_updates: int) -> None:
        """mllm_update_block_tables from `num_updates` (index, id) pairs at int32 offset `offset` of `packed`."""
        if num_updates:
            _native.lib().call("mllm_update_block_tables", self.tables.data_ptr(), self.tables.numel(),
                               packed.data_ptr() + 4 * offset, num_updates, _native.stream_ptr(self.device))


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


def decode_plan_size(decode_pages: int, decode_rows: int, pages_per_split: int) -> tuple[int, int]:
    """int4 records and merge items that hold a step's decode plan (mllm_plan): a header, one record per bin
    and two per segment, with bins = ceil(pages / pages_per_split).  A row is cut only where a bin boundary
    falls inside it, so segments <= bins + rows - 1 and cut rows <= min(rows, bins - 1)."""
    if decode_rows <= 0 or decode_pages <= 0:
        return 0, 0
    bins = -(-decode_pages // pages_per_split)
    return 1 + bins + 2 * (bins + decode_rows - 1), min(decode_rows, bins - 1)


class StaticDecodeMetadata:
    """Metadata of a decode step of exactly `num_rows` rows (one new token each) in fixed device buffers,
    for HIP graph capture: the arenas, the upload buffer and its pinned host twin never move, and the
    block ids come from a DeviceBlockTables mirror, so a captured `build()` reads whatever `load()` last
    staged.

    Rows past the step's own are padding: a cached-less token on the mirror's pad row (block id -1), so its
    slot is negative (the append skips it) and its page reads are clamped inside the pool.  The host lists
    hold the worst case (every row at the mirror's `max_blocks` blocks), which is what a plan built from
    them must cover.  The step's split-KV size is staged too (`meta.split_dev`, at least `meta.split_min`
    pages), so the captured plan splits each replayed step as an eager step of the same rows would."""

    SPLIT_MIN = 2  # the smallest split the host heuristic picks (hip_backend.MIN_SPLIT_PAGES)

    def __init__(self, num_rows: int, tables: DeviceBlockTables, block_size: int,
                 decode_records: int | None = None) -> None:
        """`decode_records` caps the plan's decode records (default: every row at `max_blocks` blocks in
        bins of SPLIT_MIN pages); a step whose plan at its staged bin size needs more must not be staged
        (DecodeGraphs.fits checks that on the host)."""
        self.num_rows, self.tables, self.block_size = num_rows, tables, block_size
        self.max_blocks = tables.max_blocks
        worst, _ = decode_plan_size(num_rows * self.max_blocks, num_rows, self.SPLIT_MIN)
        least, _ = decode_plan_size(num_rows, num_rows, self.SPLIT_MIN)  # every row one page
        self.decode_records = worst if decode_records is None else max(least, min(worst, int(decode_records)))
        dev = tables.device
        # num_cached | num_new | rows | num_blocks | split size | table updates (at most every entry of B rows)
        self._upd = 4 * num_rows + 1
        cap = self._upd + 2 * num_rows * self.max_blocks
        self.pinned = torch.empty(cap, dtype=torch.int32, pin_memory=True)
        self.packed = torch.zeros(cap, dtype=torch.int32, device=dev)
        # the last upload from `pinned`: the host waits for it before packing the next step into the same
        # pinned memory (the copy runs when the stream reaches it, which may be after the host moved on)
        self._uploaded = torch.cuda.Event()
        self.meta = AttentionMetadata._arenas(block_size, list(range(num_rows + 1)),
                                              [self.max_blocks * block_size] * num_rows, num_rows, self.max_blocks,
                                              num_rows * self.max_blocks, dev)
        self.meta.split_dev = self.packed[4 * num_rows:4 * num_rows + 1]
        self.meta.split_min = self.SPLIT_MIN
        self.meta.decode_records_cap = self.decode_records

    def split_size(self, pages_per_split: int) -> int:
        """The split size a staged step runs with (what mllm_plan_dev clamps it to)."""
        return max(self.SPLIT_MIN, min(192, int(pages_per_split)))

    def load(self, keys, seqs: list[SeqStep], pages_per_split: int = SPLIT_MIN) -> None:
        """Stages a decode step (len(seqs) <= num_rows) and its split size for the next build: host packing,
        one non-blocking copy and the mirror's update launch, on the current stream."""
        b = self.num_rows
        if len(seqs) > b:
            raise ValueError(f"{len(seqs)} rows do not fit a {b}-row decode graph")
        bs = self.block_size
        for s in seqs:
            if s.num_new != 1:
                raise ValueError("a decode graph takes rows with one new token")
            end = s.num_cached + 1
            if len(s.block_ids) * bs < end:
                raise ValueError(f"{len(s.block_ids)} blocks can't hold {end} tokens")
            if len(s.block_ids) > self.max_blocks:
                raise ValueError(f"a row of {len(s.block_ids)} blocks exceeds the graph's {self.max_blocks} blocks")
        rows, updates = self.tables.sync(keys, seqs)
        n, pad = len(seqs), b - len(seqs)
        self._uploaded.synchronize()  # no-op before the first upload
        host = self.pinned.numpy()
        host[:n] = [s.num_cached for s in seqs]
        host[n:b] = 0
        host[b:2 * b] = 1
        host[2 * b:2 * b + n] = rows
        host[2 * b + n:3 * b] = self.tables.pad_row
        host[3 * b:3 * b + n] = [len(s.block_ids) for s in seqs]
        host[3 * b + n:4 * b] = 1
        host[4 * b] = self.split_size(pages_per_split)
        u = len(updates)
        host[self._upd:self._upd + u] = updates
        end = self._upd + u
        self.packed[:end].copy_(self.pinned[:end], non_blocking=True)
        self._uploaded.record()
        self.tables.apply(self.packed, self._upd, u // 2)
        del pad

    def build(self) -> None:
        """mllm_build_metadata_rows over the staged step (capturable: fixed pointers and launch shapes)."""
        self.meta._launch_build_rows(self.packed, self.tables, self.max_blocks)
