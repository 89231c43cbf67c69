"""Oracle: the ragged paged-attention metadata, built on the CPU with numpy.  TEST INFRASTRUCTURE ONLY.

Restates reference `src/minillm/attention/metadata.py:70-103` (`AttentionMetadata.build`) for
`SeqStep(num_cached, num_new, block_ids)` inputs (reference `metadata.py:27-33`).  Fields, dtypes
and meanings are those of the reference (`metadata.py:36-51`):

  host lists : query_start_loc [S+1], seq_lens [S]
  int64      : positions [N], slot_mapping [N], block_tables [S, W] (right-padded with block 0),
               logits_index [S]
  int32      : qo_indptr [S+1], seq_lens_i32 [S], block_tables_i32 [S, W], kv_indptr [S+1],
               kv_indices [sum pages], kv_last_page_len [S]

The build is vectorised (one pass over tokens and one over pages), so configurations with tens of
thousands of tokens finish in milliseconds.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class OracleSeq:
    """One sequence of a step (reference `metadata.py:27-33`)."""

    num_cached: int
    num_new: int
    block_ids: list[int]


@dataclass
class OracleMetadata:
    block_size: int
    query_start_loc: list[int]
    seq_lens: list[int]
    positions: np.ndarray
    slot_mapping: np.ndarray
    block_tables: np.ndarray
    logits_index: np.ndarray
    qo_indptr: np.ndarray
    seq_lens_i32: np.ndarray
    block_tables_i32: np.ndarray
    kv_indptr: np.ndarray
    kv_indices: np.ndarray
    kv_last_page_len: np.ndarray
    extra: dict = field(default_factory=dict)

    @property
    def num_new(self) -> list[int]:
        q = self.query_start_loc
        return [q[i + 1] - q[i] for i in range(len(q) - 1)]

    @property
    def max_query_len(self) -> int:
        return max(self.num_new)

    @property
    def max_seq_len(self) -> int:
        return max(self.seq_lens)

    @property
    def num_seqs(self) -> int:
        return len(self.seq_lens)

    # the kernel-facing names as a dict, for comparisons
    TENSOR_FIELDS = ("positions", "slot_mapping", "block_tables", "logits_index", "qo_indptr",
                     "seq_lens_i32", "block_tables_i32", "kv_indptr", "kv_indices", "kv_last_page_len")


def build_metadata(seqs: list[OracleSeq], block_size: int) -> OracleMetadata:
    """Reference `AttentionMetadata.build` (`metadata.py:70-103`), vectorised.

    - `starts` is the exclusive scan of num_new (`:71,77`), `lens = num_cached + num_new` (`:74,78`).
    - For new token p of a sequence: position p, slot block_ids[p // bs] * bs + p % bs (`:79-81`).
    - A table shorter than ceil(len / bs) blocks raises ValueError "... blocks can't hold ... tokens" (`:75-76`).
    - block_tables pad every table with block 0 to the widest (`:82-83`).
    - pages = block_ids[:ceil(len / bs)] (`:84`); kv_indptr is their scan (`:85-87`), kv_indices their
      concatenation (`:101`), kv_last_page_len = len - (pages - 1) * bs (`:102`).
    - logits_index = starts[1:] - 1 (`:96`).
    """
    bs = int(block_size)
    s_count = len(seqs)
    cached = np.array([s.num_cached for s in seqs], dtype=np.int64)
    new = np.array([s.num_new for s in seqs], dtype=np.int64)
    nblk = np.array([len(s.block_ids) for s in seqs], dtype=np.int64)
    lens = cached + new
    for s, end, nb in zip(seqs, lens.tolist(), nblk.tolist()):
        if nb * bs < end:
            raise ValueError(f"{nb} blocks can't hold {end} tokens")
    starts = np.zeros(s_count + 1, dtype=np.int64)
    np.cumsum(new, out=starts[1:])
    n_tok = int(starts[-1])

    width = int(nblk.max()) if s_count else 0
    tables = np.zeros((s_count, width), dtype=np.int64)
    flat_ids = np.fromiter((b for s in seqs for b in s.block_ids), dtype=np.int64, count=int(nblk.sum()))
    tab_ptr = np.zeros(s_count + 1, dtype=np.int64)
    np.cumsum(nblk, out=tab_ptr[1:])
    row_of_id = np.repeat(np.arange(s_count), nblk)
    col_of_id = np.arange(flat_ids.size) - tab_ptr[row_of_id]
    tables[row_of_id, col_of_id] = flat_ids

    # per new token: its sequence, its position, its slot
    seq_of_tok = np.repeat(np.arange(s_count), new)
    positions = cached[seq_of_tok] + (np.arange(n_tok) - starts[seq_of_tok])
    blk = tables[seq_of_tok, positions // bs] if n_tok else np.zeros(0, dtype=np.int64)
    slots = blk * bs + positions % bs

    # pages in use and the CSR page list
    pages = -(-lens // bs)
    kv_indptr = np.zeros(s_count + 1, dtype=np.int64)
    np.cumsum(pages, out=kv_indptr[1:])
    seq_of_page = np.repeat(np.arange(s_count), pages)
    page_col = np.arange(int(kv_indptr[-1])) - kv_indptr[seq_of_page]
    kv_indices = tables[seq_of_page, page_col]
    last = lens - (pages - 1) * bs

    return OracleMetadata(
        block_size=bs,
        query_start_loc=starts.tolist(),
        seq_lens=lens.tolist(),
        positions=positions.astype(np.int64),
        slot_mapping=slots.astype(np.int64),
        block_tables=tables,
        logits_index=(starts[1:] - 1).astype(np.int64),
        qo_indptr=starts.astype(np.int32),
        seq_lens_i32=lens.astype(np.int32),
        block_tables_i32=tables.astype(np.int32),
        kv_indptr=kv_indptr.astype(np.int32),
        kv_indices=kv_indices.astype(np.int32),
        kv_last_page_len=last.astype(np.int32),
    )
