"""The decode part of the step plan (mllm_plan), restated in Python for the tests: decode rows' pages, rows
in sequence order, form one stream of T pages cut into nb = ceil(T / C) bins whose boundaries are
floor(b T / nb); a row's part inside a bin is a segment.  A row cut into several segments gets
consecutive partial slots and one merge item {seq, first slot, segments, 0}."""

import bisect


def restate(rows, pages_per_split):
    """rows: (seq, pages, kv_start, q_row, seq_len) of every decode row in sequence order.  Returns
    (bins, segments, merges, slots): bins[b] = [first segment, end segment]; a segment is the pair of
    records the kernel reads, ([first page in kv_indices, pages, first page within the row, row length],
    [q row, partial slot or -1, seq, 0])."""
    total = sum(r[1] for r in rows)
    if total == 0:
        return [], [], [], 0
    nb = -(-total // pages_per_split)
    bound = [b * total // nb for b in range(nb + 1)]
    bins, segs, merges, slot, off = [[None, None] for _ in range(nb)], [], [], 0, 0
    for seq, pg, kv0, qrow, length in rows:
        first, last = bisect.bisect_right(bound, off) - 1, bisect.bisect_right(bound, off + pg - 1) - 1
        parts = [(b, max(off, bound[b]), min(off + pg, bound[b + 1])) for b in range(first, last + 1)]
        cut = len(parts) > 1
        if cut:
            merges.append([seq, slot, len(parts), 0])
        for j, (b, lo, hi) in enumerate(parts):
            g = len(segs)
            if bins[b][0] is None:
                bins[b][0] = g
            bins[b][1] = g + 1
            segs.append(([kv0 + lo - off, hi - lo, lo - off, length], [qrow, slot + j if cut else -1, seq, 0]))
        slot += len(parts) if cut else 0
        off += pg
    return bins, segs, merges, slot
