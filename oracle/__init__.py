"""CPU oracle for the paged-attention hot path.  TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of minillm's torch reference backend
(reference: src/minillm/attention/{metadata,paged_torch_ref,torch_ref}.py).  It is the checker
that the HIP library is compared against.  Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it; the product package (`minillm`) never does, and
nothing here is ever the thing measured or shipped.

Modules
- `metadata`  : integer metadata build (numpy), reference `attention/metadata.py:70-103`.
- `torch_ref` : `write_kv`, `gather`, `paged_attention`, `forward`, `prefill`
                (torch CPU ops, the same library routines the reference calls),
                reference `attention/paged_torch_ref.py:23-74`, `attention/torch_ref.py:20-48`.

Pinning (how each function is checked independently of its own formula; tests/test_oracle.py)
- metadata       : the reference's known-answer test (tests/test_paged.py:41-50, fixture
                   tests/golden/metadata_kat.json), hand-derived kernel fields for that input, and
                   per-token / per-page invariants on random inputs (slot decodes to its block and
                   offset, page lists are prefixes of the tables, last-page length in [1, bs]).
- write_kv/gather: the reference's round trip (tests/test_paged.py:53-60) and an untouched-slot check.
- paged_attention: float64 softmax(QK^T/sqrt(d) + bottom-right causal mask)V written with explicit
                   loops over heads (tests/test_attention.py:11-19 restated), paged == dense
                   (tests/test_paged.py:63-93), causality, and isolation from junk pool slots.
- prefill        : naive GQA for mha/gqa/mqa and the three row kinds (tests/test_attention.py:22-55),
                   plus the key_valid "own slot" rule on a hand-checked case.
No function of this package is "parity unpinned".
"""
