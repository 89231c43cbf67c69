"""Host-side callers of the hot path, on the CPU: block accounting, the scheduler's admission,
growth and preemption rules, and the prefix-cache hash (scenarios of the reference's
tests/test_paged.py:152-240 and tests/test_prefix_cache.py:33-93)."""

import hashlib
import struct

import pytest

from minillm.cache.prefix import PrefixCache, block_hash, extend_chain, root_hash
from minillm.engine.block_manager import BlockManager
from minillm.engine.scheduler import Request, Scheduler


def test_block_manager_accounting():
    bm = BlockManager(8, 16)
    assert bm.blocks_for(1) == 1 and bm.blocks_for(16) == 1 and bm.blocks_for(17) == 2
    a, b = bm.allocate(3), bm.allocate(5)
    assert bm.num_free == 0 and len(set(a + b)) == 8
    bm.check([a, b])
    with pytest.raises(RuntimeError, match="free"):
        bm.allocate(1)
    with pytest.raises(AssertionError):
        bm.check([a, b, a[:1]])
    bm.free(a)
    assert a == [] and bm.num_free == 3
    bm.check([b])


def req(rid, n_prompt, max_tokens=4):
    return Request(rid, list(range(3, 3 + n_prompt)), max_tokens, frozenset(), {})


def prefilled(r):
    r.num_cached = r.num_tokens
    r.output.append(9)


def test_admission_by_tokens_and_blocks():
    s = Scheduler(max_num_seqs=8, max_num_batched_tokens=40, blocks=BlockManager(4, 16))
    rs = [req("r0", 10), req("r1", 10), req("r2", 30), req("r3", 5)]
    for r in rs:
        s.add(r)
    out = s.schedule()
    assert [r.req_id for r in out.prefill] == ["r0", "r1"]
    out = s.schedule()
    assert [r.req_id for r in out.prefill] == ["r2"] and len(rs[2].block_ids) == 2
    out = s.schedule()
    assert out.prefill == [] and [r.req_id for r in out.decode] == ["r0", "r1", "r2"]


def test_admission_keeps_a_block_for_a_request_about_to_cross_a_boundary():
    s = Scheduler(max_num_seqs=8, max_num_batched_tokens=100, blocks=BlockManager(2, 16))
    full = req("full", 16)
    s.add(full)
    assert s.schedule().prefill == [full] and s.blocks.num_free == 1
    prefilled(full)
    s.add(req("next", 3))
    assert s.schedule().prefill == []


def test_head_request_is_admitted_over_budget():
    s = Scheduler(max_num_seqs=4, max_num_batched_tokens=8, blocks=BlockManager(10, 16))
    s.add(req("big", 20))
    s.add(req("small", 3))
    assert [r.req_id for r in s.schedule().prefill] == ["big"]
    assert [r.req_id for r in s.schedule().prefill] == ["small"]


def test_preemption_takes_the_newest_and_requeues_it_first():
    bm = BlockManager(3, 16)
    s = Scheduler(max_num_seqs=4, max_num_batched_tokens=100, blocks=bm)
    old, new = req("old", 16), req("new", 10)
    s.add(old)
    s.schedule()
    prefilled(old)
    s.add(new)
    s.add(req("late", 1))
    assert [r.req_id for r in s.schedule().prefill] == ["new"]
    prefilled(new)
    out = s.schedule()
    assert out.preempted == [] and len(old.block_ids) == 2 and bm.num_free == 0
    old.num_cached, new.num_cached = 32, 16
    out = s.schedule()
    assert out.preempted == [new] and [r.req_id for r in out.decode] == ["old"] and len(old.block_ids) == 3
    assert new.block_ids == [] and new.num_cached == 0 and new.num_preemptions == 1
    assert [r.req_id for r in s.waiting] == ["new", "late"]
    assert new.uncached() == new.prompt + new.output
    bm.check([r.block_ids for r in s.running])


def test_hash_spec_is_byte_exact():
    keys = {"model": "m@abc", "kv_dtype": "bfloat16", "layout": "NHD", "block_size": 16, "salt": ""}
    canonical = b'{"block_size":16,"kv_dtype":"bfloat16","layout":"NHD","model":"m@abc","salt":""}'
    root = hashlib.sha256(b"minillm-kv-v1\x00" + canonical).digest()
    assert root_hash(keys) == root
    toks = list(range(100, 116))
    assert block_hash(root, toks) == hashlib.sha256(root + struct.pack("<16I", *toks)).digest()
    chain = []
    extend_chain(chain, root, list(range(40)), 2, 16)
    assert chain[1] == hashlib.sha256(chain[0] + struct.pack("<16I", *range(16, 32))).digest()


def test_prefix_cache_refcounts_and_lru():
    pc = PrefixCache()
    bm = BlockManager(4, 16, pc)
    a, b = bm.allocate(2), bm.allocate(2)
    pc.insert(b"a0", a[0])
    pc.insert(b"b0", b[0])
    a_ids, b_ids = list(a), list(b)
    bm.free(a)
    bm.free(b)
    assert bm.num_free == 4 and bm.num_cached == 2
    shared = pc.lookup([b"b0"])
    bm.acquire(shared)
    bm.acquire(shared)
    bm.check([shared, shared])
    got = bm.allocate(3)  # two free blocks, then the least recently freed cached one (a0)
    assert a_ids[0] in got and pc.lookup([b"a0"]) == [] and pc.lookup([b"b0"]) == [b_ids[0]]
    bm.free(got)
    bm.free(list(shared))
    bm.free(shared)
    bm.check([])
    bm.clear_cache()
    assert bm.num_cached == 0 and len(pc) == 0 and bm.num_free == 4
