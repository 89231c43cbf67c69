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


# ---------------------------------------------------------------- chunked prefill (mixed steps)


def test_mixed_step_packs_decodes_then_chunks_under_the_budget():
    s = Scheduler(max_num_seqs=8, max_num_batched_tokens=24, blocks=BlockManager(20, 16), chunked_prefill=True)
    a, b = req("a", 10), req("b", 40)
    s.add(a)
    s.add(b)
    out = s.schedule()  # a whole, then b's first 14 tokens
    assert out.decode == [] and out.rows() == [(a, 10), (b, 14)]
    prefilled(a)  # a sampled its first token
    b.num_cached += 14
    c = req("c", 5)
    s.add(c)
    out = s.schedule()  # a decodes, b continues with 23 of its remaining 26, c waits for budget
    assert out.rows() == [(a, 1), (b, 23)] and list(s.waiting) == [c]
    a.num_cached += 1
    a.output.append(9)
    b.num_cached += 23
    out = s.schedule()  # a decodes, b's last 3 tokens, c admitted whole
    assert out.rows() == [(a, 1), (b, 3), (c, 5)] and not s.waiting
    assert all(len(r.block_ids) * 16 >= r.num_cached + out.chunks[r] for r in (a, b, c))
    s.blocks.check([r.block_ids for r in s.running])


def test_mixed_admission_is_fcfs_and_keeps_the_boundary_reserve():
    s = Scheduler(max_num_seqs=8, max_num_batched_tokens=100, blocks=BlockManager(3, 16), chunked_prefill=True)
    full = req("full", 16)  # its first sampled token will need a second block
    s.add(full)
    assert s.schedule().rows() == [(full, 16)] and s.blocks.num_free == 2
    prefilled(full)
    s.add(req("two", 17))  # needs 2 blocks + the reserve for `full`: does not fit
    s.add(req("one", 3))  # fits, but FCFS does not skip `two`
    out = s.schedule()
    assert out.rows() == [(full, 1)] and [r.req_id for r in s.waiting] == ["two", "one"]
    assert len(full.block_ids) == 2 and s.blocks.num_free == 1


def test_mixed_preemption_of_a_request_inside_its_prompt():
    bm = BlockManager(5, 16)
    s = Scheduler(max_num_seqs=4, max_num_batched_tokens=20, blocks=bm, chunked_prefill=True)
    old, long_ = req("old", 16), req("long", 40)
    s.add(old)
    s.add(long_)
    out = s.schedule()  # old whole (16), long (3 blocks) gets 4 tokens; one block stays free for old
    assert out.rows() == [(old, 16), (long_, 4)] and bm.num_free == 1
    prefilled(old)
    long_.num_cached += 4
    out = s.schedule()  # old crosses a boundary and takes the last block; long continues
    assert out.preempted == [] and bm.num_free == 0 and out.rows() == [(old, 1), (long_, 19)]
    old.num_cached += 1
    old.output.append(9)
    long_.num_cached += 19
    old.num_cached = 32  # pretend old filled its second block: its next decode needs a sixth block
    old.output += [9] * 15
    out = s.schedule()  # no free block: the newest request (long, mid-prompt) is preempted
    assert out.preempted == [long_] and long_.num_cached == 0 and list(s.waiting) == [long_]
    assert out.rows() == [(old, 1)]
    bm.check([r.block_ids for r in s.running])


def test_chunked_engine_tokens_equal_unchunked_on_cpu():
    # the whole engine on the CPU in float32 with the oracle hot path: prompts split into chunks
    # across mixed steps give exactly the greedy tokens of whole-prompt prefill steps
    import torch

    from minillm.engine.core import AddRequest, EngineCore
    from minillm.model.config import LlamaConfig
    from minillm.model.llama import LlamaForCausalLM, random_init_
    from oracle_engine import OracleBackend, oracle_metadata

    cfg = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-5,
                      rope_theta=10000.0, max_position_embeddings=512)
    model = LlamaForCausalLM(cfg)
    random_init_(model, std=0.2, seed=0)
    model.set_backend(OracleBackend())
    gen = torch.Generator().manual_seed(1)
    prompts = [torch.randint(3, 97, (int(n),), generator=gen).tolist() for n in (5, 70, 33, 1, 120, 16)]

    def run(**kw):
        core = EngineCore(model, max_model_len=512, max_batch_size=4, num_kv_blocks=40, metadata_builder=oracle_metadata,
                          enable_prefix_caching=False, step_log=True, **kw)
        for i, p in enumerate(prompts):
            core.add_request(AddRequest(f"r{i}", p, 12, ignore_eos=True))
        outs = {}
        while core.has_work():
            for o in core.step().outputs:
                outs.setdefault(o.req_id, []).extend(o.new_token_ids)
            core.check_blocks()
        return outs, core

    whole, _ = run()
    chunked, core = run(chunked_prefill=True, max_num_batched_tokens=24)
    assert chunked == whole and all(len(v) == 12 for v in whole.values())
    mixed = [r for r in core.step_log if r.prefill_tokens and r.decode_tokens]
    assert mixed and max(r.prefill_tokens + r.decode_tokens for r in core.step_log) <= 24


def test_fp8_pool_engine_on_cpu():
    # the engine over an fp8 (e4m3fn) pool with per-tensor scales, oracle hot path on the CPU: it runs
    # end to end, chunked and whole-prompt prefill give the same tokens, the pool is one byte per
    # element, and the prefix-cache root is keyed by the pool format and its scales
    import torch

    from minillm.cache.paged import PagedKVCache
    from minillm.cache.prefix import root_hash
    from minillm.engine.core import AddRequest, EngineCore
    from minillm.model.config import LlamaConfig
    from minillm.model.llama import LlamaForCausalLM, random_init_
    from oracle_engine import OracleBackend, oracle_metadata

    cfg = LlamaConfig(vocab_size=97, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-5,
                      rope_theta=10000.0, max_position_embeddings=512)
    model = LlamaForCausalLM(cfg)
    random_init_(model, std=0.2, seed=0)
    model.set_backend(OracleBackend())
    gen = torch.Generator().manual_seed(2)
    prompts = [torch.randint(3, 97, (int(n),), generator=gen).tolist() for n in (9, 70, 1, 41)]
    fp8 = torch.float8_e4m3fn

    def run(**kw):
        core = EngineCore(model, max_model_len=512, max_batch_size=4, num_kv_blocks=40, metadata_builder=oracle_metadata,
                          step_log=True, kv_cache_dtype=fp8, kv_scales=(0.5, 0.25), **kw)
        for i, p in enumerate(prompts):
            core.add_request(AddRequest(f"r{i}", p, 10, ignore_eos=True))
        outs = {}
        while core.has_work():
            for o in core.step().outputs:
                outs.setdefault(o.req_id, []).extend(o.new_token_ids)
            core.check_blocks()
        return outs, core

    whole, core = run()
    chunked, _ = run(chunked_prefill=True, max_num_batched_tokens=16)
    assert chunked == whole and all(len(v) == 10 for v in whole.values())
    assert core.cache.k[0].dtype == fp8 and core.cache.scales(1) == {"k_scale": 0.5, "v_scale": 0.25}
    assert core.cache.k[0].view(torch.uint8).any()  # something was written
    assert PagedKVCache.bytes_per_block(cfg, fp8) * 2 == PagedKVCache.bytes_per_block(cfg, torch.float32) // 2
    keys = dict(core._salt_keys)
    assert keys["kv_dtype"] == "float8_e4m3fn" and keys["kv_scales"] == [0.5, 0.25]
    plain = {k: v for k, v in keys.items() if k != "kv_scales"} | {"kv_dtype": "bfloat16"}
    assert root_hash({**keys, "salt": ""}) != root_hash({**plain, "salt": ""})
    with pytest.raises(ValueError, match="fp8 pools only"):
        PagedKVCache(cfg, 4, "cpu", torch.bfloat16, k_scale=2.0)


class _ListModel:
    """The block manager's rules written out with plain lists: blank blocks in release order (initially
    0 .. n-1), named idle blocks in least-recently-released order, holder counts per block."""

    def __init__(self, n):
        self.blank, self.named_idle, self.holders, self.named = list(range(n)), [], [0] * n, set()

    def allocate(self, k):
        out = []
        for _ in range(k):
            if self.blank:
                b = self.blank.pop(0)
            else:
                b = self.named_idle.pop(0)
                self.named.discard(b)
            self.holders[b] = 1
            out.append(b)
        return out

    def acquire(self, blocks):
        for b in blocks:
            if self.holders[b] == 0:
                self.named_idle.remove(b)
            self.holders[b] += 1

    def free(self, table):
        for b in reversed(table):
            self.holders[b] -= 1
            if self.holders[b] == 0:
                (self.named_idle if b in self.named else self.blank).append(b)

    def clear(self):
        for b in self.named_idle:
            self.named.discard(b)
            self.blank.append(b)
        self.named_idle = []


@pytest.mark.parametrize("seed", range(6))
def test_block_manager_random_churn_matches_the_rules(seed):
    import random

    rng = random.Random(seed)
    n = rng.choice([8, 24, 64])
    pc = PrefixCache()
    bm, model = BlockManager(n, 16, pc), _ListModel(n)
    tables, ticket = [], 0
    for _ in range(600):
        op = rng.random()
        if op < 0.35:  # a new table
            k = rng.randint(1, 4)
            if k <= bm.num_free:
                got = bm.allocate(k)
                assert got == model.allocate(k)
                tables.append(got)
            else:
                with pytest.raises(RuntimeError):
                    bm.allocate(k)
        elif op < 0.6 and tables:  # a table released, tail first
            t = tables.pop(rng.randrange(len(tables)))
            model.free(list(t))
            bm.free(t)
            assert t == []
        elif op < 0.8 and tables:  # a held block filled and is named
            b = rng.choice(rng.choice(tables))
            ticket += 1
            pc.insert(ticket.to_bytes(8, "little"), b)
            model.named.add(b)
        elif op < 0.95:  # a prefix hit: named blocks (held or idle) shared by a new table
            cands = sorted(model.named)
            if cands:
                hit = rng.sample(cands, rng.randint(1, min(3, len(cands))))
                bm.acquire(hit)
                model.acquire(hit)
                tables.append(list(hit))
        else:
            bm.clear_cache()
            model.clear()
        assert bm.num_free == len(model.blank) + len(model.named_idle)
        assert bm.num_cached == len(model.named_idle)
        assert all(bm.is_cached_unheld(b) == (b in model.named_idle) for b in range(n))
        bm.check(tables)
    assert {b for b in range(n) if pc.is_cached(b)} == model.named
