"""Decode steps as captured HIP graphs (DecodeGraphs): every replay equals the same step run eagerly, bit
for bit, with eager steps (prefills, other buckets) and synchronisations between replays; the engine
with graphs gives the eager engine's greedy tokens, on bf16 and fp8 pools, also when steps exceed a
bucket's plan capacity and run eagerly; and it gives the oracle engine's greedy tokens."""

import pytest
import torch

from test_gpu_engine import assert_greedy_match, prompts, run_engine, tiny_model

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _engine(model, **kw):
    from minillm.engine.core import EngineCore

    return EngineCore(model, max_batch_size=8, num_kv_blocks=200, max_model_len=2048, **kw)


def test_every_replay_equals_the_eager_step(hip):
    # after every replay the same step runs eagerly on the same staged inputs; prefill steps (eager) and
    # replays of other buckets come in between as the batch fills and drains
    from minillm.attention import get_backend
    from minillm.engine.core import AddRequest

    model = tiny_model(seed=31)
    model.set_backend(get_backend("hip"))
    core = _engine(model, decode_graphs=(2, 8))
    for i, (p, n) in enumerate(zip(prompts(5, 1, 200, seed=32), (4, 7, 9, 30, 40))):
        core.add_request(AddRequest(f"r{i}", p, n, ignore_eos=True))  # the batch drains from 5 rows to 1
    seen, buckets = 0, set()
    while core.has_work():
        core.step()
        if core.graphs.replays == seen:
            continue
        seen = core.graphs.replays
        c = core.graphs._captured[core.graphs.last_bucket]
        got_logits, got_tokens = c.logits.clone(), c.tokens.clone()
        ref_logits, ref_tokens = core.graphs.eager_reference()
        torch.cuda.synchronize()
        assert torch.equal(got_tokens, ref_tokens), core.graphs.last_bucket
        assert torch.equal(got_logits.view(torch.int16), ref_logits.view(torch.int16)), core.graphs.last_bucket
        buckets.add(core.graphs.last_bucket)
    assert seen >= 30 and buckets == {2, 8}


@pytest.mark.parametrize("kv", ["fp16", "fp8"])
def test_graph_engine_matches_eager_engine(hip, kv):
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=41)
    ps = prompts(11, 1, 300, seed=42)
    kw = dict(max_batch_size=8, num_kv_blocks=300, max_model_len=2048)
    if kv == "fp8":
        kw.update(kv_cache_dtype=torch.float8_e4m3fn, kv_scales=(0.5, 0.25))
    got, core = run_engine(model, get_backend("hip"), None, ps, 20, decode_graphs=True, **kw)
    exp, _ = run_engine(model, get_backend("hip"), AttentionMetadata.build, ps, 20, **kw)
    assert_greedy_match(got, exp)
    assert core.graphs.replays > 10 and len(core.graphs._captured) >= 2  # batch shrinks as requests finish


def test_host_running_ahead_of_the_gpu_changes_nothing(hip):
    # a sampler that returns its tokens without reading the GPU lets the host stage the next replay while
    # the GPU still works on earlier steps (held back here by a bounded spin kernel per step): the staged
    # inputs of a later step must not reach a step still queued
    from minillm.attention import get_backend
    from minillm.engine.core import AddRequest, EngineCore

    model = tiny_model(seed=61)
    model.set_backend(get_backend("hip"))
    ps = prompts(6, 1, 120, seed=62)

    def run(sampler):
        core = EngineCore(model, max_batch_size=8, num_kv_blocks=200, max_model_len=2048, decode_graphs=True,
                          sampler=sampler)
        for i, p in enumerate(ps):
            core.add_request(AddRequest(f"r{i}", p, 24, ignore_eos=True))
        out = {}
        while core.has_work():
            for o in core.step().outputs:
                out.setdefault(o.req_id, []).extend(o.new_token_ids)
        return out, core

    def keeper(store, tokens=None):
        def sample(reqs, logits):
            for r, row in zip(reqs, logits):
                store[(r.req_id, len(r.output))] = row.clone()
            if tokens is None:
                return logits.argmax(dim=-1).tolist()  # reads the GPU: host and GPU in step
            torch.cuda._sleep(20_000_000)
            return [tokens[r.req_id][len(r.output)] for r in reqs]  # never waits for the GPU
        return sample

    synced, ahead = {}, {}
    tokens, core = run(keeper(synced))
    forced, core2 = run(keeper(ahead, tokens))
    torch.cuda.synchronize()
    assert core.graphs.replays > 10 and core2.graphs.replays == core.graphs.replays
    assert forced == tokens and synced.keys() == ahead.keys()
    for key, row in synced.items():
        assert torch.equal(row.view(torch.int16), ahead[key].view(torch.int16)), key


def test_graph_rejects_what_it_cannot_hold(hip):
    from minillm.attention.metadata import DeviceBlockTables, SeqStep, StaticDecodeMetadata

    sm = StaticDecodeMetadata(4, DeviceBlockTables(8, 8, DEV), 16)
    with pytest.raises(ValueError, match="decode graph"):
        sm.load(list(range(5)), [SeqStep(0, 1, [1])] * 5)
    with pytest.raises(ValueError, match="one new token"):
        sm.load([0], [SeqStep(0, 2, [1])])
    with pytest.raises(ValueError, match="exceeds"):
        sm.load([0], [SeqStep(200, 1, list(range(13)))])


def test_graph_steps_beyond_the_plan_capacity_run_eagerly(hip):
    # a bucket's split-KV capacity is sized from the pool; rows sharing a long prompt head (prefix cache)
    # reference more pages than the pool holds, so those steps fall back to eager launches, while the
    # steps that fit still replay; tokens equal the eager engine's either way
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=61)
    head = prompts(1, 300, 301, seed=62)[0]
    ps = [head + p for p in prompts(8, 1, 12, seed=63)]
    kw = dict(max_batch_size=8, num_kv_blocks=40, max_model_len=2048)
    got, core = run_engine(model, get_backend("hip"), None, ps, 40, decode_graphs=True, **kw)
    exp, _ = run_engine(model, get_backend("hip"), AttentionMetadata.build, ps, 40, **kw)
    assert_greedy_match(got, exp)
    g = core.graphs
    assert g.eager_fallbacks > 0 and g.replays > 0
    assert g.capacity(8) < 8 * -(-core.tables.max_blocks // 8)  # sized from the pool, not max_model_len
    assert core.stats().prefix_cache_hits > 0


def test_graph_engine_matches_oracle_engine(hip):
    # decode steps replayed from graphs against the oracle engine (metadata and attention from the oracle,
    # float32), greedy; tests/test_gpu_engine_8b.py compares them teacher-forced at the 8B shape
    from oracle_engine import OracleBackend, oracle_metadata

    from minillm.attention import get_backend

    model = tiny_model(seed=71)
    ps = prompts(10, 1, 300, seed=72)
    kw = dict(max_batch_size=8, num_kv_blocks=300, max_model_len=2048)
    got, core = run_engine(model, get_backend("hip"), None, ps, 24, decode_graphs=True, **kw)
    exp, _ = run_engine(model, OracleBackend(), oracle_metadata, ps, 24, **kw)
    assert_greedy_match(got, exp)
    assert core.graphs.replays > 10
