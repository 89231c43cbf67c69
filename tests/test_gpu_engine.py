"""End-to-end on the GPU: the engine (scheduler, block manager, paged pool, Llama model) with the HIP
hot path against the same engine with the oracle's metadata build and attention (float32), on the same
weights and requests.  Small Llama shapes with head_dim 128 (the kernels' head size)."""

import random

import pytest
import torch

from oracle_engine import OracleBackend, oracle_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def tiny_model(seed=0, layers=2, heads=4, kv_heads=2, vocab=256, std=0.05, head_std=0.6, dtype=torch.float16):
    from minillm.model.config import LlamaConfig
    from minillm.model.llama import LlamaForCausalLM, random_init_

    cfg = LlamaConfig(vocab_size=vocab, hidden_size=heads * 128, intermediate_size=1024, num_hidden_layers=layers,
                      num_attention_heads=heads, num_key_value_heads=kv_heads, head_dim=128, rms_norm_eps=1e-5,
                      rope_theta=10000.0, max_position_embeddings=4096)
    model = LlamaForCausalLM(cfg).to(device=DEV, dtype=dtype)
    random_init_(model, std=std, seed=seed)
    with torch.no_grad():  # wider logits
        model.lm_head.weight.mul_(head_std / std)
    return model


def prompts(n, lo, hi, seed, vocab=256):
    rng = random.Random(seed)
    return [[rng.randrange(3, vocab) for _ in range(rng.randrange(lo, hi))] for _ in range(n)]


def run_engine(model, backend, builder, ps, max_tokens, **kw):
    """Runs the engine to completion; returns {req_id: [(token, top1 - top2 margin in logit ulps), ...]}.
    Tokens are the greedy argmax of each row's logits, picked by a sampler that also records the row's
    margin under its request id (rows and logits arrive together, also for steps replayed from graphs and
    for chunk rows that sample nothing)."""
    from minillm.engine.core import AddRequest, EngineCore

    margin = {}

    def greedy(reqs, logits):
        top2 = logits.float().topk(2, dim=-1).values
        # the margin in units of the logits' own rounding step at the top logit
        ulp = torch.finfo(logits.dtype).eps * top2[:, 0].abs().clamp_min(1.0)
        for r, m in zip(reqs, ((top2[:, 0] - top2[:, 1]) / ulp).tolist()):
            margin[r.req_id] = m
        return logits.argmax(dim=-1).tolist()

    model.set_backend(backend)
    core = EngineCore(model, metadata_builder=builder, sampler=greedy, **kw)
    for i, p in enumerate(ps):
        core.add_request(AddRequest(f"r{i}", p, max_tokens))
    outs = {}
    while core.has_work():
        for o in core.step().outputs:
            outs.setdefault(o.req_id, []).extend((t, margin[o.req_id]) for t in o.new_token_ids)
        core.check_blocks()
    return outs, core


NEAR_TIE = 8  # ulps of the logits' dtype at the top logit: a choice this close may flip between kernels


def assert_greedy_match(got, exp):
    """Tokens identical; a divergence is accepted only at a near-tie of the oracle's logits (after
    which the two continuations are different sequences and are not compared)."""
    compared = 0
    for rid, ref in exp.items():
        mine = got[rid]
        assert len(mine) == len(ref), rid
        for (t1, _), (t2, margin) in zip(mine, ref):
            if t1 != t2:
                assert margin < NEAR_TIE, f"{rid}: token {t1} != {t2} at a clear margin of {margin:.1f} ulps"
                break
            compared += 1
    total = sum(len(v) for v in exp.values())
    # every divergence is already checked to be a near-tie; this only guards against a run that
    # diverges everywhere at once
    assert compared >= 0.5 * total, f"only {compared} of {total} tokens compared before divergences"


def test_engine_greedy_tokens_match_oracle(hip):
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model()
    ps = prompts(12, 1, 300, seed=1)
    kw = dict(max_batch_size=8, num_kv_blocks=400, max_model_len=4096)
    got, core = run_engine(model, get_backend("hip"), None, ps, 24, **kw)  # resident block tables
    exp, _ = run_engine(model, OracleBackend(), oracle_metadata, ps, 24, **kw)
    assert_greedy_match(got, exp)
    assert core.stats().num_running == 0 and core.tables is not None
    csr, _ = run_engine(model, get_backend("hip"), AttentionMetadata.build, ps, 24, **kw)  # tables uploaded whole
    assert csr == got


def test_engine_with_preemption_and_prefix_sharing(hip):
    # a small pool forces preemption and recompute; shared prompt heads hit the prefix cache
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=3)
    head = prompts(1, 48, 49, seed=5)[0]
    ps = [head + p for p in prompts(6, 5, 40, seed=6)]
    kw = dict(max_batch_size=6, num_kv_blocks=24, max_model_len=4096)
    got, core = run_engine(model, get_backend("hip"), None, ps, 40, **kw)
    exp, _ = run_engine(model, OracleBackend(), oracle_metadata, ps, 40, **kw)
    assert_greedy_match(got, exp)
    st = core.stats()
    assert st.num_preemptions > 0 and st.prefix_cache_hits > 0


def test_teacher_forced_logits_close(hip):
    # the same ragged steps through both hot paths: half of every prompt, the rest on top of the cached
    # half (multi-token rows over a cached prefix), then six decode steps feeding fixed tokens
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata, SeqStep
    from minillm.cache.paged import PagedKVCache

    model = tiny_model(seed=7, layers=3, vocab=512, dtype=torch.bfloat16)
    seqs = [s + [5] * 6 for s in prompts(6, 20, 400, seed=8, vocab=512)]
    lens = [len(s) - 6 for s in seqs]
    perm = torch.randperm(400, generator=torch.Generator().manual_seed(9)).tolist()
    blocks = [perm[i * 40:(i + 1) * 40] for i in range(len(seqs))]
    schedule = [[(0, n // 2) for n in lens], [(n // 2, n) for n in lens]]
    schedule += [[(n + j, n + j + 1) for n in lens] for j in range(6)]

    def logits(backend, builder):
        model.set_backend(backend)
        cache = PagedKVCache(model.config, 400, DEV, torch.bfloat16)
        out = []
        for step in schedule:
            meta = builder([SeqStep(c, u - c, b) for (c, u), b in zip(step, blocks)], 16, DEV)
            ids = torch.tensor([[t for s, (c, u) in zip(seqs, step) for t in s[c:u]]], device=DEV)
            with torch.inference_mode():
                out.append(model(ids, kv_cache=cache.step(meta), last_index=meta.logits_index)[:, 0].float().cpu())
        return out

    a = logits(get_backend("hip"), AttentionMetadata.build)
    b = logits(OracleBackend(), oracle_metadata)
    for x, y in zip(a, b):
        assert (x - y).abs().max().item() <= 0.03 * y.abs().max().item() + 0.1
        top2 = y.topk(2, dim=-1).values
        clear = (top2[:, 0] - top2[:, 1]) > 0.5
        assert bool(((x.argmax(-1) == y.argmax(-1)) | ~clear).all())


def test_engine_fused_rotary_is_bit_identical(hip):
    # RoPE folded into the KV-append launch changes no bit of the engine's logits or tokens
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=11, dtype=torch.bfloat16)
    ps = prompts(8, 1, 200, seed=12)
    kw = dict(max_batch_size=8, num_kv_blocks=300, max_model_len=4096)
    fused, unfused = get_backend("hip"), get_backend("hip")
    unfused.fuse_rotary = False
    assert fused.fuse_rotary
    a, _ = run_engine(model, fused, AttentionMetadata.build, ps, 16, **kw)
    b, _ = run_engine(model, unfused, AttentionMetadata.build, ps, 16, **kw)
    assert a == b  # tokens and logit margins alike


def test_chunked_prefill_engine_matches_oracle(hip):
    # mixed steps: prompts cut into chunks under a 96-token budget, decode rows in the same launches
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=13)
    ps = prompts(10, 1, 400, seed=14)
    got, core = run_engine(model, get_backend("hip"), None, ps, 20, max_batch_size=8,
                           num_kv_blocks=400, max_model_len=4096, chunked_prefill=True, max_num_batched_tokens=96,
                           step_log=True)
    exp, _ = run_engine(model, OracleBackend(), oracle_metadata, ps, 20, max_batch_size=8, num_kv_blocks=400,
                        max_model_len=4096)
    assert_greedy_match(got, exp)
    mixed = [r for r in core.step_log if r.prefill_tokens and r.decode_tokens]
    assert mixed and max(r.prefill_tokens + r.decode_tokens for r in core.step_log) <= 96


def test_fp8_pool_engine_matches_oracle(hip):
    # an fp8 (e4m3fn) pool with per-tensor scales, fused RoPE + quantizing append, fp8 decode and prefill,
    # with preemption and prefix sharing, against the oracle engine on an fp8 pool of the same format
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata

    model = tiny_model(seed=21)
    head = prompts(1, 40, 41, seed=22)[0]
    ps = [head + p for p in prompts(8, 1, 300, seed=23)]
    kw = dict(max_batch_size=6, num_kv_blocks=64, max_model_len=4096, kv_cache_dtype=torch.float8_e4m3fn,
              kv_scales=(0.5, 0.25))
    got, core = run_engine(model, get_backend("hip"), None, ps, 24, **kw)
    exp, _ = run_engine(model, OracleBackend(), oracle_metadata, ps, 24, **kw)
    assert_greedy_match(got, exp)
    assert core.cache.k[0].dtype == torch.float8_e4m3fn
    st = core.stats()
    assert st.num_preemptions > 0 and st.prefix_cache_hits > 0


def test_prefix_cache_changes_no_token(hip):
    # reference tests/test_prefix_cache.py:112-209: shared prompt heads served from cached pages give the
    # tokens of a run without the cache, also when a small pool evicts cached blocks LRU
    from minillm.attention import get_backend

    model = tiny_model(seed=51)
    heads = prompts(3, 48, 49, seed=52)
    ps = [heads[i % 3] + p for i, p in enumerate(prompts(9, 1, 60, seed=53))]
    kw = dict(max_batch_size=3, max_model_len=4096)
    off, _ = run_engine(model, get_backend("hip"), None, ps, 16, num_kv_blocks=300, enable_prefix_caching=False, **kw)
    on, core = run_engine(model, get_backend("hip"), None, ps, 16, num_kv_blocks=300, **kw)
    tight, core_t = run_engine(model, get_backend("hip"), None, ps, 16, num_kv_blocks=18, **kw)
    assert_greedy_match(on, off)
    assert_greedy_match(tight, off)
    assert core.stats().prefix_cache_hits > 0 and core_t.stats().prefix_cache_hits > 0


def _pick(row):
    """Greedy token of a logits row and its top-1 - top-2 margin in ulps of the row's dtype (as run_engine)."""
    top2 = row.float().topk(2).values
    ulp = torch.finfo(row.dtype).eps * top2[0].abs().clamp_min(1.0)
    return int(row.argmax()), float((top2[0] - top2[1]) / ulp)


@torch.no_grad()
def _run_paged(model, backend, ps, steps, chunk_first=None, num_blocks=64):
    """The reference's hand-driven ragged run (tests/test_paged.py:99-136) on the GPU: one ragged step for
    every sequence each time, blocks scattered at random and the pool filled with 1e4 beforehand, so reading
    any slot a sequence does not own changes its logits; `chunk_first` prefills that many tokens of every
    prompt first, then the rest on top of them.  Returns per sequence [(token, margin)]."""
    from minillm.attention.metadata import AttentionMetadata, SeqStep
    from minillm.cache.paged import PagedKVCache

    bs = 16
    model.set_backend(backend)
    cache = PagedKVCache(model.config, num_blocks, DEV, next(model.parameters()).dtype)
    for buf in cache.k + cache.v:
        buf.fill_(1e4)
    free = list(range(num_blocks))
    random.Random(2).shuffle(free)
    tokens, blocks, cached = [list(p) for p in ps], [[] for _ in ps], [0] * len(ps)
    gen = [[] for _ in ps]
    while min(len(g) for g in gen) < steps:
        upto = [len(t) for t in tokens]
        if chunk_first and not any(cached):
            upto = [min(chunk_first, len(t)) for t in tokens]
        for i, b in enumerate(blocks):
            while len(b) * bs < upto[i]:
                b.append(free.pop())
        meta = AttentionMetadata.build([SeqStep(cached[i], upto[i] - cached[i], blocks[i]) for i in range(len(ps))],
                                       bs, DEV)
        ids = torch.tensor([[t for i, tok in enumerate(tokens) for t in tok[cached[i]:upto[i]]]], device=DEV)
        logits = model(ids, kv_cache=cache.step(meta), last_index=meta.logits_index)
        assert torch.isfinite(logits).all()
        for i in range(len(ps)):
            if upto[i] < len(tokens[i]):  # mid-prompt chunk: nothing sampled yet
                cached[i] = upto[i]
                continue
            cached[i] = len(tokens[i])
            tok, margin = _pick(logits[i, -1])
            tokens[i].append(tok)
            gen[i].append((tok, margin))
    return gen


@torch.no_grad()
def _greedy_no_cache(model, backend, p, steps):
    """Batch-1 greedy generation that runs the model over the whole sequence every step (the reference's
    generate.py:12-36), here with the contiguous attention of `backend`.  Returns [(token, margin)]."""
    model.set_backend(backend)
    ids, out = list(p), []
    for _ in range(steps):
        tok, margin = _pick(model(torch.tensor([ids], device=DEV))[0, -1])
        ids.append(tok)
        out.append((tok, margin))
    return out


def _prompt(seed, n):
    return torch.randint(3, 256, (n,), generator=torch.Generator().manual_seed(seed)).tolist()


@pytest.mark.parametrize("chunk_first", [None, 13])
def test_ragged_paged_generation_matches_batch_1(hip, chunk_first):
    # reference tests/test_paged.py:139-151: ragged paged generation over a 1e4-filled pool equals batch-1
    # greedy generation, also when every prompt's first prefill is cut into a chunk and the rest on top;
    # here the HIP ragged path against batch-1 generation with the oracle's float32 attention (a
    # divergence is accepted only at a near-tie of the oracle's logits, as in the engine tests)
    from minillm.attention import get_backend

    model = tiny_model(seed=3)
    if chunk_first:
        ps, steps = [_prompt(5, 30), _prompt(6, 21)], 8
    else:
        ps, steps = [_prompt(1, 3), _prompt(2, 17), _prompt(3, 1), _prompt(4, 40)], 20  # 40 tokens: three blocks
    got = _run_paged(model, get_backend("hip"), ps, steps, chunk_first=chunk_first)
    exp = {f"s{i}": _greedy_no_cache(model, OracleBackend(), p, steps) for i, p in enumerate(ps)}
    assert_greedy_match({f"s{i}": g[:steps] for i, g in enumerate(got)}, exp)
