"""GPU parity of the HIP paged path against the oracle, on identical seeded inputs.

- metadata: every tensor field bit-identical (value and dtype) to the oracle's build, plus host lists;
- KV append: the pool bit-identical to the oracle's write_kv;
- attention: within 2e-2 abs / 1e-2 rel of the oracle's gather + SDPA computed in float32;
- junk in pool slots a row does not own never changes a bit of the output.
The oracle runs on the same GPU in float32 (torch's bf16 batched matmul is not used).
"""

import json
import random
from pathlib import Path

import pytest
import torch

import decode_plan
from harness import ATOL, RTOL, bits, hip_step, oracle_step
from oracle.metadata import OracleSeq, build_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLDEN = Path(__file__).resolve().parent / "golden"


def _meta_fields_equal(meta, om):
    assert meta.query_start_loc == om.query_start_loc
    assert meta.seq_lens == om.seq_lens
    for name in om.TENSOR_FIELDS:
        got = getattr(meta, name)
        exp = torch.from_numpy(getattr(om, name))
        assert got.dtype == exp.dtype, name
        assert got.shape == exp.shape, name
        assert torch.equal(got.cpu(), exp), name


# ------------------------------------------------------------------ metadata


def test_metadata_known_answer(hip):
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    g = json.loads((GOLDEN / "metadata_kat.json").read_text())
    meta = AttentionMetadata.build([SeqStep(c, n, b) for c, n, b in g["seqs"]], g["block_size"], DEV)
    for name, exp in g["expected"].items():
        got = getattr(meta, name)
        got = got if isinstance(got, list) else got.cpu().tolist()
        assert got == exp, name
    for name, dt in g["dtypes"].items():
        assert str(getattr(meta, name).dtype) == f"torch.{dt}", name


@pytest.mark.parametrize("bs", [1, 4, 16, 32])
@pytest.mark.parametrize("seed", range(3))
def test_metadata_random_steps(hip, bs, seed):
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    rng = random.Random(seed)
    steps = []
    for _ in range(rng.randrange(1, 1500)):
        cached = rng.choice([0, rng.randrange(0, 3000)])
        new = rng.choice([1, 1, 1, rng.randrange(1, 300)])
        steps.append((cached, new, -(-(cached + new) // bs) + rng.randrange(0, 3)))
    total = sum(need for _, _, need in steps)
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).tolist()
    seqs, o = [], 0
    for cached, new, need in steps:
        seqs.append((cached, new, perm[o:o + need]))
        o += need
    meta = AttentionMetadata.build([SeqStep(*s) for s in seqs], bs, DEV)
    _meta_fields_equal(meta, build_metadata([OracleSeq(*s) for s in seqs], bs))


@pytest.mark.parametrize("bs", [4, 16])
def test_metadata_from_resident_tables(hip, bs):
    # the device mirror across 40 steps of a churning request set: tables grow by appends, some requests
    # leave (rows released and reused), some come back with a new list; every step's fields equal the
    # oracle's build from the full tables, bit for bit, and the KAT holds on a fresh mirror
    from minillm.attention.metadata import DeviceBlockTables, SeqStep

    g = json.loads((GOLDEN / "metadata_kat.json").read_text())
    kat = DeviceBlockTables(4, 8, DEV).build(["x", "y"], [SeqStep(c, n, b) for c, n, b in g["seqs"]],
                                             g["block_size"])
    for name, exp in g["expected"].items():
        got = getattr(kat, name)
        assert (got if isinstance(got, list) else got.cpu().tolist()) == exp, name

    rng = random.Random(bs)
    tables = DeviceBlockTables(64, 6000 // bs + 16, DEV)  # rows reach 1000 + 40 x 100 tokens at most
    live: dict[int, list] = {}  # key -> [num_cached, block_ids]
    next_block, next_key = 0, 0
    for step in range(40):
        for key in [k for k in live if rng.random() < 0.1]:  # finished, or preempted and requeued
            tables.release(key)
            if rng.random() < 0.5:
                live[key] = [0, []]  # back later under the same key with a new list, recomputed from 0
            else:
                del live[key]
        while len(live) < 40 and rng.random() < 0.7:  # admitted, some with a long cached prefix
            cached = rng.choice([0, rng.randrange(0, 1000)])
            live[next_key] = [cached, []]
            next_key += 1
        keys = [k for k in live if rng.random() < 0.9] or list(live)[:1]
        seqs = []
        for k in keys:
            cached, ids = live[k]
            new = rng.choice([1, 1, 1, rng.randrange(1, 100)])
            while len(ids) * bs < cached + new:
                ids.append(next_block % 5000)  # in-place appends: only these travel
                next_block += 7
            seqs.append(SeqStep(cached, new, ids))
            live[k][0] = cached + new
        meta = tables.build(keys, seqs, bs)
        _meta_fields_equal(meta, build_metadata([OracleSeq(s.num_cached, s.num_new, list(s.block_ids))
                                                 for s in seqs], bs))


@pytest.mark.parametrize("name", ["decode_4", "decode_256", "mixed_128", "prefix_64"])
def test_metadata_workloads(hip, name):
    from minillm import workloads
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    wl = workloads.WORKLOADS[name]()
    meta = AttentionMetadata.build([SeqStep(*s) for s in wl.seqs], wl.block_size, DEV)
    _meta_fields_equal(meta, build_metadata([OracleSeq(*s) for s in wl.seqs], wl.block_size))


# ------------------------------------------------------------------ append + attention on the workloads


@pytest.mark.parametrize("name", ["decode_4", "decode_256"])
def test_workload_parity(hip, name):
    from minillm import workloads

    wl = workloads.WORKLOADS[name]()
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("name", ["mixed_128", "prefix_64"])
def test_prefill_workload_parity(hip, name, prefill_rows):
    # both prefill kernels on the two prefill workloads: pools bit-exact, outputs within tolerance
    from minillm import workloads
    from minillm.attention.hip_backend import HipBackend

    wl = workloads.WORKLOADS[name]()
    backend = HipBackend()
    out, pk, pv, _ = hip_step(wl, DEV, backend=backend)
    assert backend._plan.q_tile * (wl.h // wl.hkv) == prefill_rows
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_mixed_step_overlap_is_bit_identical(hip):
    # the prefill launch on a second stream beside decode + merge gives the sequential step's output
    from minillm import workloads
    from minillm.attention.hip_backend import HipBackend

    wl = workloads.mixed_128()
    outs = []
    for overlap in (False, True):
        be = HipBackend()
        be.overlap_mixed = overlap
        outs.append(hip_step(wl, DEV, backend=be)[0])
    torch.cuda.synchronize()
    assert torch.equal(bits(outs[0]), bits(outs[1]))


@pytest.mark.parametrize("pool", ["bf16", "fp8"])
@pytest.mark.parametrize("rotary", [False, True])
def test_one_call_layer_equals_separate_launches(hip, pool, rotary):
    # mllm_attention_forward (forward / forward_rotary's single host call) against the same launches made
    # one entry point at a time (append or RoPE + append, decode, merge, prefill): pools, rotated q and
    # output bit for bit, on a step with every row kind
    from minillm import workloads
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, SeqStep
    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import RotaryEmbedding

    wl = workloads.mixed_128()
    fp8 = pool == "fp8"
    ks, vs = (0.75, 1.25) if fp8 else (1.0, 1.0)
    results = []
    for one_call in (True, False):
        be = HipBackend()
        meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
        q, k, v = wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV)
        pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
        if fp8:
            pk, pv = pk.to(torch.float8_e4m3fn), pv.to(torch.float8_e4m3fn)
        cos = sin = None
        if rotary:
            cos, sin = RotaryEmbedding(LlamaConfig(**LLAMA_3_1_8B))(meta.positions[None], q.dtype)
            cos, sin = cos[0], sin[0]
        out = torch.full_like(q, float("nan"))
        q_rot = torch.full_like(q, float("nan")) if rotary else None
        if one_call:
            be.run_layer(q, k, v, pk, pv, meta, out, cos, sin, q_rot, ks, vs)
        else:
            qa = q
            if rotary:
                qa = q_rot = be.rope_append(q, k, v, cos, sin, pk, pv, meta, ks, vs)
            else:
                be.append(k, v, pk, pv, meta, ks, vs)
            be.attend(qa, pk, pv, meta, out, ks, vs)
        torch.cuda.synchronize()
        results.append((out, q_rot, pk, pv))
    (o1, r1, k1, v1), (o2, r2, k2, v2) = results
    assert torch.isfinite(o1).all()
    assert torch.equal(bits(o1), bits(o2))
    assert torch.equal(k1.view(torch.uint8), k2.view(torch.uint8)) and torch.equal(v1.view(torch.uint8), v2.view(torch.uint8))
    if rotary:
        assert torch.equal(bits(r1), bits(r2))


def test_fp16_pool_parity(hip):
    from minillm import workloads

    wl = workloads.mixed_128(dtype=torch.float16)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def _junk(value):
    def fill(pk, pv, wl):
        used = torch.zeros(wl.num_blocks * wl.block_size, dtype=torch.bool)
        for c, n, blocks in wl.seqs:
            for p in range(c):  # cached context stays; everything else becomes junk
                used[blocks[p // wl.block_size] * wl.block_size + p % wl.block_size] = True
        junk = ~used.to(pk.device)
        if value == "nan":
            pk.view(-1, wl.hkv, wl.dh)[junk] = float("nan")
            pv.view(-1, wl.hkv, wl.dh)[junk] = float("nan")
        else:
            pk.view(-1, wl.hkv, wl.dh)[junk] = value
            pv.view(-1, wl.hkv, wl.dh)[junk] = value
    return fill


@pytest.mark.parametrize("name", ["decode_4", "mixed_128"])
def test_slots_a_row_does_not_own_never_matter(hip, name):
    # reference tests/test_paged.py:104-106 fills the pool with 1e4; NaN junk is stricter still
    from minillm import workloads

    wl = workloads.WORKLOADS[name]()
    outs = [hip_step(wl, DEV, pool_fill=_junk(v))[0] for v in (0.0, 1e4, "nan")]
    assert torch.equal(bits(outs[0]), bits(outs[1])) and torch.equal(bits(outs[0]), bits(outs[2]))


# ------------------------------------------------------------------ the reference's own kernel harness


def _kernel_case(h=8, hkv=2, dh=128, bs=16, dtype=torch.bfloat16, steps=None, seed=0, num_blocks=64):
    """tests/test_kernels.py:29-48 of the reference: a ragged step with every row kind over a
    random-junk pool and shuffled blocks."""
    from minillm.workloads import Workload

    g = torch.Generator().manual_seed(seed)
    steps = steps or [(0, 37), (90, 1), (40, 25), (0, 1), (300, 1)]
    pool_k = torch.randn(num_blocks, bs, hkv, dh, generator=g).to(dtype)
    pool_v = torch.randn(num_blocks, bs, hkv, dh, generator=g).to(dtype)
    free = list(range(num_blocks))
    random.Random(3).shuffle(free)
    seqs = []
    for cached, new in steps:
        n = cached + new
        seqs.append((cached, new, [free.pop() for _ in range(-(-n // bs))]))
    n = sum(new for _, new in steps)
    q = torch.randn(n, h, dh, generator=g).to(dtype)
    k = torch.randn(n, hkv, dh, generator=g).to(dtype)
    v = torch.randn(n, hkv, dh, generator=g).to(dtype)
    return Workload("kernel_case", seqs, num_blocks, q, k, v, pool_k, pool_v, h=h, hkv=hkv, dh=dh, block_size=bs)


def test_reference_mixed_step(hip):
    wl = _kernel_case()
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))  # identical writes
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_reference_decode_only_step(hip):
    # tests/test_kernels.py:62-72: contexts 5 / 63 / 17, 4-block tables (wider than needed)
    wl = _kernel_case(steps=[(5, 1), (63, 1), (17, 1)])
    wl.seqs = [(c, n, list(range(i * 4, i * 4 + 4))) for i, (c, n, _) in enumerate(wl.seqs)]
    out, *_ = hip_step(wl, DEV)
    ref, *_ = oracle_step(wl, DEV)
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("h,hkv", [(8, 8), (16, 8), (32, 4), (64, 4), (4, 1), (16, 1), (32, 1)],
                         ids=["g1", "g2", "g8", "g16", "mqa-g4", "mqa-g16", "g32"])
def test_group_sizes(hip, h, hkv):
    steps = [(0, 37), (90, 1), (40, 25), (0, 1), (300, 1), (17, 70)]
    wl = _kernel_case(h=h, hkv=hkv, steps=steps)
    if h // hkv > 16:  # decode supports up to 16 query heads per KV head
        with pytest.raises(ValueError, match="16 query heads"):
            hip_step(wl, DEV)
        return
    out, *_ = hip_step(wl, DEV)
    ref, *_ = oracle_step(wl, DEV)
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bs", [32, 64])
def test_larger_blocks(hip, bs):
    wl = _kernel_case(bs=bs, steps=[(0, 37), (90, 1), (40, 25), (0, 1), (300, 1), (129, 130)], num_blocks=48)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("h,hkv", [(32, 1), (64, 2)], ids=["g32", "g32-hkv2"])
def test_prefill_group_32(hip, prefill_rows, h, hkv):
    # 32 query heads per KV head: decode does not take it, prefill does (one token per wavefront, 8 per
    # q tile); rows with several new tokens only, fresh and cached, lengths not tile-aligned
    steps = [(0, 37), (40, 25), (17, 70), (300, 2), (129, 130), (0, 9)]
    wl = _kernel_case(h=h, hkv=hkv, steps=steps, num_blocks=64)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bs", [128, 256])
def test_blocks_of_several_key_tiles(hip, prefill_rows, bs):
    # a page of 128 or 256 tokens holds 2 or 4 of the prefill kernel's 64-key tiles and 8 or 16 of
    # decode's 16-token tiles; rows of every kind, prefixes past one page and past several
    steps = [(0, 37), (90, 1), (40, 25), (0, 1), (300, 1), (129, 130), (700, 300), (1000, 1), (255, 2)]
    nb = sum(-(-(c + n) // bs) for c, n in steps) + 4
    wl = _kernel_case(h=32, hkv=8, bs=bs, steps=steps, num_blocks=nb)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_prefill_tile_and_pair_boundaries(hip, prefill_rows):
    # the prefill kernel runs 64-key tiles in pairs: rows whose visible keys end one before, on and one
    # after a tile, pair and q-tile boundary (odd and even tile counts, a pair's second tile past the row
    # or past a wavefront's last row), with 2 to 65 new tokens
    steps = []
    for kv_end in (63, 64, 65, 127, 128, 129, 191, 192, 193, 256, 257, 320):
        for new in (2, 33, 64, 65):
            if new <= kv_end:
                steps.append((kv_end - new, new))
    nb = sum(-(-(c + n) // 16) for c, n in steps) + 4
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=nb, seed=5)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("seed", range(4))
def test_random_mixed_steps(hip, prefill_rows, seed):
    # seeded random steps with every row kind (fresh and cached, one and many new tokens, lengths not
    # page-aligned) at the Llama GQA shape: the prefill items of many lengths exercise the plan's
    # longest-first order and record fields; pools bit-exact, outputs within tolerance of the oracle
    rng = random.Random(1000 + seed)
    bs = rng.choice([16, 32])
    steps = []
    for _ in range(rng.randrange(4, 14)):
        new = rng.choice([1, 1, 1, 2, rng.randrange(3, 200), rng.randrange(200, 420)])
        steps.append((rng.randrange(0, 900), new))
    nb = sum(-(-(c + n) // bs) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, bs=bs, steps=steps, seed=seed, num_blocks=nb)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("seed", range(6))
def test_random_decode_heavy_steps(hip, seed):
    # seeded steps of 60-300 rows, mostly decode, over contexts from one page to 100 pages and block sizes
    # 16 / 32 / 64: the plan's equal bins cut rows at varied offsets (rows inside one bin, rows over
    # several, bins of several rows); pools bit-exact, outputs within tolerance of the oracle
    rng = random.Random(3000 + seed)
    bs = rng.choice([16, 32, 64])
    steps = [(rng.randrange(0, rng.choice([16, 200, 1600])), rng.choice([1] * 9 + [rng.randrange(2, 90)]))
             for _ in range(rng.randrange(60, 300))]
    nb = sum(-(-(c + n) // bs) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, bs=bs, steps=steps, seed=seed, num_blocks=nb)
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_llama_call_site_views(hip):
    # the model passes q[0].transpose(0, 1) of a [1, H, N, Dh] tensor: token stride Dh, head stride N*Dh
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    wl = _kernel_case(h=32, hkv=8)
    n = wl.num_tokens
    q4 = wl.q.transpose(0, 1).contiguous()[None]  # [1, H, N, Dh]
    k4 = wl.k.transpose(0, 1).contiguous()[None]
    v4 = wl.v.transpose(0, 1).contiguous()[None]
    meta = AttentionMetadata.build([SeqStep(*s) for s in wl.seqs], wl.block_size, DEV)
    pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
    qd, kd, vd = (t.to(DEV)[0].transpose(0, 1) for t in (q4, k4, v4))
    assert not qd.is_contiguous() and qd.shape == (n, 32, 128)
    out = get_backend("hip").forward(qd, kd, vd, pk, pv, meta)
    ref, rk, _ = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_plan_is_reused_per_metadata(hip):
    from minillm.attention import get_backend

    wl = _kernel_case()
    backend = get_backend("hip")
    out1, pk, pv, meta = hip_step(wl, DEV, backend=backend)
    plan = backend._plan
    out2 = backend.forward(wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV), pk, pv, meta)
    assert backend._plan is plan  # same metadata object: no re-plan (the 32-layer reuse)
    assert torch.equal(bits(out1), bits(out2))


def test_plan_contents(hip):
    # the GPU plan against the rules it implements, on rows of many lengths.  Decode rows' pages, rows in
    # sequence order, form one stream of T pages cut into nb = ceil(T / C) bins of floor / ceil(T / nb)
    # pages; a row's part in a bin is a segment, rows cut into several segments get consecutive partial
    # slots and one merge item.  A prefill row gets one item per q_tile new tokens, launched in decreasing
    # number of 64-key tiles its causal context spans
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, SeqStep, decode_plan_size

    rng = random.Random(7)
    steps = [(rng.randrange(0, 5000), rng.choice([1, 1, 2, 40, 200])) for _ in range(300)]
    seqs, o = [], 0
    for c, n in steps:
        need = -(-(c + n) // 16)
        seqs.append(SeqStep(c, n, list(range(o, o + need))))
        o += need
    meta = AttentionMetadata.build(seqs, 16, DEV)
    backend = HipBackend()
    backend._make_plan(meta, 32, 8, 128, torch.device(DEV), torch.cuda.current_stream().cuda_stream)
    p = backend._plan
    c = p.pages_per_split
    dec = p.decode_work.view(-1, 4).cpu().tolist()
    starts = [0]
    for _, n in steps:
        starts.append(starts[-1] + n)
    kv_starts = [0]
    for cc, n in steps:
        kv_starts.append(kv_starts[-1] + -(-(cc + n) // 16))
    rows = [(s, -(-(cc + n) // 16), kv_starts[s], starts[s], cc + n) for s, (cc, n) in enumerate(steps) if n == 1]
    bins, exp_segs, exp_merge, slot = decode_plan.restate(rows, c)
    nb, total = len(bins), sum(r[1] for r in rows)
    assert dec[0] == [nb, len(exp_segs), slot, 0]
    assert [r[:3] for r in dec[1:1 + nb]] == [b + [1 + nb] for b in bins]
    got_segs = dec[1 + nb:1 + nb + 2 * len(exp_segs)]
    assert [(got_segs[2 * i], got_segs[2 * i + 1]) for i in range(len(exp_segs))] == exp_segs
    sizes = [sum(exp_segs[g][0][1] for g in range(b0, b1)) for b0, b1 in bins]
    assert max(sizes) - min(sizes) <= 1 and max(sizes) <= c
    assert all(seg[0][1] <= 128 for seg in exp_segs)
    n_rec, n_merge = decode_plan_size(total, len(rows), c)
    assert 1 + nb + 2 * len(exp_segs) <= n_rec == p.num_decode and len(exp_merge) <= n_merge == p.num_merge
    mw = p.merge_work.view(-1, 4).cpu().tolist()
    assert mw[:len(exp_merge)] == exp_merge and all(r[0] == -1 for r in mw[len(exp_merge):])
    exp_pf = []
    for s, (cc, n) in enumerate(steps):
        if n > 1:
            nt = -(-n // p.q_tile)
            exp_pf += [[s, (nt - 1 - j) * p.q_tile] for j in range(nt)]
    recs = p.prefill_work.view(-1, 8).cpu().tolist()
    assert sorted(r[:2] for r in recs) == sorted(exp_pf)
    for s, t0, qs, nn, cached, kv0, kv_end, ntiles in recs:
        c, n = steps[s]
        assert (qs, nn, cached, kv0) == (starts[s], n, c, kv_starts[s])
        assert kv_end == c + min(t0 + p.q_tile, n) and ntiles == -(-kv_end // 64)
    spans = [r[7] for r in recs]
    assert spans == sorted(spans, reverse=True) and len(set(spans)) > 20


def test_plan_and_attention_over_more_rows_than_one_plan_chunk(hip):
    # the plan walks the rows 1,024 at a time (its scans carry a base from chunk to chunk): 2,500 rows of
    # every kind, the plan's decode records against their restatement and the outputs against the oracle
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    rng = random.Random(31)
    steps = [(rng.randrange(0, 60), rng.choice([1, 1, 1, 1, rng.randrange(2, 20)])) for _ in range(2500)]
    nb = sum(-(-(c + n) // 16) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=nb, seed=31)
    out, pk, pv, meta = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)
    backend = HipBackend()
    backend._make_plan(meta, 32, 8, 128, torch.device(DEV), torch.cuda.current_stream().cuda_stream)
    p = backend._plan
    starts, kv_starts = [0], [0]
    for c, n in steps:
        starts.append(starts[-1] + n)
        kv_starts.append(kv_starts[-1] + -(-(c + n) // 16))
    rows = [(s, -(-(c + n) // 16), kv_starts[s], starts[s], c + n) for s, (c, n) in enumerate(steps) if n == 1]
    bins, segs, merges, slot = decode_plan.restate(rows, p.pages_per_split)
    dec = p.decode_work.view(-1, 4).cpu().tolist()
    assert dec[0] == [len(bins), len(segs), slot, 0]
    got = dec[1 + len(bins):1 + len(bins) + 2 * len(segs)]
    assert [(got[2 * i], got[2 * i + 1]) for i in range(len(segs))] == segs
    assert p.merge_work.view(-1, 4).cpu().tolist()[:len(merges)] == merges


@pytest.mark.parametrize("pages_per_split", [8, 13])
def test_decode_rows_with_pages_past_their_last_token(hip, pages_per_split):
    # a caller's page lists may run past a row's last token (pages held ahead).  The plan counts those
    # pages, so a bin boundary can leave a segment of such pages only, with no tile to stream: the wave
    # must still load the next segment's first tile itself.  Decode rows with 0-5 extra pages each,
    # through the C ABI, against the oracle on the same rows without them
    from minillm import _native
    from minillm.attention.hip_backend import HipBackend, _ptr
    from minillm.attention.metadata import AttentionMetadata, SeqStep, decode_plan_size

    rng = random.Random(21)
    steps = [(rng.randrange(0, 300), 1) for _ in range(40)]
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=400, seed=21)
    extra = [rng.randrange(0, 6) for _ in steps]
    lists = [list(b) + [rng.randrange(wl.num_blocks) for _ in range(e)] for (_, _, b), e in zip(wl.seqs, extra)]
    rows = [(i, len(lst), 0, i, c + 1) for i, ((c, _), lst) in enumerate(zip(steps, lists))]
    _, segs, _, _ = decode_plan.restate(rows, pages_per_split)
    assert any(r0[2] * 16 >= r0[3] for r0, _ in segs)  # some segment holds extra pages only

    ref, rk, rv = oracle_step(wl, DEV)
    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    q, k, v = wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV)
    pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
    HipBackend().append(k, v, pk, pv, meta)
    kv_indptr = torch.tensor([0] + [sum(len(x) for x in lists[:i + 1]) for i in range(len(lists))],
                             dtype=torch.int32, device=DEV)
    kv_indices = torch.tensor([b for lst in lists for b in lst], dtype=torch.int32, device=DEV)
    total = sum(len(x) for x in lists)
    n_rec, n_merge = decode_plan_size(total, len(lists), pages_per_split)
    dec = torch.full((4 * n_rec,), -1, dtype=torch.int32, device=DEV)
    mrg = torch.full((4 * n_merge,), -1, dtype=torch.int32, device=DEV)
    lib = _native.lib()
    st = _native.stream_ptr(DEV)
    lib.call("mllm_plan", meta.qo_indptr.data_ptr(), kv_indptr.data_ptr(), meta.seq_lens_i32.data_ptr(), len(lists),
             pages_per_split, 64, dec.data_ptr(), n_rec, _ptr(mrg), n_merge, 0, 0, st)
    ws = torch.empty(lib.workspace_bytes(n_rec, 32, 128), dtype=torch.uint8, device=DEV)
    out = torch.full_like(q, float("nan"))
    nb, bs, hkv, dh = pk.shape
    lib.call("mllm_paged_decode", q.data_ptr(), q.stride(0), q.stride(1), pk.data_ptr(), pv.data_ptr(), nb, bs, 32,
             hkv, dh, meta.qo_indptr.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
             meta.seq_lens_i32.data_ptr(), dec.data_ptr(), n_rec, _ptr(mrg), n_merge, pages_per_split, dh ** -0.5,
             _native.dtype_code(q.dtype), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), st)
    lib.call("mllm_merge_splits", _ptr(mrg), n_merge, n_rec, 32, dh, meta.qo_indptr.data_ptr(),
             _native.dtype_code(q.dtype), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), st)
    torch.cuda.synchronize()
    assert dec[0].item() == -(-total // pages_per_split)  # the plan fit its capacity
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("pages_per_split", [128, 150, 192])
def test_decode_bins_of_up_to_192_pages(hip, monkeypatch, pages_per_split):
    # a bin holds up to 192 pages (three page-id registers per lane): long decode rows cut into such bins,
    # bf16 and fp8 pools (the one-head and the pair kernels), against the oracle
    from minillm.attention.hip_backend import HipBackend

    rng = random.Random(pages_per_split)
    steps = [(rng.randrange(1500, 7000), 1) for _ in range(24)] + [(rng.randrange(0, 200), 1) for _ in range(8)]
    nb = sum(-(-(c + n) // 16) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=nb, seed=pages_per_split)
    monkeypatch.setenv("MLLM_PAGES_PER_SPLIT", str(pages_per_split))
    be = HipBackend()
    out, pk, pv, meta = hip_step(wl, DEV, backend=be)
    assert be._plan.pages_per_split == pages_per_split
    segs = be._plan.decode_work.view(-1, 4)[1 + be._plan.decode_work[0].item():].cpu()
    longest = segs[0::2][:, 1].max().item()  # bins hold floor or ceil(T / bins) pages: some segment fills one
    assert pages_per_split - 1 <= longest <= pages_per_split and longest > 127
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)
    from test_gpu_fp8 import _check, fp8_step

    _check(*fp8_step(wl, 0.5, 2.0))  # the pair kernel (two KV heads per wavefront)


@pytest.mark.parametrize("h,hkv", [(32, 8), (64, 16)])
def test_whole_page_launch_equals_four_wave_launch(hip, h, hkv):
    # the library picks whole-page workgroups (8 KV heads each, one per CU) from 24 pages a bin up and
    # 4-wavefront workgroups below; over the same plan the two launch shapes give the same bits (each
    # wavefront's arithmetic is the same), and both match the oracle
    from minillm import _native
    from minillm.attention.hip_backend import HipBackend, _ptr, whole_page
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    rng = random.Random(hkv)
    steps = [(rng.randrange(100, 3000), 1) for _ in range(96)] + [(rng.randrange(0, 40), rng.randrange(2, 90))
                                                                  for _ in range(3)]
    nb = sum(-(-(c + n) // 16) for c, n in steps) + 8
    wl = _kernel_case(h=h, hkv=hkv, steps=steps, num_blocks=nb, seed=hkv)
    be = HipBackend()
    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    q, k, v = wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV)
    pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
    be.append(k, v, pk, pv, meta)
    plan = be.plan(meta, h, hkv, 128, torch.device(DEV))
    assert whole_page(False, hkv, plan.pages_per_split)  # the backend sized this step for whole pages
    ws = torch.empty(max(plan.workspace_bytes, 16), dtype=torch.uint8, device=DEV)
    lib, st = _native.lib(), _native.stream_ptr(DEV)
    outs = []
    for split_arg in (plan.pages_per_split, 8):  # the same plan, launched whole-page, then 4-wavefront
        assert whole_page(False, hkv, split_arg) == (split_arg >= 24)
        out = torch.full_like(q, float("nan"))
        lib.call("mllm_paged_decode", q.data_ptr(), q.stride(0), q.stride(1), pk.data_ptr(), pv.data_ptr(),
                 pk.shape[0], 16, h, hkv, 128, *plan.meta_ptrs, _ptr(plan.decode_work), plan.num_decode,
                 _ptr(plan.merge_work), plan.num_merge, split_arg, 128 ** -0.5, _native.dtype_code(q.dtype),
                 out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), st)
        lib.call("mllm_merge_splits", _ptr(plan.merge_work), plan.num_merge, plan.num_decode, h, 128,
                 meta.qo_indptr.data_ptr(), _native.dtype_code(q.dtype), out.data_ptr(), out.stride(0),
                 out.stride(1), ws.data_ptr(), ws.numel(), st)
        outs.append(out)
    torch.cuda.synchronize()
    rows = torch.tensor([i for i, (c, n) in enumerate(steps) if n == 1], device=DEV)  # decode rows: q row = i
    assert torch.equal(bits(outs[0][rows]), bits(outs[1][rows]))
    ref, _, _ = oracle_step(wl, DEV)
    torch.testing.assert_close(outs[0][rows].float(), ref[rows].float(), atol=ATOL, rtol=RTOL)


def test_plan_overflow_is_reported(hip):
    # a decode plan sized one record (or one merge) short of what the step needs gets no decode work at all,
    # and its header reports {0, records needed, merges needed, -1}, which check_plan_header turns into an
    # error; at the exact size it fits and the header is {bins, segments, slots, 0}
    from minillm import _native
    from minillm.attention.hip_backend import PlanOverflowError, _ptr, check_plan_header
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    rng = random.Random(5)
    steps = [(rng.randrange(0, 300), 1) for _ in range(40)]
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=400, seed=5)
    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    split = 8
    rows, kv0 = [], 0
    for i, (c, n) in enumerate(steps):
        pages = -(-(c + n) // 16)
        rows.append((i, pages, kv0, i, c + n))
        kv0 += pages
    bins, segs, merges, slots = decode_plan.restate(rows, split)
    need, need_m = 1 + len(bins) + 2 * len(segs), len(merges)
    assert need_m > 1
    lib = _native.lib()
    st = _native.stream_ptr(DEV)
    for cap, cap_m, fits in ((need, need_m, True), (need - 1, need_m, False), (need, need_m - 1, False)):
        dec = torch.full((4 * cap,), -1, dtype=torch.int32, device=DEV)
        mrg = torch.full((4 * cap_m,), -1, dtype=torch.int32, device=DEV)
        lib.call("mllm_plan", meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(), meta.seq_lens_i32.data_ptr(),
                 len(steps), split, 64, dec.data_ptr(), cap, _ptr(mrg), cap_m, 0, 0, st)
        torch.cuda.synchronize()
        if fits:
            assert dec[:4].tolist() == [len(bins), len(segs), slots, 0]
            check_plan_header(dec)
        else:
            assert dec[:4].tolist() == [0, need, need_m, -1]
            assert (dec[4:] == -1).all() and (mrg == -1).all()  # no decode work written
            with pytest.raises(PlanOverflowError, match=f"{need} records and {need_m} merges"):
                check_plan_header(dec)


def test_prefill_item_without_visible_keys_writes_nothing(hip):
    # a plan record whose row has no visible key (kv_end 0: seq_lens below the new-token count, which the
    # metadata build never produces) makes the workgroup return before any load; out keeps its sentinel
    from minillm import _native

    lib = _native.lib()
    h, hkv, dh, bs, nb = 32, 8, 128, 16, 8
    q = torch.randn(64, h, dh, device=DEV).to(torch.bfloat16)
    pool = torch.zeros(nb, bs, hkv, dh, dtype=torch.bfloat16, device=DEV)
    out = torch.full((64, h, dh), 7.0, dtype=torch.bfloat16, device=DEV)
    qo = torch.tensor([0, 64], dtype=torch.int32, device=DEV)
    kvp = torch.tensor([4, 8], dtype=torch.int32, device=DEV)
    kvi = torch.arange(8, dtype=torch.int32, device=DEV)
    lens = torch.tensor([0], dtype=torch.int32, device=DEV)
    # {seq, t0, qs, nn, cached, kv_start, kv_end, ntiles}
    rec = torch.tensor([0, 0, 0, 64, -64, 4, 0, 0], dtype=torch.int32, device=DEV)
    lib.call("mllm_paged_prefill", q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), pool.data_ptr(), nb, bs,
             h, hkv, dh, qo.data_ptr(), kvp.data_ptr(), kvi.data_ptr(), lens.data_ptr(), rec.data_ptr(), 1,
             256 // (h // hkv), dh ** -0.5, _native.dtype_code(torch.bfloat16), out.data_ptr(), out.stride(0),
             out.stride(1), _native.stream_ptr(torch.device(DEV)))
    # the same record as a 128-row item (4-wavefront workgroups)
    lib.call("mllm_paged_prefill", q.data_ptr(), q.stride(0), q.stride(1), pool.data_ptr(), pool.data_ptr(), nb, bs,
             h, hkv, dh, qo.data_ptr(), kvp.data_ptr(), kvi.data_ptr(), lens.data_ptr(), rec.data_ptr(), 1,
             128 // (h // hkv), dh ** -0.5, _native.dtype_code(torch.bfloat16), out.data_ptr(), out.stride(0),
             out.stride(1), _native.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


def test_unsupported_shapes_raise(hip):
    wl = _kernel_case(dh=64)
    with pytest.raises(ValueError, match="head_dim"):
        hip_step(wl, DEV)


@pytest.mark.parametrize("kv", ["bf16", "fp8"])
def test_maximum_sizes(hip, kv):
    # a 65,536-token decode context (4,096 pages, 32+ splits merged), a 4,096-token prompt over 4,096
    # cached tokens (64 query tiles, 128 key tiles each), and short rows beside them, on a shuffled pool
    from minillm.workloads import Workload

    g = torch.Generator().manual_seed(7)
    h, hkv, dh, bs = 32, 8, 128, 16
    steps = [(65535, 1), (4096, 4096), (0, 3), (17, 1), (100, 40)]
    need = sum(-(-(c + n) // bs) for c, n in steps)
    nb = need + 64
    perm = torch.randperm(nb, generator=g).tolist()
    seqs, o = [], 0
    for c, n in steps:
        k = -(-(c + n) // bs)
        seqs.append((c, n, perm[o:o + k]))
        o += k
    n_tok = sum(n for _, n in steps)

    def mk(*shape):
        return torch.randn(*shape, generator=g).to(torch.bfloat16)

    wl = Workload("max_sizes", seqs, nb, mk(n_tok, h, dh), mk(n_tok, hkv, dh), mk(n_tok, hkv, dh),
                  mk(nb, bs, hkv, dh), mk(nb, bs, hkv, dh))
    if kv == "bf16":
        out, pk, pv, _ = hip_step(wl, DEV)
        ref, rk, rv = oracle_step(wl, DEV)
        assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    else:
        from test_gpu_fp8 import fp8_step

        out, pools, ref, exp = fp8_step(wl, 0.05, 0.05)
        assert torch.equal(pools[0].view(torch.uint8), exp[0].view(torch.uint8))
        assert torch.equal(pools[1].view(torch.uint8), exp[1].view(torch.uint8))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_rows_without_new_tokens(hip):
    """Rows with no new token, which the reference's build accepts (metadata.py:70-103) and its
    multi-token loop attends with zero queries (paged_torch_ref.py:61-73): the metadata is bit-identical
    to the oracle's (a first row without tokens has logits_index -1), the pools too, and every new token's
    output matches the oracle."""
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    steps = [(40, 0), (37, 1), (100, 0), (0, 5), (300, 1), (17, 0), (64, 33), (250, 0), (129, 1)]
    wl = _kernel_case(h=32, hkv=8, steps=steps, num_blocks=96, seed=5)
    meta = AttentionMetadata.build([SeqStep(c, n, b) for c, n, b in wl.seqs], wl.block_size, DEV)
    _meta_fields_equal(meta, build_metadata([OracleSeq(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size))
    assert meta.logits_index[0].item() == -1
    out, pk, pv, _ = hip_step(wl, DEV)
    ref, rk, rv = oracle_step(wl, DEV)
    assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_stream_handle_is_the_current_stream():
    """Every launch goes on the raw stream `_native.stream_ptr` returns: torch's current stream of the device
    (the default one, a side stream inside `torch.cuda.stream`, and the capture stream of a graph being
    recorded), whatever form the device is given in."""
    from minillm import _native

    dev = torch.device(DEV)
    want = torch.cuda.current_stream(dev).cuda_stream
    assert _native.stream_ptr(dev) == _native.stream_ptr(DEV) == _native.stream_ptr(0) == want
    assert _native.stream_ptr(torch.device("cuda")) == want
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        assert _native.stream_ptr(dev) == side.cuda_stream != want
    x = torch.zeros(4, device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        got, cap = _native.stream_ptr(dev), torch.cuda.current_stream(dev).cuda_stream
        x.add_(1)
    assert got == cap != want
    graph.replay()
    torch.cuda.synchronize()
    assert x.tolist() == [1.0] * 4
