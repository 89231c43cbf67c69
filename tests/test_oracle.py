"""Pins the CPU oracle against the reference's own known answers and against the mathematics.

Nothing here compares the oracle with a retyped copy of itself: metadata is checked against the
reference's KAT and against per-token/per-page invariants; attention against float64 textbook
attention written with explicit per-head loops (tests/naive.py).
"""

import json
import math
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from naive import causal_allowed, dense_context, naive_attention
from oracle import torch_ref
from oracle.metadata import OracleSeq, build_metadata

GOLDEN = Path(__file__).resolve().parent / "golden"


def kat():
    return json.loads((GOLDEN / "metadata_kat.json").read_text())


# ---------------------------------------------------------------- metadata


def test_metadata_known_answer():
    g = kat()
    meta = build_metadata([OracleSeq(c, n, b) for c, n, b in g["seqs"]], g["block_size"])
    exp = g["expected"]
    assert meta.query_start_loc == exp["query_start_loc"]
    assert meta.seq_lens == exp["seq_lens"]
    assert meta.num_new == exp["num_new"]
    for name, dt in g["dtypes"].items():
        arr = getattr(meta, name)
        assert arr.dtype == np.dtype(dt), name
        assert arr.tolist() == exp[name], name


def test_metadata_short_table_raises():
    g = kat()["short_table"]
    with pytest.raises(ValueError, match=g["error"]):
        build_metadata([OracleSeq(c, n, b) for c, n, b in g["seqs"]], g["block_size"])


def random_steps(rng, count, bs, max_ctx=300, slack=2):
    seqs = []
    used = set()
    nxt = 0
    perm = list(range(100000))
    rng.shuffle(perm)
    for _ in range(count):
        cached = rng.choice([0, rng.randrange(0, max_ctx)])
        new = rng.choice([1, 1, rng.randrange(1, 70)])
        need = -(-(cached + new) // bs) + rng.randrange(0, slack + 1)  # tables may be wider than needed
        blocks = perm[nxt:nxt + need]
        nxt += need
        used.update(blocks)
        seqs.append(OracleSeq(cached, new, blocks))
    return seqs


@pytest.mark.parametrize("bs", [1, 4, 16])
@pytest.mark.parametrize("seed", range(4))
def test_metadata_invariants(bs, seed):
    rng = random.Random(seed)
    seqs = random_steps(rng, rng.randrange(1, 40), bs)
    meta = build_metadata(seqs, bs)
    starts = meta.query_start_loc
    assert starts[0] == 0 and all(starts[i + 1] - starts[i] == s.num_new for i, s in enumerate(seqs))
    assert meta.qo_indptr.tolist() == starts
    assert meta.seq_lens == [s.num_cached + s.num_new for s in seqs] == meta.seq_lens_i32.tolist()
    width = max(len(s.block_ids) for s in seqs)
    assert meta.block_tables.shape == (len(seqs), width)
    for i, s in enumerate(seqs):
        row = meta.block_tables[i].tolist()
        assert row[:len(s.block_ids)] == s.block_ids and all(b == 0 for b in row[len(s.block_ids):])
        # every new token: position = cached + offset, slot decodes to (table[pos // bs], pos % bs)
        for j in range(s.num_new):
            t = starts[i] + j
            pos = int(meta.positions[t])
            slot = int(meta.slot_mapping[t])
            assert pos == s.num_cached + j
            assert slot // bs == s.block_ids[pos // bs] and slot % bs == pos % bs
        # pages: a prefix of the table, exactly enough blocks for the context
        lo, hi = int(meta.kv_indptr[i]), int(meta.kv_indptr[i + 1])
        length = meta.seq_lens[i]
        assert (hi - lo - 1) * bs < length <= (hi - lo) * bs
        assert meta.kv_indices[lo:hi].tolist() == s.block_ids[:hi - lo]
        last = int(meta.kv_last_page_len[i])
        assert 1 <= last <= bs and (hi - lo - 1) * bs + last == length
        assert int(meta.logits_index[i]) == starts[i + 1] - 1
    assert int(meta.kv_indptr[-1]) == meta.kv_indices.size
    assert np.array_equal(meta.block_tables_i32, meta.block_tables.astype(np.int32))


# ---------------------------------------------------------------- write_kv / gather


def test_write_then_gather_round_trip():
    # reference tests/test_paged.py:53-60
    pool = torch.zeros(6, 4, 2, 3)
    other = torch.zeros_like(pool)
    k = torch.randn(7, 2, 3)
    slots = torch.tensor([5 * 4 + i for i in range(4)] + [1 * 4 + i for i in range(3)])
    torch_ref.write_kv(pool, other, slots, k, k)
    got = torch_ref.gather(pool, torch.tensor([[5, 1]]), 7)
    torch.testing.assert_close(got[0].transpose(0, 1), k)


def test_write_touches_only_its_slots():
    g = torch.Generator().manual_seed(5)
    pool_k = torch.randn(10, 4, 2, 8, generator=g)
    pool_v = torch.randn(10, 4, 2, 8, generator=g)
    before_k, before_v = pool_k.clone(), pool_v.clone()
    slots = torch.tensor([3, 17, 38, 0])
    k, v = torch.randn(4, 2, 8, generator=g), torch.randn(4, 2, 8, generator=g)
    torch_ref.write_kv(pool_k, pool_v, slots, k, v)
    flat_k, flat_v = pool_k.view(-1, 2, 8), pool_v.view(-1, 2, 8)
    assert torch.equal(flat_k[slots], k) and torch.equal(flat_v[slots], v)
    keep = torch.ones(40, dtype=torch.bool)
    keep[slots] = False
    assert torch.equal(flat_k[keep], before_k.view(-1, 2, 8)[keep])
    assert torch.equal(flat_v[keep], before_v.view(-1, 2, 8)[keep])


# ---------------------------------------------------------------- paged attention


def build_step(case, dtype=torch.float32, junk=None):
    """The reference's paged == dense harness (tests/test_paged.py:63-93): earlier tokens are already
    in the pool, this step's are passed in."""
    torch.manual_seed(case["torch_seed"])
    h, hkv, dh, bs, nb = case["h"], case["hkv"], case["dh"], case["bs"], case["num_blocks"]
    pool_k = torch.zeros(nb, bs, hkv, dh, dtype=dtype)
    pool_v = torch.zeros(nb, bs, hkv, dh, dtype=dtype)
    if junk is not None:
        pool_k.fill_(junk)
        pool_v.fill_(junk)
    free = list(range(nb))
    random.Random(case["shuffle_seed"]).shuffle(free)
    seqs, ctx_k, ctx_v = [], [], []
    for cached, new in case["steps"]:
        n = cached + new
        blocks = [free.pop() for _ in range(-(-n // bs))]
        k, v = torch.randn(n, hkv, dh).to(dtype), torch.randn(n, hkv, dh).to(dtype)
        if cached:
            slots = torch.tensor([blocks[p // bs] * bs + p % bs for p in range(cached)])
            torch_ref.write_kv(pool_k, pool_v, slots, k[:cached], v[:cached])
        seqs.append(OracleSeq(cached, new, blocks))
        ctx_k.append(k)
        ctx_v.append(v)
    meta = build_metadata(seqs, bs)
    q = torch.randn(sum(new for _, new in case["steps"]), h, dh).to(dtype)
    new_k = torch.cat([k[c:] for k, (c, _) in zip(ctx_k, case["steps"])])
    new_v = torch.cat([v[c:] for v, (c, _) in zip(ctx_v, case["steps"])])
    return q, new_k, new_v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v


def cases():
    return json.loads((GOLDEN / "cases.json").read_text())


def test_paged_attention_equals_textbook():
    case = cases()["paged_equals_dense"]
    q, k, v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v = build_step(case)
    out = torch_ref.forward(q, k, v, pool_k, pool_v, torch_ref.torch_meta(meta, "cpu"))
    for i, s in enumerate(seqs):
        st, n, length = meta.query_start_loc[i], s.num_new, meta.seq_lens[i]
        exp = naive_attention(q[st:st + n].transpose(0, 1), ctx_k[i].transpose(0, 1), ctx_v[i].transpose(0, 1),
                              causal_allowed(n, length))
        torch.testing.assert_close(out[st:st + n].double(), exp.transpose(0, 1), atol=1e-5, rtol=1e-5)
        # and the pool really holds the context at the table's slots
        assert torch.equal(dense_context(pool_k, s.block_ids, length), ctx_k[i].transpose(0, 1))


def test_paged_attention_ignores_slots_it_does_not_own():
    case = cases()["paged_equals_dense"]
    outs = []
    for junk in (None, 1e4):
        q, k, v, pool_k, pool_v, meta, *_ = build_step(case, junk=junk)
        outs.append(torch_ref.forward(q, k, v, pool_k, pool_v, torch_ref.torch_meta(meta, "cpu")))
    torch.testing.assert_close(outs[0], outs[1], atol=1e-6, rtol=1e-6)


def test_paged_attention_bf16_kernel_case_close_to_textbook():
    # the reference's kernel harness shapes (tests/test_kernels.py:29-48) run on the CPU oracle in bf16
    case = cases()["kernel_mixed_step"]
    q, k, v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v = build_step(case, dtype=torch.bfloat16)
    out = torch_ref.forward(q, k, v, pool_k, pool_v, torch_ref.torch_meta(meta, "cpu"))
    for i, s in enumerate(seqs):
        st, n, length = meta.query_start_loc[i], s.num_new, meta.seq_lens[i]
        exp = naive_attention(q[st:st + n].transpose(0, 1), ctx_k[i].transpose(0, 1), ctx_v[i].transpose(0, 1),
                              causal_allowed(n, length))
        torch.testing.assert_close(out[st:st + n].double(), exp.transpose(0, 1), atol=2e-2, rtol=1e-2)


def _kernel_case_step():
    case = cases()["kernel_mixed_step"]  # decode rows, a fresh prompt and a prompt over cached tokens
    q, k, v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v = build_step(case)
    tm = torch_ref.torch_meta(meta, "cpu")
    torch_ref.write_kv(pool_k, pool_v, tm.slot_mapping, k, v)
    return q, pool_k, pool_v, tm, meta, seqs, ctx_k, ctx_v


def test_rounded_p_variant_without_rounding_is_sdpa():
    # the written-out attention of the noise-floor variant, with a rounding that changes nothing (float32
    # probabilities stay float32), equals the library SDPA path and the float64 textbook on every row kind
    q, pool_k, pool_v, tm, meta, seqs, ctx_k, ctx_v = _kernel_case_step()
    lib = torch_ref.paged_attention(q, pool_k, pool_v, tm)
    explicit = torch_ref.paged_attention(q, pool_k, pool_v, tm, p_round=torch.float32)
    torch.testing.assert_close(explicit, lib, atol=2e-6, rtol=1e-5)
    for i, s in enumerate(seqs):
        st, n, length = meta.query_start_loc[i], s.num_new, meta.seq_lens[i]
        exp = naive_attention(q[st:st + n].transpose(0, 1), ctx_k[i].transpose(0, 1), ctx_v[i].transpose(0, 1),
                              causal_allowed(n, length))
        torch.testing.assert_close(explicit[st:st + n].double(), exp.transpose(0, 1), atol=1e-5, rtol=1e-5)


def test_rounded_p_variant_moves_outputs_by_at_most_the_bf16_rounding_of_p():
    # rounding each probability to bf16 (relative error <= 2^-9) moves an output by at most
    # 2^-9 * sum_j p_j |v_j| <= 2^-9 * max |v|, and it does move them
    q, pool_k, pool_v, tm, meta, seqs, ctx_k, ctx_v = _kernel_case_step()
    exact = torch_ref.paged_attention(q, pool_k, pool_v, tm)
    rounded = torch_ref.paged_attention(q, pool_k, pool_v, tm, p_round=torch.bfloat16)
    vmax = max(v.abs().max().item() for v in ctx_v)
    diff = (rounded - exact).abs().max().item()
    assert 0 < diff <= 2 ** -9 * vmax + 1e-5


# ---------------------------------------------------------------- contiguous prefill


def naive_dense(q, k, v, allowed):
    return torch.stack([naive_attention(q[b], k[b], v[b], allowed[b]) for b in range(q.shape[0])])


@pytest.mark.parametrize("h,hkv", [(4, 4), (4, 2), (8, 1)], ids=["mha", "gqa", "mqa"])
def test_prefill_matches_textbook(h, hkv):
    # reference tests/test_attention.py:22-30
    g = torch.Generator().manual_seed(0)
    b, t, dh = 2, 7, 16
    q, k, v = (torch.randn(b, n, t, dh, generator=g) for n in (h, hkv, hkv))
    out = torch_ref.prefill(q, k, v)
    allowed = causal_allowed(t, t)[None].expand(b, t, t)
    torch.testing.assert_close(out.double(), naive_dense(q, k, v, allowed), atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("tq,tk", [(1, 9), (4, 9), (9, 9)], ids=["decode", "continue", "fresh"])
def test_prefill_on_top_of_cache(tq, tk):
    # reference tests/test_attention.py:47-55
    g = torch.Generator().manual_seed(2)
    q_all, k, v = (torch.randn(1, n, tk, 16, generator=g) for n in (4, 2, 2))
    q = q_all[:, :, -tq:]
    out = torch_ref.prefill(q, k, v)
    allowed = causal_allowed(tq, tk)[None]
    torch.testing.assert_close(out.double(), naive_dense(q, k, v, allowed), atol=1e-5, rtol=1e-5)


def test_prefill_is_causal():
    # reference tests/test_attention.py:33-44
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 5, 8, generator=g) for _ in range(3))
    before = torch_ref.prefill(q, k, v)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, -1] += 10
    v2[:, :, -1] += 10
    after = torch_ref.prefill(q, k2, v2)
    torch.testing.assert_close(before[:, :, :-1], after[:, :, :-1])
    assert not torch.allclose(before[:, :, -1], after[:, :, -1])


def test_prefill_key_valid_own_slot_rule():
    # left padding: query 0 has no real key and sees only its own position, the others skip key 0
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, n, 3, 8, generator=g) for n in (2, 1, 1))
    key_valid = torch.tensor([[False, True, True]])
    out = torch_ref.prefill(q, k, v, key_valid=key_valid)
    allowed = torch.tensor([[[True, False, False], [False, True, False], [False, True, True]]])
    torch.testing.assert_close(out.double(), naive_dense(q, k, v, allowed), atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(out[0, :, 0], v[0, 0, 0].expand(2, 8))


# ---------------------------------------------------------------- rotary embedding + append


def test_rope_rotates_pairs_by_hand():
    # Dh = 4: pairs (0, 2) and (1, 3) at angles a and b; a' = a cos - b sin, b' = b cos + a sin
    a_ang, b_ang = 0.7, -1.3
    x = torch.tensor([[[1.0, 2.0, 3.0, 4.0]]], dtype=torch.float64)
    cos = torch.tensor([[math.cos(a_ang), math.cos(b_ang), math.cos(a_ang), math.cos(b_ang)]], dtype=torch.float64)
    sin = torch.tensor([[math.sin(a_ang), math.sin(b_ang), math.sin(a_ang), math.sin(b_ang)]], dtype=torch.float64)
    exp = [1 * math.cos(a_ang) - 3 * math.sin(a_ang), 2 * math.cos(b_ang) - 4 * math.sin(b_ang),
           3 * math.cos(a_ang) + 1 * math.sin(a_ang), 4 * math.cos(b_ang) + 2 * math.sin(b_ang)]
    got = torch_ref.apply_rotary(x, cos, sin)[0, 0].tolist()
    assert got == pytest.approx(exp, abs=1e-12)


def _angles(n, dh, seed=0):
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(0, 100000, (n,), generator=g).double()
    inv = 1.0 / (500000.0 ** (torch.arange(0, dh, 2, dtype=torch.float64) / dh))
    ang = pos[:, None] * inv
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


def test_rope_is_a_rotation():
    # norms of every pair are kept, and rotating back by -angle restores the input
    n, h, dh = 64, 4, 16
    x = torch.randn(n, h, dh, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    cos, sin = _angles(n, dh)
    y = torch_ref.apply_rotary(x, cos, sin)
    pair_norm = lambda t: t[..., : dh // 2] ** 2 + t[..., dh // 2:] ** 2  # noqa: E731
    torch.testing.assert_close(pair_norm(y), pair_norm(x), atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(torch_ref.apply_rotary(y, cos, -sin), x, atol=1e-10, rtol=1e-10)


def test_rope_score_depends_only_on_relative_position():
    # the reference's property test (tests/test_layers.py:75-85): q.k after rotation depends on m - n only
    dh = 16
    gen = torch.Generator().manual_seed(2)
    q = torch.randn(1, 1, dh, dtype=torch.float64, generator=gen)
    k = torch.randn(1, 1, dh, dtype=torch.float64, generator=gen)
    inv = 1.0 / (10000.0 ** (torch.arange(0, dh, 2, dtype=torch.float64) / dh))

    def score(m, n):
        def cs(p):
            ang = torch.cat([p * inv, p * inv])[None]
            return ang.cos(), ang.sin()

        return (torch_ref.apply_rotary(q, *cs(m)) * torch_ref.apply_rotary(k, *cs(n))).sum().item()

    assert score(5, 2) == pytest.approx(score(103, 100), abs=1e-9)
    assert score(7, 7) == pytest.approx(score(0, 0), abs=1e-9)
    assert score(5, 2) != pytest.approx(score(5, 3), abs=1e-3)


def test_rope_then_write_kv_writes_rotated_k_and_plain_v():
    n, h, hkv, dh, nb, bs = 6, 4, 2, 8, 4, 4
    gen = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(n, x, dh, generator=gen) for x in (h, hkv, hkv))
    cos, sin = (t.float() for t in _angles(n, dh))
    kc, vc = torch.zeros(nb, bs, hkv, dh), torch.zeros(nb, bs, hkv, dh)
    slots = torch.tensor([13, 2, 7, 0, 15, 9])
    q_rot = torch_ref.rope_then_write_kv(q, k, v, cos, sin, kc, vc, slots)
    flat_k, flat_v = kc.view(-1, hkv, dh), vc.view(-1, hkv, dh)
    for i, s in enumerate(slots.tolist()):
        # the pair rule on the written row itself: k'[d] = k[d] cos - k[d + half] sin for d < half
        half = dh // 2
        exp = k[i, :, :half] * cos[i, :half] - k[i, :, half:] * sin[i, :half]
        torch.testing.assert_close(flat_k[s, :, :half], exp, atol=1e-6, rtol=1e-6)
        assert torch.equal(flat_v[s], v[i])
    assert q_rot.shape == q.shape
    untouched = sorted(set(range(nb * bs)) - set(slots.tolist()))
    assert torch.count_nonzero(flat_k[untouched]) == 0 and torch.count_nonzero(flat_v[untouched]) == 0


# ---------------------------------------------------------------- fp8 (e4m3fn) pool


def e4m3fn_value(code: int) -> float:
    """OCP e4m3fn decoded from its bit fields: 1 sign, 4 exponent (bias 7) and 3 mantissa bits; exponent
    0 is subnormal (m / 8 * 2^-6); S.1111.111 is NaN; there are no infinities."""
    s, e, m = code >> 7, (code >> 3) & 15, code & 7
    if e == 15 and m == 7:
        return math.nan
    mag = (m / 8) * 2.0 ** -6 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
    return -mag if s else mag


def fp8_bytes(x: torch.Tensor, scale: float = 1.0) -> list[int]:
    return torch_ref.quantize_fp8(x, scale).view(torch.uint8).tolist()


def test_fp8_encodings_by_hand():
    x = torch.tensor([1.0, -1.5, 0.1, 448.0, 464.0, 465.0, 480.0, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -10, 0.0, -0.0,
                      math.inf, -math.inf, math.nan, -465.0])
    assert fp8_bytes(x) == [0x38, 0xBC, 0x1D, 0x7E, 0x7E, 0x7F, 0x7F, 0x01, 0x00, 0x01, 0x00, 0x80, 0x7F, 0xFF, 0x7F,
                            0xFF]
    # the stored value is x * (1 / scale): 3 / 2 = 1.5 -> 0x3C, 1 / 0.25 = 4 -> 0x48
    assert fp8_bytes(torch.tensor([3.0]), 2.0) == [0x3C]
    assert fp8_bytes(torch.tensor([1.0]), 0.25) == [0x48]
    assert torch_ref.inv_scale(3.0) == np.float32(1.0) / np.float32(3.0)


def test_fp8_decoding_matches_the_bit_fields():
    got = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch_ref.FP8).float().tolist()
    for code, value in enumerate(got):
        exp = e4m3fn_value(code)
        assert (math.isnan(exp) and math.isnan(value)) or exp == value, hex(code)


def test_fp8_quantize_is_round_to_nearest_even_on_the_grid():
    finite = [c for c in range(256) if not math.isnan(e4m3fn_value(c))]
    # every finite code is its own encoding
    assert fp8_bytes(torch.tensor([e4m3fn_value(c) for c in finite])) == finite
    pos = list(range(0x7F))  # non-negative finite codes, increasing with value
    grid = [e4m3fn_value(c) for c in pos]
    # midpoints of neighbours: the even code wins
    mids = torch.tensor([(grid[i] + grid[i + 1]) / 2 for i in range(len(grid) - 1)])
    assert fp8_bytes(mids) == [pos[i] if pos[i] % 2 == 0 else pos[i + 1] for i in range(len(grid) - 1)]
    # brute force: the nearest grid value of log-uniform magnitudes; above 464 the cast gives NaN
    g = torch.Generator().manual_seed(0)
    mag = torch.exp2(torch.rand(20000, generator=g) * 21 - 12)  # 2^-12 .. 2^9
    sign = torch.where(torch.rand(20000, generator=g) < 0.5, -1.0, 1.0)
    xs = (mag * sign).float()
    got = fp8_bytes(xs)
    for x, code in zip(xs.tolist(), got):
        a = abs(x)
        if a > 464:
            exp = 0x7F
        else:
            d = [abs(a - v) for v in grid]
            best = min(d)
            ties = [pos[i] for i, di in enumerate(d) if di == best]
            exp = next(c for c in ties if c % 2 == 0) if len(ties) > 1 else ties[0]
        if x < 0:
            exp |= 0x80
        assert code == exp, (x, hex(code), hex(exp))


def test_fp8_write_kv_quantizes_into_its_slots_only():
    g = torch.Generator().manual_seed(4)
    kc = torch.zeros(6, 4, 2, 8, dtype=torch_ref.FP8)
    vc = torch.zeros_like(kc)
    k, v = torch.randn(7, 2, 8, generator=g) * 3, torch.randn(7, 2, 8, generator=g) * 0.1
    slots = torch.tensor([21, 22, 23, 20, 5, 4, 6])
    torch_ref.write_kv(kc, vc, slots, k, v, k_scale=2.0, v_scale=0.05)
    fk, fv = kc.view(torch.uint8).view(-1, 2, 8), vc.view(torch.uint8).view(-1, 2, 8)
    assert torch.equal(fk[slots], torch_ref.quantize_fp8(k, 2.0).view(torch.uint8))
    assert torch.equal(fv[slots], torch_ref.quantize_fp8(v, 0.05).view(torch.uint8))
    keep = torch.ones(24, dtype=torch.bool)
    keep[slots] = False
    assert torch.count_nonzero(fk[keep]) == 0 and torch.count_nonzero(fv[keep]) == 0
    # dequantized, each value is within half a grid step of the input (3 mantissa bits: 2^-4 relative)
    back = torch_ref.dequantize_fp8(kc.view(-1, 2, 8)[slots], 2.0)
    assert torch.all((back - k).abs() <= 2.0 ** -4 * k.abs() + 2.0 * 2.0 ** -10)


def test_fp8_paged_attention_equals_textbook_over_dequantized_context():
    case = cases()["paged_equals_dense"]
    q, k, v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v = build_step(case)
    ks, vs = 0.5, 0.125  # distinct, so swapping K's and V's scales fails
    k8, v8 = (torch.zeros(pool_k.shape, dtype=torch_ref.FP8) for _ in range(2))
    for i, s in enumerate(seqs):
        slots = torch.tensor([s.block_ids[p // case["bs"]] * case["bs"] + p % case["bs"] for p in range(s.num_cached)],
                             dtype=torch.long)
        torch_ref.write_kv(k8, v8, slots, ctx_k[i][:s.num_cached], ctx_v[i][:s.num_cached], ks, vs)
    out = torch_ref.forward(q, k, v, k8, v8, torch_ref.torch_meta(meta, "cpu"), k_scale=ks, v_scale=vs)
    for i, s in enumerate(seqs):
        st, n, length = meta.query_start_loc[i], s.num_new, meta.seq_lens[i]
        dk = torch_ref.dequantize_fp8(torch_ref.quantize_fp8(ctx_k[i], ks), ks)
        dv = torch_ref.dequantize_fp8(torch_ref.quantize_fp8(ctx_v[i], vs), vs)
        exp = naive_attention(q[st:st + n].transpose(0, 1), dk.transpose(0, 1), dv.transpose(0, 1),
                              causal_allowed(n, length))
        torch.testing.assert_close(out[st:st + n].double(), exp.transpose(0, 1), atol=1e-5, rtol=1e-5)


def test_rows_without_new_tokens_attend_nothing():
    """A row with no new token, which the reference's build accepts (metadata.py:70-103) and its
    multi-token loop attends with zero queries (paged_torch_ref.py:61-73), adds no output row and leaves
    every other row's output bit-identical to the same step without it; its logits_index is
    starts[i + 1] - 1, so -1 when it comes first."""
    g = torch.Generator().manual_seed(11)
    h, hkv, dh, bs, nblk = 4, 2, 16, 4, 64
    rows = [(5, 1), (0, 6), (9, 3), (13, 1), (7, 0), (12, 0), (3, 0)]  # the last three have no new token
    pool_k = torch.randn(nblk, bs, hkv, dh, generator=g)
    pool_v = torch.randn(nblk, bs, hkv, dh, generator=g)
    perm = torch.randperm(nblk, generator=g).tolist()
    blocks = [[perm.pop() for _ in range(-(-(c + n) // bs))] for c, n in rows]
    ntok = sum(n for _, n in rows)
    q = torch.randn(ntok, h, dh, generator=g)
    k = torch.randn(ntok, hkv, dh, generator=g)
    v = torch.randn(ntok, hkv, dh, generator=g)

    def run(order):
        meta = build_metadata([OracleSeq(*rows[i], blocks[i]) for i in order], bs)
        out = torch_ref.forward(q, k, v, pool_k.clone(), pool_v.clone(), torch_ref.torch_meta(meta, "cpu"))
        return out, meta

    out_a, _ = run([0, 1, 2, 3])
    out_b, meta_b = run([4, 0, 5, 1, 2, 6, 3])
    assert out_b.shape == (ntok, h, dh)
    assert torch.equal(out_a, out_b)
    assert meta_b.query_start_loc == [0, 0, 1, 1, 7, 10, 10, 11]
    assert meta_b.logits_index.tolist() == [-1, 0, 0, 6, 9, 9, 10]
