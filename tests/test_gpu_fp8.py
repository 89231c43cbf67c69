"""GPU parity of the fp8 (e4m3fn) KV pool path against the oracle.

- append (`mllm_kv_append_fp8`, `mllm_rope_kv_append_fp8`): pool bytes identical to torch's quantizing
  cast computed on the CPU, over every 16-bit input pattern and several scales;
- attention (`mllm_paged_decode_fp8`, `mllm_merge_splits`, `mllm_paged_prefill_fp8`): within
  2e-2 abs / 1e-2 rel of the oracle's gather + SDPA in float32 over the dequantized pool (value x scale);
- every e4m3fn code, subnormals under a large scale, junk in unowned slots (NaN codes included).
"""

import pytest
import torch

from harness import ATOL, RTOL, bits
from oracle import torch_ref
from oracle.metadata import OracleSeq, build_metadata

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
U8 = torch.uint8


def _u8(t):
    return t.view(U8)


def fp8_step(wl, ks, vs, fill=None):
    """One layer of `wl` on fp8 pools through the HIP backend and through the oracle.

    The initial pools are `wl`'s quantized with torch's cast on the GPU (input preparation), then
    `fill(pk8, pv8)` may set codes directly.  The oracle's pools are those plus the step's rows quantized
    on the CPU; its attention runs in float32 on the GPU.  Returns (out, pools, ref, expected pools)."""
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    pk8 = torch_ref.quantize_fp8(wl.pool_k.to(DEV), ks)
    pv8 = torch_ref.quantize_fp8(wl.pool_v.to(DEV), vs)
    if fill is not None:
        fill(pk8, pv8)
    om = build_metadata([OracleSeq(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size)
    tm = torch_ref.torch_meta(om, DEV)
    exp_k, exp_v = pk8.clone(), pv8.clone()
    slots = tm.slot_mapping
    _u8(exp_k).view(-1, wl.hkv, wl.dh).index_copy_(0, slots, _u8(torch_ref.quantize_fp8(wl.k, ks)).to(DEV))
    _u8(exp_v).view(-1, wl.hkv, wl.dh).index_copy_(0, slots, _u8(torch_ref.quantize_fp8(wl.v, vs)).to(DEV))

    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    out = get_backend("hip").forward(wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV), pk8, pv8, meta, k_scale=ks,
                                     v_scale=vs)
    ref = torch_ref.paged_attention(wl.q.to(DEV, torch.float32), exp_k, exp_v, tm, compute_dtype=torch.float32,
                                    k_scale=ks, v_scale=vs)
    return out, (pk8, pv8), ref, (exp_k, exp_v)


def _check(out, pools, ref, exp):
    assert torch.equal(_u8(pools[0]), _u8(exp[0])) and torch.equal(_u8(pools[1]), _u8(exp[1]))
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


# ------------------------------------------------------------------ append


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ks,vs", [(1.0, 1.0), (0.37, 3.0), (2.0 ** -6, 2.0 ** 7)])
def test_append_every_16bit_pattern(hip, dtype, ks, vs):
    # all 65536 bit patterns (NaN, inf, subnormals, overflow past 464 included) as K, reversed as V
    from minillm.attention.hip_backend import HipBackend

    pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(dtype).reshape(512, 1, 128)
    k, v = pat, pat.flip(0)
    slots = torch.randperm(1024, generator=torch.Generator().manual_seed(1))[:512]
    kc = torch.zeros(64, 16, 1, 128, dtype=torch_ref.FP8)
    vc = torch.zeros_like(kc)
    exp_k, exp_v = kc.clone(), vc.clone()
    torch_ref.write_kv(exp_k, exp_v, slots, k, v, ks, vs)
    gk, gv = kc.to(DEV), vc.to(DEV)

    class Meta:
        slot_mapping = slots.to(DEV)

    HipBackend().append(k.to(DEV), v.to(DEV), gk, gv, Meta, ks, vs)
    assert torch.equal(_u8(gk).cpu(), _u8(exp_k)) and torch.equal(_u8(gv).cpu(), _u8(exp_v))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rope_append_into_fp8_pool(hip, dtype):
    from minillm.attention.hip_backend import HipBackend
    from test_gpu_rope import _inputs, _Meta

    for n, (h, hkv, dh), seed in [(1, (32, 8, 128), 0), (300, (32, 8, 128), 1), (53, (16, 2, 256), 2),
                                  (37, (8, 8, 64), 3)]:
        q, k, v, cos, sin, (pk, pv), slots = _inputs(n, h, hkv, dh, dtype, seed)
        kc, vc = torch_ref.quantize_fp8(pk, 0.5), torch_ref.quantize_fp8(pv, 0.25)
        exp_k, exp_v = kc.clone(), vc.clone()
        exp_q = torch_ref.rope_then_write_kv(q, k, v, cos, sin, exp_k, exp_v, slots, 0.5, 0.25)
        gk, gv = kc.to(DEV), vc.to(DEV)
        got_q = HipBackend().rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), gk, gv,
                                         _Meta(slots.to(DEV)), 0.5, 0.25)
        assert torch.equal(bits(got_q.cpu()), bits(exp_q)), (n, h, hkv, dh)
        assert torch.equal(_u8(gk).cpu(), _u8(exp_k)) and torch.equal(_u8(gv).cpu(), _u8(exp_v)), (n, h, hkv, dh)


# ------------------------------------------------------------------ attention


@pytest.mark.parametrize("name", ["decode_4", "decode_256"])
def test_workload_parity(hip, name):
    from minillm import workloads

    wl = workloads.WORKLOADS[name]()
    _check(*fp8_step(wl, 0.05, 0.03))


@pytest.mark.parametrize("name", ["mixed_128", "prefix_64"])
def test_prefill_workload_parity(hip, name, prefill_rows):
    # both prefill kernels (256- and 128-row items) on the prefill workloads over fp8 pools
    from minillm import workloads

    wl = workloads.WORKLOADS[name]()
    _check(*fp8_step(wl, 0.05, 0.03))


def test_fp16_activations(hip):
    from minillm import workloads

    wl = workloads.mixed_128(dtype=torch.float16)
    _check(*fp8_step(wl, 1.0, 1.0))


def _kernel_case(h=8, hkv=2, bs=16, steps=None, num_blocks=64, seed=0):
    from test_gpu_paged import _kernel_case as case

    return case(h=h, hkv=hkv, bs=bs, steps=steps, num_blocks=num_blocks, seed=seed)


@pytest.mark.parametrize("h,hkv,bs", [(8, 8, 16), (16, 8, 16), (32, 4, 16), (64, 4, 16), (32, 8, 32), (32, 8, 64),
                                     (32, 8, 128), (32, 8, 256)],
                         ids=["g1", "g2", "g8", "g16", "bs32", "bs64", "bs128", "bs256"])
def test_group_sizes_and_blocks(hip, h, hkv, bs):
    steps = [(0, 37), (90, 1), (40, 25), (0, 1), (300, 1), (17, 70), (129, 130)]
    wl = _kernel_case(h=h, hkv=hkv, bs=bs, steps=steps, num_blocks=max(64, 1100 // bs))
    _check(*fp8_step(wl, 0.02, 0.02))


def test_prefill_group_32(hip, prefill_rows):
    # 32 query heads per KV head, prefill rows only (decode takes at most 16)
    steps = [(0, 37), (40, 25), (17, 70), (300, 2), (129, 130)]
    wl = _kernel_case(h=32, hkv=1, steps=steps, num_blocks=64, seed=7)
    _check(*fp8_step(wl, 0.04, 0.05))


@pytest.mark.parametrize("h,hkv", [(12, 3), (12, 6), (10, 2), (20, 4), (40, 10), (14, 2)],
                         ids=["odd-hkv", "hkv6", "g5", "g5-hkv4", "hkv10", "g7"])
def test_decode_head_pairing(hip, h, hkv):
    # fp8 decode pairs adjacent KV heads in one wavefront when the KV heads are even and a pair's query
    # heads fit the 16 MFMA columns, else runs one head per wavefront: odd KV heads, workgroups whose
    # last wavefronts have no pair (6 and 10 KV heads), 5 and 7 query heads per KV head (unused columns);
    # decode rows only, short and split
    steps = [(0, 1), (90, 1), (300, 1), (17, 1), (1000, 1), (129, 1), (15, 1), (16, 1)]
    wl = _kernel_case(h=h, hkv=hkv, steps=steps, num_blocks=200, seed=hkv)
    _check(*fp8_step(wl, 0.03, 0.04))


@pytest.mark.parametrize("seed", range(3))
def test_random_mixed_steps(hip, prefill_rows, seed):
    # seeded random steps with every row kind at the Llama GQA shape, fp8 pools with random scales
    import random

    rng = random.Random(2000 + seed)
    bs = rng.choice([16, 32])
    steps = []
    for _ in range(rng.randrange(4, 12)):
        new = rng.choice([1, 1, 2, rng.randrange(3, 200), rng.randrange(200, 400)])
        steps.append((rng.randrange(0, 900), new))
    nb = sum(-(-(c + n) // bs) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, bs=bs, steps=steps, num_blocks=nb, seed=seed)
    _check(*fp8_step(wl, rng.uniform(0.02, 0.5), rng.uniform(0.02, 0.5)))


@pytest.mark.parametrize("seed", range(3))
def test_random_decode_heavy_steps(hip, seed):
    # as the bf16 test of that name: 60-300 mostly-decode rows, block sizes 16 / 32 / 64, fp8 pools with
    # random scales (the pair kernel's bins are sized for its own occupancy)
    import random

    rng = random.Random(4000 + seed)
    bs = rng.choice([16, 32, 64])
    steps = [(rng.randrange(0, rng.choice([16, 200, 1600])), rng.choice([1] * 9 + [rng.randrange(2, 90)]))
             for _ in range(rng.randrange(60, 300))]
    nb = sum(-(-(c + n) // bs) for c, n in steps) + 8
    wl = _kernel_case(h=32, hkv=8, bs=bs, steps=steps, num_blocks=nb, seed=seed)
    _check(*fp8_step(wl, rng.uniform(0.02, 0.5), rng.uniform(0.02, 0.5)))


@pytest.mark.parametrize("h,hkv", [(32, 8), (21, 7)], ids=["pair-kernel", "one-head-kernel"])
def test_decode_rows_with_pages_past_their_last_token(hip, h, hkv):
    # the fp8 decode kernels' stream across a segment with no tile (a page list that runs past the row's
    # last token): rows with 0-5 extra pages through mllm_paged_decode_fp8, against the oracle on the
    # rows without them; 8 KV heads run the pair kernel, 7 the one-head kernel
    import random

    import decode_plan
    from minillm import _native
    from minillm.attention.hip_backend import _ptr
    from minillm.attention.metadata import AttentionMetadata, SeqStep, decode_plan_size

    rng = random.Random(23)
    steps = [(rng.randrange(0, 300), 1) for _ in range(40)]
    wl = _kernel_case(h=h, hkv=hkv, steps=steps, num_blocks=400, seed=23)
    ks, vs = 0.05, 0.04
    _, _, ref, (exp_k, exp_v) = fp8_step(wl, ks, vs)  # the oracle's output and pools after the append
    extra = [rng.randrange(0, 6) for _ in steps]
    lists = [list(b) + [rng.randrange(wl.num_blocks) for _ in range(e)] for (_, _, b), e in zip(wl.seqs, extra)]
    c = 8
    _, segs, _, _ = decode_plan.restate([(i, len(x), 0, i, cc + 1) for i, ((cc, _), x) in enumerate(zip(steps, lists))], c)
    assert any(r0[2] * 16 >= r0[3] for r0, _ in segs)  # some segment holds extra pages only

    meta = AttentionMetadata.build([SeqStep(cc, n, list(b)) for cc, n, b in wl.seqs], wl.block_size, DEV)
    pk8, pv8 = exp_k.clone(), exp_v.clone()  # the pools after this step's append (checked by fp8_step)
    q = wl.q.to(DEV)
    kv_indptr = torch.tensor([0] + [sum(len(x) for x in lists[:i + 1]) for i in range(len(lists))],
                             dtype=torch.int32, device=DEV)
    kv_indices = torch.tensor([b for x in lists for b in x], dtype=torch.int32, device=DEV)
    total = sum(len(x) for x in lists)
    n_rec, n_merge = decode_plan_size(total, len(lists), c)
    dec = torch.full((4 * n_rec,), -1, dtype=torch.int32, device=DEV)
    mrg = torch.full((4 * n_merge,), -1, dtype=torch.int32, device=DEV)
    lib = _native.lib()
    st = _native.stream_ptr(DEV)
    lib.call("mllm_plan", meta.qo_indptr.data_ptr(), kv_indptr.data_ptr(), meta.seq_lens_i32.data_ptr(), len(lists),
             c, 64, dec.data_ptr(), n_rec, _ptr(mrg), n_merge, 0, 0, st)
    ws = torch.empty(lib.workspace_bytes(n_rec, h, 128), dtype=torch.uint8, device=DEV)
    out = torch.full_like(q, float("nan"))
    nb, bs, _, dh = pk8.shape
    lib.call("mllm_paged_decode_fp8", q.data_ptr(), q.stride(0), q.stride(1), pk8.data_ptr(), pv8.data_ptr(), nb, bs,
             h, hkv, dh, meta.qo_indptr.data_ptr(), kv_indptr.data_ptr(), kv_indices.data_ptr(),
             meta.seq_lens_i32.data_ptr(), dec.data_ptr(), n_rec, _ptr(mrg), n_merge, c, dh ** -0.5,
             _native.dtype_code(q.dtype), ks, vs, out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(),
             ws.numel(), st)
    lib.call("mllm_merge_splits", _ptr(mrg), n_merge, n_rec, h, dh, meta.qo_indptr.data_ptr(),
             _native.dtype_code(q.dtype), out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), ws.numel(), st)
    torch.cuda.synchronize()
    assert dec[0].item() == -(-total // c)
    assert torch.isfinite(out).all()
    torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def test_random_shapes_sweep(hip):
    # 24 seeded steps over the whole shape space at once: 1-8 KV heads, 1-16 query heads per KV head, block
    # sizes 16-128, 1-160 rows of decode and prefill rows, bf16 or fp8 pools (a third); each case is named
    # before it runs
    import random

    from harness import hip_step, oracle_step

    for i in range(24):
        rng = random.Random(90000 + i)
        hkv = rng.choice([1, 2, 4, 8])
        g = rng.choice([1, 2, 4, 8] + ([16] if hkv <= 4 else []))
        bs = rng.choice([16, 32, 64, 128])
        fp8 = rng.random() < 0.35
        steps = [(rng.randrange(0, rng.choice([20, 400, 3000])), 1 if rng.random() < 0.6 else rng.randrange(2, 300))
                 for _ in range(rng.randrange(1, 160))]
        nb = sum(-(-(c + n) // bs) for c, n in steps) + 4
        print(f"sweep case {i}: h={hkv * g} hkv={hkv} bs={bs} fp8={fp8} rows={len(steps)}", flush=True)
        wl = _kernel_case(h=hkv * g, hkv=hkv, bs=bs, steps=steps, num_blocks=nb, seed=i)
        if fp8:
            _check(*fp8_step(wl, rng.uniform(0.02, 0.5), rng.uniform(0.02, 0.5)))
        else:
            out, pk, pv, _ = hip_step(wl, DEV)
            ref, rk, rv = oracle_step(wl, DEV)
            assert torch.equal(bits(pk), bits(rk)) and torch.equal(bits(pv), bits(rv))
            torch.testing.assert_close(out.float(), ref.float(), atol=ATOL, rtol=RTOL)


def _owned_slots(wl, include_new=True):
    used = torch.zeros(wl.num_blocks * wl.block_size, dtype=torch.bool)
    for c, n, blocks in wl.seqs:
        for p in range(c + n if include_new else c):
            used[blocks[p // wl.block_size] * wl.block_size + p % wl.block_size] = True
    return used


def test_every_code_and_subnormals(hip):
    # the cached context cycles through every finite e4m3fn code (K and V offset differently); the
    # second case holds only subnormal codes under a large scale, where a flushed subnormal would show
    steps = [(0, 37), (90, 1), (40, 25), (300, 1), (129, 130)]
    finite = torch.tensor([c for c in range(256) if c & 0x7F != 0x7F], dtype=U8)
    subnormal = torch.tensor([c | s for c in range(1, 8) for s in (0, 0x80)], dtype=U8)
    for codes, ks, vs in [(finite, 2.0 ** -6, 2.0 ** -6), (subnormal, 2.0 ** 7, 2.0 ** 8)]:
        wl = _kernel_case(steps=steps, num_blocks=64)

        def fill(pk8, pv8, codes=codes):
            n = pk8.numel()
            idx = torch.arange(n, device=DEV)
            cd = codes.to(DEV)
            _u8(pk8).view(-1)[:] = cd[idx % len(cd)]
            _u8(pv8).view(-1)[:] = cd[(idx * 7 + 3) % len(cd)]

        _check(*fp8_step(wl, ks, vs, fill))


@pytest.mark.parametrize("name", ["decode_4", "mixed_128"])
def test_slots_a_row_does_not_own_never_matter(hip, name):
    # NaN (0x7F / 0xFF) and the largest codes in every slot no row owns leave the output bit-identical
    from minillm import workloads

    wl = workloads.WORKLOADS[name]()
    owned = _owned_slots(wl).to(DEV)
    outs = []
    for code in (0x00, 0x7E, 0x7F, 0xFF):
        def fill(pk8, pv8, code=code):
            for p in (pk8, pv8):
                flat = _u8(p).view(-1, wl.hkv * wl.dh)
                flat[~owned] = code

        outs.append(fp8_step(wl, 0.05, 0.03, fill)[0])
    for o in outs[1:]:
        assert torch.equal(bits(o), bits(outs[0]))


def test_fp8_is_closer_to_bf16_than_its_tolerance(hip):
    # the same step on a bf16 pool and on an fp8 pool of the same values: quantization moves the output
    # by about the e4m3 step (2^-4 relative), well inside what attention on this data tolerates
    from minillm import workloads
    from harness import hip_step

    wl = workloads.mixed_128()
    out16, *_ = hip_step(wl, DEV)
    out8, *_ = fp8_step(wl, 1.0, 1.0)
    err = (out8.float() - out16.float()).abs()
    assert err.max().item() < 0.5 and err.mean().item() < 0.05


def test_scale_and_dtype_errors(hip):
    from minillm import workloads
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    wl = workloads.decode_4()
    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    be = get_backend("hip")
    q, k, v = wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV)
    pk8 = torch.zeros(wl.pool_k.shape, dtype=torch_ref.FP8, device=DEV)
    pv8 = torch.zeros_like(pk8)
    with pytest.raises(ValueError, match="positive"):
        be.forward(q, k, v, pk8, pv8, meta, k_scale=0.0)
    with pytest.raises(ValueError, match="positive"):
        be.forward(q, k, v, pk8, pv8, meta, v_scale=float("inf"))
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        be.forward(q.float(), k.float(), v.float(), pk8, pv8, meta)
    pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
    with pytest.raises(ValueError, match="fp8 pools only"):
        be.forward(q, k, v, pk, pv, meta, k_scale=2.0)
    with pytest.raises(ValueError, match="share one dtype"):
        be.forward(q, k, v, pk8, pv, meta)
    torch.cuda.synchronize()
