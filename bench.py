#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

Default workload (decode_256): one layer of a ragged decode step of Llama-3.1-8B's attention shape
(32 query / 8 KV heads, head_dim 128, 16-token blocks, bf16) over 256 rows whose cached contexts are
uniform in [128, 4096], one new token each, pool = 2x the pages with a shuffled assignment.  A step
is KV append + split-KV paged decode + split merge, with the step's metadata and work plan built
beforehand (they are built once per engine step and shared by all 32 layers; their cost is reported
separately).  `value` is decode tokens/s of the 32-layer model: 256 / (32 x layer time).

Prints one JSON line with the roofline of the dominant kernel (the decode kernel: algorithmic bytes
per launch / its mean duration from HIP events around each launch in the timed region) and a CPU
baseline: the oracle's restatement of the reference torch backend (gather + SDPA, bf16) timed on this
host's cores on a bounded sample of the same rows.

    python bench.py [--steps K] [--warmup W] [--workload decode_256|decode_4|mixed_128|prefix_64]
    python bench.py --workload engine_8b [--compare-oracle]   # end-to-end engine, random-init Llama-3.1-8B
    python bench.py --workload copy_1gib                      # counter calibration: a 1 GiB device copy
    python bench.py --workload gemm_8192                      # attainable bf16 MFMA rate of a library GEMM
    python bench.py --kv-dtype fp8                            # the same step on an fp8 (e4m3fn) pool

With --kv-dtype fp8 the pool holds the workload's values cast to e4m3fn (scale 1: the N(0, 1) data is
well inside e4m3's range) and the step runs the _fp8 entry points; the algorithmic bytes count one
byte per pool element.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "mini-llm-inference-server_amd"), str(ROOT / "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "ragged paged-attn decode tokens/s + achieved HBM GB/s (% of 8 TB/s), 256 seqs"
HBM_PEAK_GBPS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
LAYERS = 32


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="decode_256")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-rows", type=int, default=16)
    ap.add_argument("--compare-oracle", action="store_true",
                    help="engine_8b: also run the engine with the oracle hot path and compare greedy tokens")
    ap.add_argument("--requests", type=int, default=128)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--unfused-rotary", action="store_true",
                    help="engine_8b: RoPE in torch before the backend call instead of in the KV-append launch")
    ap.add_argument("--chunked-prefill", action="store_true",
                    help="engine_8b: mixed steps (decode rows + prompt chunks under the token budget)")
    ap.add_argument("--max-num-batched-tokens", type=int, default=8192)
    ap.add_argument("--decode-graphs", action="store_true",
                    help="engine_8b: run pure decode steps as captured HIP graphs (batch buckets 1..128)")
    ap.add_argument("--kv-dtype", choices=["bf16", "fp8"], default="bf16",
                    help="KV pool format: bf16 (the reference's) or fp8 e4m3fn with per-tensor scales")
    return ap.parse_args()


def cpu_baseline(wl, rows: int):
    """The oracle (reference torch backend restated: write_kv, gather, SDPA; bf16) on this host's cores
    over the first `rows` rows of the workload, same pool and tensors."""
    import torch

    from harness import oracle_step
    from minillm.workloads import Workload

    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    sel = list(range(min(rows, len(wl.seqs))))
    starts = [0]
    for c, n, _ in wl.seqs:
        starts.append(starts[-1] + n)
    tok = [t for i in sel for t in range(starts[i], starts[i + 1])]
    sub = Workload(wl.name + "_sample", [wl.seqs[i] for i in sel], wl.num_blocks, wl.q[tok], wl.k[tok], wl.v[tok],
                   wl.pool_k, wl.pool_v)
    oracle_step(sub, "cpu", dtype=torch.bfloat16)  # warm-up
    times, t_end = [], time.perf_counter() + 20.0
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 20):
        t0 = time.perf_counter()
        oracle_step(sub, "cpu", dtype=torch.bfloat16)
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    n_tok = len(tok)
    return {"value": n_tok / (LAYERS * t), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first {len(sel)} of {len(wl.seqs)} rows, one layer x {len(times)} reps (median "
                      f"{t * 1e3:.1f} ms), scaled to {LAYERS} layers; effective "
                      f"{sub.algorithmic_bytes() / t / 1e9:.2f} GB/s on the same algorithmic bytes"}


def rotary_append_times(wl, backend, meta, q, k, v, pool_k, pool_v, reps=20):
    """The step right before attention, per layer: the fused RoPE + KV append launch against the
    reference sequence (RoPE of q and k in torch, then the KV-append launch), on the workload's tokens
    taken as pre-RoPE activations at their positions (Llama-3.1-8B rotary table)."""
    import torch

    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import RotaryEmbedding, apply_rotary

    cos, sin = RotaryEmbedding(LlamaConfig(**LLAMA_3_1_8B))(meta.positions[None], q.dtype)
    cos, sin = cos[0], sin[0]

    def fused():
        backend.rope_append(q, k, v, cos, sin, pool_k, pool_v, meta)

    def unfused():
        qr = apply_rotary(q.transpose(0, 1)[None], cos[None], sin[None])
        kr = apply_rotary(k.transpose(0, 1)[None], cos[None], sin[None])
        backend.append(kr[0].transpose(0, 1), v, pool_k, pool_v, meta)
        return qr

    out = {}
    for name, fn in (("fused_us", fused), ("torch_rope_then_append_us", unfused)):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        out[name] = round(a.elapsed_time(b) / reps * 1e3, 2)
    n = q.shape[0]
    moved = (n * q.shape[2] * (2 * q.shape[1] * q.element_size() + 2 * k.shape[1] * k.element_size()
                               + 2 * k.shape[1] * pool_k.element_size()) + 2 * cos.numel() * cos.element_size())
    out["fused_gbps"] = round(moved / (out["fused_us"] * 1e-6) / 1e9, 1)
    out["tokens"] = n
    return out


def bench_engine(args):
    """End-to-end engine on a random-init Llama-3.1-8B (bf16 weights ~ N(0, 0.02), seed 0): `--requests`
    prompts of 256-2048 random tokens, each decoded greedily for `--decode-steps` tokens, continuously
    batched (all requests admitted up to 8192 prompt tokens per prefill step), 16-token blocks, pool
    sized for 90% occupancy.  Reports decode tokens/s over the decode steps (StepRecord durations)."""
    import torch

    from minillm.attention import get_backend
    from minillm.engine.core import AddRequest, EngineCore
    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import LlamaForCausalLM, random_init_

    dev = torch.device("cuda:0")
    cfg = LlamaConfig(**LLAMA_3_1_8B)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    model = model.to_empty(device=dev).to(torch.bfloat16)
    random_init_(model, std=0.02, seed=0)
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(256, 2049, (args.requests,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    blocks = -(-sum(-(-(n + args.decode_steps) // 16) for n in lens) * 10 // 9)

    def run(backend, builder):
        model.set_backend(backend)
        core = EngineCore(model, max_model_len=4096, step_log=True, max_batch_size=args.requests,
                          num_kv_blocks=blocks, enable_prefix_caching=False, metadata_builder=builder,
                          chunked_prefill=args.chunked_prefill, max_num_batched_tokens=args.max_num_batched_tokens,
                          kv_cache_dtype=torch.float8_e4m3fn if args.kv_dtype == "fp8" else None,
                          decode_graphs=args.decode_graphs and backend is hip_backend)
        for i, p in enumerate(prompts):
            core.add_request(AddRequest(f"r{i}", p, args.decode_steps, ignore_eos=True))
        out, margins, last = {}, {}, {}
        hook = model.register_forward_hook(lambda mod, a, o: last.__setitem__("l", o))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while core.has_work():
            step = core.step()
            top2 = last["l"][:, -1].float().topk(2, dim=-1).values
            for o, m in zip(step.outputs, (top2[:, 0] - top2[:, 1]).tolist()):
                out.setdefault(o.req_id, []).extend(o.new_token_ids)
                margins.setdefault(o.req_id, []).append(m)
        wall = time.perf_counter() - t0
        hook.remove()
        dec = [r for r in core.step_log if r.decode_tokens]
        pre = [r for r in core.step_log if r.prefill_tokens]
        generated = sum(len(v) for v in out.values())
        stats = {"decode_tokens_per_s": sum(r.decode_tokens for r in dec) / (sum(r.duration_ns for r in dec) * 1e-9),
                 "output_tokens_per_s": generated / (sum(r.duration_ns for r in core.step_log) * 1e-9),
                 "mixed_steps": sum(1 for r in core.step_log if r.decode_tokens and r.prefill_tokens),
                 "decode_steps": len(dec), "prefill_steps": len(pre),
                 "prefill_tokens_per_s": sum(r.prefill_tokens for r in pre) / (sum(r.duration_ns for r in pre) * 1e-9),
                 "median_decode_step_ms": statistics.median(r.duration_ns for r in dec) * 1e-6,
                 "wall_s": wall, "preemptions": core.stats().num_preemptions}
        del core
        torch.cuda.empty_cache()
        return out, margins, stats

    hip_backend = get_backend("hip")
    hip_backend.fuse_rotary = not args.unfused_rotary
    got, _, st = run(hip_backend, None)  # the engine's default: resident block tables
    line = {"metric": "engine decode tokens/s, random-init Llama-3.1-8B, continuous batching", "unit": "tokens/s",
            "value": round(st["decode_tokens_per_s"], 1), "n_gpus": 1, "higher_is_better": True, "dtype": "bf16",
            "data": "synthetic", "config": {"workload": f"engine_8b: {args.requests} requests, prompts U[256,2048], "
                                                        f"{args.decode_steps} greedy steps, pool {blocks} blocks (90%)",
                                            "rotary": "torch" if args.unfused_rotary else "fused into the KV append",
                                            "scheduling": (f"chunked prefill, {args.max_num_batched_tokens}-token steps"
                                                           if args.chunked_prefill else "prefill-first"),
                                            "kv_dtype": "fp8_e4m3fn (scales 1)" if args.kv_dtype == "fp8" else "bf16",
                                            "decode_steps_as": "HIP graphs" if args.decode_graphs else "eager launches"},
            "engine": {k: round(v, 3) if isinstance(v, float) else v for k, v in st.items()}}
    if args.compare_oracle:
        from oracle_engine import OracleBackend, oracle_metadata

        exp, margins, st_ref = run(OracleBackend(), oracle_metadata)
        same = sum(got[r] == exp[r] for r in exp)
        first_div = []
        for r in exp:
            for j, (a, b) in enumerate(zip(got[r], exp[r])):
                if a != b:
                    first_div.append((j, margins[r][j]))
                    break
        line["oracle_comparison"] = {
            "requests_identical": same, "requests": len(exp),
            "tokens_identical_before_first_divergence": sum(
                next((j for j, (a, b) in enumerate(zip(got[r], exp[r])) if a != b), len(exp[r])) for r in exp),
            "tokens": sum(len(v) for v in exp.values()),
            "divergence_margins": [round(m, 4) for _, m in first_div],
            "oracle_decode_tokens_per_s": round(st_ref["decode_tokens_per_s"], 1)}
    print(json.dumps(line), flush=True)


def copy_calibration():
    """A plain device copy of 1 GiB, three times: the known-size reference against which rocprofv3's
    FETCH_SIZE / WRITE_SIZE counters are scaled when reporting a kernel's HBM traffic."""
    import torch

    x = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_launch": x.numel() * 4, "launches": 3}), flush=True)


def gemm_calibration():
    """The attainable bf16 MFMA rate of a library GEMM on this GPU: torch.mm (hipBLASLt) on 8192^3 bf16
    operands, random N(0, 1) and all-zero (the clock the MFMA stream sustains depends on the data it
    switches), each the mean of 20 launches after 5 warm-up ones."""
    import torch

    n = 8192
    g = torch.Generator(device="cuda:0").manual_seed(0)
    out = {"gemm": f"torch.mm bf16 {n}x{n}x{n}", "peak_tflops": BF16_PEAK_TFLOPS}
    for name in ("random", "zeros"):
        if name == "random":
            a = torch.randn(n, n, generator=g, device="cuda:0", dtype=torch.bfloat16)
            b = torch.randn(n, n, generator=g, device="cuda:0", dtype=torch.bfloat16)
        else:
            a = torch.zeros(n, n, device="cuda:0", dtype=torch.bfloat16)
            b = torch.zeros_like(a)
        for _ in range(5):
            torch.mm(a, b)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch.mm(a, b)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 20
        out[f"{name}_us"] = round(ms * 1e3, 1)
        out[f"{name}_tflops"] = round(2 * n ** 3 / (ms * 1e-3) / 1e12, 1)
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build runs the paged hot path on a single MI355X "
              "(sharding is described, not built); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from minillm import workloads
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, DeviceBlockTables, SeqStep

    if args.workload == "engine_8b":
        return bench_engine(args)
    if args.workload == "copy_1gib":
        return copy_calibration()
    if args.workload == "gemm_8192":
        return gemm_calibration()
    dev = torch.device("cuda:0")
    wl = workloads.WORKLOADS[args.workload]()
    q, k, v = wl.q.to(dev), wl.k.to(dev), wl.v.to(dev)
    pool_k, pool_v = wl.pool_k.to(dev), wl.pool_v.to(dev)
    fp8 = args.kv_dtype == "fp8"
    kv_elem = 1 if fp8 else 2
    ks = vs = 1.0
    if fp8:
        pool_k, pool_v = pool_k.to(torch.float8_e4m3fn), pool_v.to(torch.float8_e4m3fn)
    seqs = [SeqStep(c, n, b) for c, n, b in wl.seqs]
    backend = HipBackend()

    # per-step costs shared by the 32 layers: metadata build (host + GPU) and the GPU work plan, with every
    # table uploaded (AttentionMetadata.build) and from the engine's resident tables in steady state (a
    # step that allocated no new block: only num_cached, num_new and row ids travel)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        meta = AttentionMetadata.build(seqs, wl.block_size, dev)
        backend._planned = None
        backend.plan(meta, wl.h, wl.hkv, wl.dh, dev)
    torch.cuda.synchronize()
    meta_plan_ms = (time.perf_counter() - t0) / 5 * 1e3
    tables = DeviceBlockTables(len(seqs), max(len(s.block_ids) for s in seqs), dev)
    keys = list(range(len(seqs)))
    tables.build(keys, seqs, wl.block_size)  # the first step uploads every table
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(5):
        rmeta = tables.build(keys, seqs, wl.block_size)
        backend._planned = None
        backend.plan(rmeta, wl.h, wl.hkv, wl.dh, dev)
    torch.cuda.synchronize()
    resident_ms = (time.perf_counter() - t0) / 5 * 1e3
    del rmeta
    backend._planned = None
    backend.plan(meta, wl.h, wl.hkv, wl.dh, dev)

    out = torch.empty_like(q)
    plan = backend.plan(meta, wl.h, wl.hkv, wl.dh, dev)

    def step(ev=None):
        backend.append(k, v, pool_k, pool_v, meta, ks, vs)
        if plan.num_decode:
            if ev is not None:
                ev[0].record()
            backend.run_decode(q, pool_k, pool_v, meta, out, ks, vs)
            if ev is not None:
                ev[1].record()
            backend.run_merge(q, meta, out)
        if plan.num_prefill:
            if ev is not None:
                ev[2].record()
            backend.run_prefill(q, pool_k, pool_v, meta, out, ks, vs)
            if ev is not None:
                ev[3].record()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps between two synchronisations; per-launch events around the dominant kernels
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    start.record()
    for i in range(args.steps):
        step(evs[i])
    stop.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - w0) * 1e3
    step_ms = start.elapsed_time(stop) / args.steps
    dec_ms = statistics.mean(e[0].elapsed_time(e[1]) for e in evs) if plan.num_decode else 0.0
    pf_ms = statistics.mean(e[2].elapsed_time(e[3]) for e in evs) if plan.num_prefill else 0.0

    n_rows = len(wl.seqs)
    step_bytes = wl.algorithmic_bytes(kv_elem)
    per_layer_tok_s = wl.num_tokens / (step_ms * 1e-3)
    value = wl.num_tokens / (LAYERS * step_ms * 1e-3)
    if plan.num_decode:
        dec_bytes = wl.decode_kernel_bytes(kv_elem)
        achieved = dec_bytes / (dec_ms * 1e-3) / 1e9
        traffic = None
        tfile = ROOT / "profiles" / f"decode_kernel_{wl.name}{'_fp8' if fp8 else ''}_traffic.json"
        if tfile.exists():
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                    "kernel": "decode_kernel", "algorithmic_bytes": dec_bytes, "mean_us": round(dec_ms * 1e3, 2)}
    else:
        flops = wl.prefill_flops()
        achieved = flops / (pf_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None, "kernel": "prefill_kernel",
                    "algorithmic_flops": flops, "mean_us": round(pf_ms * 1e3, 2)}

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"{wl.name}: one attention layer of Llama-3.1-8B shape (32/8 heads, d=128, block 16,"
                               f" bf16), {n_rows} rows, {wl.num_tokens} new tokens; step = KV append + paged "
                               f"attention (+ split merge); value = tokens/s scaled to {LAYERS} layers",
                   "kv_dtype": "fp8_e4m3fn (scales 1)" if fp8 else "bf16",
                   "rows": n_rows, "new_tokens": wl.num_tokens, "context_tokens": sum(wl.lens),
                   "pages_per_split": plan.pages_per_split, "decode_items": plan.num_decode,
                   "prefill_items": plan.num_prefill},
        "roofline": roofline,
        "per_layer": {"tokens_per_s": round(per_layer_tok_s, 1), "algorithmic_bytes": step_bytes,
                      "hbm_gbps": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
                      "hbm_frac": round(step_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                      "decode_us": round(dec_ms * 1e3, 2), "prefill_us": round(pf_ms * 1e3, 2),
                      "prefill_tflops": round(wl.prefill_flops() / (pf_ms * 1e-3) / 1e12, 1) if pf_ms else None},
        "per_step_shared_ms": {"metadata_build_and_plan": round(meta_plan_ms, 3),
                               "resident_tables_build_and_plan": round(resident_ms, 3)},
        "wall_ms_timed_region": round(wall_ms, 2),
    }
    if plan.num_decode and plan.num_prefill:  # the backend's own mixed step: prefill beside decode
        def ostep():
            backend.append(k, v, pool_k, pool_v, meta, ks, vs)
            backend.attend(q, pool_k, pool_v, meta, out, ks, vs)

        for _ in range(3):
            ostep()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            ostep()
        b.record()
        torch.cuda.synchronize()
        o_ms = a.elapsed_time(b) / args.steps
        line["mixed_overlap"] = {"step_us": round(o_ms * 1e3, 2), "sequential_step_us": round(step_ms * 1e3, 2),
                                 "tokens_per_s": round(wl.num_tokens / (LAYERS * o_ms * 1e-3), 1),
                                 "note": "append, then the prefill launch on a second stream beside decode + merge"}
    line["rotary_append"] = rotary_append_times(wl, backend, meta, q, k, v, pool_k, pool_v)
    if not args.no_cpu_baseline:  # the reference's own format: the oracle on the bf16 pool
        line["cpu_baseline"] = cpu_baseline(wl, args.cpu_sample_rows)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
