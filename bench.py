#!/usr/bin/env python3
"""Benchmark of the paged-attention hot path on one MI355X.

Headline workload (decode_256): one layer of a ragged decode step of Llama-3.1-8B's attention shape
(32 query / 8 KV heads, head_dim 128, 16-token blocks, bf16) over 256 rows whose cached contexts are
uniform in [128, 4096], one new token each, pool = 2x the pages with a shuffled assignment.  A step
is KV append + split-KV paged decode + split merge, issued by one host call per layer
(mllm_attention_forward), with the step's metadata and work plan built beforehand (they are built once per engine step and shared by all 32 layers; their cost is reported
separately, as a median after a warm-up).  `value` is decode tokens/s of the 32-layer model:
256 / (32 x layer time).

The line carries the roofline of the dominant kernel (the decode kernel: algorithmic bytes per launch
over its mean duration from HIP events around each launch in the timed region) and a CPU baseline:
the oracle's restatement of the reference torch backend (write_kv, gather padded to the longest row,
SDPA; bf16) over all 256 rows on this host's cores (torch.set_num_threads(os.cpu_count())), median of
3 runs after a warm-up.  Under "configs" it also carries, from the same run, the other layer
workloads on the GPU with their own kernels' rates and the same CPU baseline:
  decode_4    4 rows (contexts 37/128/211/500 + 1): step and decode-launch time (latency-bound);
  mixed_128   8 prefill + 120 decode rows: prefill launch TFLOP/s and fraction of the bf16 peak over
              its own launch, decode launch GB/s, and the step (append, decode + merge, prefill);
  prefix_64   64 rows over a shared 2,048-token prefix: prefill launch TFLOP/s and fraction;
  decode_256_fp8  the headline step on an fp8 (e4m3fn) pool: decode launch GB/s and fraction;
  gemm_8192   torch.mm (hipBLASLt) on 8192^3 bf16 operands, random and zero: the MFMA rate this GPU
              sustains for a library GEMM; the prefill sub-lines also report their rate against it;
  engine_8b   the end-to-end engine on a random-init Llama-3.1-8B, 128 requests x 256 greedy tokens:
              decode tokens/s over its decode steps.

    python bench.py [--steps K] [--warmup W] [--workload decode_256|decode_4|mixed_128|prefix_64]
    python bench.py --workload engine_8b [--compare-oracle]   # end-to-end engine, random-init Llama-3.1-8B
    python bench.py --workload copy_1gib                      # counter calibration: a 1 GiB device copy
    python bench.py --workload gemm_8192                      # attainable bf16 MFMA rate of a library GEMM
    python bench.py --workload decode_uniform_384x89          # decode_256's bytes in equal rows (no tail)
    python bench.py --kv-dtype fp8                            # the same step on an fp8 (e4m3fn) pool
    python bench.py --workload prefix_64 --no-configs --no-cpu-baseline   # one workload alone (profiling)

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
    ap.add_argument("--no-configs", action="store_true",
                    help="measure only --workload (no decode_4 / mixed_128 / prefix_64 / fp8 sub-lines)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU baseline threads (default: os.cpu_count())")
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


def cpu_model() -> str:
    """The host CPU's model name, as lscpu prints it."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_step_seconds(wl, threads: int, reps: int = 3):
    """The oracle (reference torch backend restated: write_kv, gather padded to the longest decode row,
    SDPA; bf16) over every row of the workload on this host's CPU: median of `reps` runs after one
    warm-up, in seconds per layer, and the run times."""
    import torch

    from harness import oracle_step

    torch.set_num_threads(threads)
    oracle_step(wl, "cpu", dtype=torch.bfloat16)  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        oracle_step(wl, "cpu", dtype=torch.bfloat16)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times


def cpu_threads(args) -> int:
    return args.cpu_threads or os.cpu_count() or 1


def cpu_baseline(wl, args):
    """The CPU baseline of the headline line: every row of the workload, one layer, scaled to 32 layers."""
    threads = cpu_threads(args)
    t, times = cpu_step_seconds(wl, threads)
    return {"value": wl.num_tokens / (LAYERS * t), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"all {len(wl.seqs)} rows of {wl.name}, one layer, median of {len(times)} runs after a "
                      f"warm-up ({', '.join(f'{x * 1e3:.0f}' for x in times)} ms), scaled to {LAYERS} layers",
            "layer_ms": round(t * 1e3, 2), "hbm_gbps_same_bytes": round(wl.algorithmic_bytes() / t / 1e9, 2),
            "os_cpu_count": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "cpu_model": cpu_model()}


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


def engine_8b_model(requests: int, decode_steps: int):
    """A random-init Llama-3.1-8B (bf16 weights ~ N(0, 0.02), seed 0) on cuda:0, `requests` prompts of
    U[256, 2048] random tokens (seed 0), and the pool size for 90% occupancy with `decode_steps` tokens
    each: (model, prompts, blocks)."""
    import torch

    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import LlamaForCausalLM, random_init_

    cfg = LlamaConfig(**LLAMA_3_1_8B)
    with torch.device("meta"):
        model = LlamaForCausalLM(cfg)
    model = model.to_empty(device=torch.device("cuda:0")).to(torch.bfloat16)
    random_init_(model, std=0.02, seed=0)
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(256, 2049, (requests,), generator=g).tolist()
    prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in lens]
    blocks = -(-sum(-(-(n + decode_steps) // 16) for n in lens) * 10 // 9)
    return model, prompts, blocks


def engine_run(model, prompts, blocks, backend, builder, decode_steps: int, chunked_prefill: bool = False,
               max_num_batched_tokens: int = 8192, kv_fp8: bool = False, decode_graphs: bool = False,
               record_margins: bool = False):
    """Every prompt through the engine (continuous batching, 16-token blocks, greedy, ignore EOS) until each
    has `decode_steps` tokens; returns ({req_id: tokens}, {req_id: top-2 logit margins} (with
    `record_margins`, through a sampler that also takes the argmax), stats from the step log)."""
    import torch

    from minillm.engine.core import AddRequest, EngineCore

    margins, pending = {}, {}

    def greedy_with_margins(reqs, logits):
        top2 = logits.float().topk(2, dim=-1).values
        for r, m in zip(reqs, (top2[:, 0] - top2[:, 1]).tolist()):
            pending[r.req_id] = m
        return logits.argmax(dim=-1).tolist()

    model.set_backend(backend)
    core = EngineCore(model, max_model_len=4096, step_log=True, max_batch_size=len(prompts), num_kv_blocks=blocks,
                      enable_prefix_caching=False, metadata_builder=builder, chunked_prefill=chunked_prefill,
                      max_num_batched_tokens=max_num_batched_tokens,
                      kv_cache_dtype=torch.float8_e4m3fn if kv_fp8 else None, decode_graphs=decode_graphs,
                      sampler=greedy_with_margins if record_margins else None)
    for i, p in enumerate(prompts):
        core.add_request(AddRequest(f"r{i}", p, decode_steps, ignore_eos=True))
    out = {}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while core.has_work():
        for o in core.step().outputs:
            out.setdefault(o.req_id, []).extend(o.new_token_ids)
            if record_margins:
                margins.setdefault(o.req_id, []).append(pending[o.req_id])
    wall = time.perf_counter() - t0
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


def bench_engine(args):
    """End-to-end engine on a random-init Llama-3.1-8B (bf16 weights ~ N(0, 0.02), seed 0): `--requests`
    prompts of 256-2048 random tokens, each decoded greedily for `--decode-steps` tokens, continuously
    batched (all requests admitted up to 8192 prompt tokens per prefill step), 16-token blocks, pool
    sized for 90% occupancy.  Reports decode tokens/s over the decode steps (StepRecord durations)."""
    from minillm.attention import get_backend

    model, prompts, blocks = engine_8b_model(args.requests, args.decode_steps)

    def run(backend, builder, record_margins=False):
        return engine_run(model, prompts, blocks, backend, builder, args.decode_steps,
                          chunked_prefill=args.chunked_prefill, max_num_batched_tokens=args.max_num_batched_tokens,
                          kv_fp8=args.kv_dtype == "fp8", decode_graphs=args.decode_graphs and backend is hip_backend,
                          record_margins=record_margins)

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

        exp, margins, st_ref = run(OracleBackend(), oracle_metadata, record_margins=True)
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


def gemm_rates() -> dict:
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
        del a, b
    torch.cuda.empty_cache()
    return out


def gemm_calibration():
    print(json.dumps(gemm_rates()), flush=True)


def shared_step_costs(wl, backend, dev, reps: int = 10):
    """Per-step costs shared by the 32 layers, host + GPU, median of `reps` after one warm-up each:
    the metadata build with every table uploaded (AttentionMetadata.build) plus the GPU work plan, and
    the same from the engine's resident tables in steady state (a step that allocated no new block:
    only num_cached, num_new and row ids travel)."""
    import torch

    from minillm.attention.metadata import AttentionMetadata, DeviceBlockTables, SeqStep

    seqs = [SeqStep(c, n, b) for c, n, b in wl.seqs]
    tables = DeviceBlockTables(len(seqs), max(len(s.block_ids) for s in seqs), dev)
    keys = list(range(len(seqs)))

    def full():
        meta = AttentionMetadata.build(seqs, wl.block_size, dev)
        backend.invalidate_plan()
        backend.plan(meta, wl.h, wl.hkv, wl.dh, dev)

    def resident():
        meta = tables.build(keys, seqs, wl.block_size)
        backend.invalidate_plan()
        backend.plan(meta, wl.h, wl.hkv, wl.dh, dev)

    out = {}
    for name, fn in (("metadata_build_and_plan", full), ("resident_tables_build_and_plan", resident)):
        fn()  # warm-up (the resident path's first call also uploads every table)
        torch.cuda.synchronize()
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            times.append(time.perf_counter() - t0)
        out[name] = round(statistics.median(times) * 1e3, 3)
    out["note"] = f"host + GPU, median of {reps} after a warm-up"
    backend.invalidate_plan()
    return out


def measure_layer(wl, backend, dev, steps: int, warmup: int, fp8: bool):
    """One layer's step on the GPU: KV append, decode + merge and prefill in one host call
    (HipBackend.run_layer, mllm_attention_forward) on the current stream; `warmup` untimed steps, then
    `steps` timed ones between two synchronisations, then the same `steps` again as separate calls with
    HIP events on that stream around every decode and prefill launch (the kernels' own durations; the
    events stay out of the timed steps).  Also times the public `forward` (argument checks and the output
    allocation included) over the same steps."""
    import torch

    from minillm.attention.metadata import AttentionMetadata, SeqStep

    q, k, v = wl.q.to(dev), wl.k.to(dev), wl.v.to(dev)
    pool_k, pool_v = wl.pool_k.to(dev), wl.pool_v.to(dev)
    if fp8:
        pool_k, pool_v = pool_k.to(torch.float8_e4m3fn), pool_v.to(torch.float8_e4m3fn)
    ks = vs = 1.0
    meta = AttentionMetadata.build([SeqStep(c, n, b) for c, n, b in wl.seqs], wl.block_size, dev)
    backend.invalidate_plan()
    plan = backend.plan(meta, wl.h, wl.hkv, wl.dh, dev, fp8)
    out = torch.empty_like(q)

    def step():
        backend.run_layer(q, k, v, pool_k, pool_v, meta, out, k_scale=ks, v_scale=vs)

    def step_events(ev):
        backend.append(k, v, pool_k, pool_v, meta, ks, vs)
        if plan.num_decode:
            ev[0].record()
            backend.run_decode(q, pool_k, pool_v, meta, out, ks, vs)
            ev[1].record()
            backend.run_merge(q, meta, out)
        if plan.num_prefill:
            ev[2].record()
            backend.run_prefill(q, pool_k, pool_v, meta, out, ks, vs)
            ev[3].record()

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        start.record()
        for _ in range(steps):  # no events between the launches
            fn()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / steps, (time.perf_counter() - w0) * 1e3

    step_ms, wall_ms = timed(step)
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for i in range(steps):  # the same steps as separate calls, with HIP events around each launch
        step_events(evs[i])
    torch.cuda.synchronize()
    forward_ms, _ = timed(lambda: backend.forward(q, k, v, pool_k, pool_v, meta, ks, vs))
    return {"wall_ms": wall_ms, "step_ms": step_ms, "forward_ms": forward_ms,
            "dec_ms": statistics.mean(e[0].elapsed_time(e[1]) for e in evs) if plan.num_decode else 0.0,
            "pf_ms": statistics.mean(e[2].elapsed_time(e[3]) for e in evs) if plan.num_prefill else 0.0,
            "plan": plan, "meta": meta, "tensors": (q, k, v, pool_k, pool_v)}


def kernel_rates(wl, r, kv_elem: int) -> dict:
    """Rates of the layer's launches over their own mean durations, against MI355X's published peaks."""
    out = {"step_us": round(r["step_ms"] * 1e3, 2), "tokens": wl.num_tokens, "rows": len(wl.seqs)}
    if r["dec_ms"]:
        gbps = wl.decode_kernel_bytes(kv_elem) / (r["dec_ms"] * 1e-3) / 1e9
        out.update(decode_us=round(r["dec_ms"] * 1e3, 2), decode_bytes=wl.decode_kernel_bytes(kv_elem),
                   decode_gbps=round(gbps, 1), decode_frac_of_8tbps=round(gbps / HBM_PEAK_GBPS, 4))
    if r["pf_ms"]:
        tf = wl.prefill_flops() / (r["pf_ms"] * 1e-3) / 1e12
        out.update(prefill_us=round(r["pf_ms"] * 1e3, 2), prefill_flops=wl.prefill_flops(),
                   prefill_tflops=round(tf, 1), prefill_frac_of_bf16_peak=round(tf / BF16_PEAK_TFLOPS, 4))
        if r.get("plan") is not None:  # which prefill kernel ran: items of 256 or 128 (token, head) rows
            from minillm.attention.hip_backend import prefill_kernel_name

            rows = r["plan"].q_tile * (wl.h // wl.hkv)
            out.update(prefill_kernel=prefill_kernel_name(kv_elem == 1, rows), prefill_rows_per_item=rows)
    out["forward_us"] = round(r["forward_ms"] * 1e3, 2)  # the public forward: checks + allocation + the call
    return out


def engine_subline() -> dict:
    """The end-to-end engine (random-init Llama-3.1-8B, 128 requests x 256 greedy tokens, eager steps) as a
    sub-line of the default run; an error there is reported in the line instead of ending the run."""
    import torch

    from minillm.attention import get_backend

    model = None
    try:
        model, prompts, blocks = engine_8b_model(128, 256)
        _, _, st = engine_run(model, prompts, blocks, get_backend("hip"), None, 256)
        out = {k: round(v, 3) if isinstance(v, float) else v for k, v in st.items()}
        out["workload"] = (f"engine_8b: 128 requests, prompts U[256, 2048], 256 greedy tokens each, pool {blocks} "
                           f"blocks (90% occupancy), prefill-first, RoPE fused into the KV append")
        return out
    except Exception as e:  # noqa: BLE001 - the headline line must still print
        return {"error": f"{type(e).__name__}: {e}"}
    finally:
        del model
        torch.cuda.empty_cache()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build runs the paged hot path on a single MI355X "
              "(sharding is described, not built); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    from minillm import workloads
    from minillm.attention.hip_backend import HipBackend, decode_kernel_name, prefill_kernel_name

    if args.workload == "engine_8b":
        return bench_engine(args)
    if args.workload == "copy_1gib":
        return copy_calibration()
    if args.workload == "gemm_8192":
        return gemm_calibration()
    dev = torch.device("cuda:0")
    wl = workloads.by_name(args.workload)
    fp8 = args.kv_dtype == "fp8"
    kv_elem = 1 if fp8 else 2
    backend = HipBackend()

    shared = shared_step_costs(wl, backend, dev)
    r = measure_layer(wl, backend, dev, args.steps, args.warmup, fp8)
    plan, meta = r["plan"], r["meta"]
    step_ms, dec_ms, pf_ms = r["step_ms"], r["dec_ms"], r["pf_ms"]

    n_rows = len(wl.seqs)
    step_bytes = wl.algorithmic_bytes(kv_elem)
    value = wl.num_tokens / (LAYERS * step_ms * 1e-3)
    if plan.num_decode:
        dec_bytes = wl.decode_kernel_bytes(kv_elem)
        achieved = dec_bytes / (dec_ms * 1e-3) / 1e9
        traffic = None
        kname = decode_kernel_name(fp8, wl.h, wl.hkv)
        tfile = ROOT / "profiles" / f"{kname}_{wl.name}{'_fp8' if fp8 else ''}_traffic.json"
        if tfile.exists():
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic,
                    "kernel": kname, "algorithmic_bytes": dec_bytes, "mean_us": round(dec_ms * 1e3, 2)}
    else:
        flops = wl.prefill_flops()
        achieved = flops / (pf_ms * 1e-3) / 1e12
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None,
                    "kernel": prefill_kernel_name(fp8, r["plan"].q_tile * (wl.h // wl.hkv)),
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
                   "pages_per_split": plan.pages_per_split,
                   "decode_plan": dict(zip(("bins", "segments", "partial_slots"),
                                           plan.decode_work[:3].tolist() if plan.num_decode else (0, 0, 0))),
                   "prefill_items": plan.num_prefill},
        "roofline": roofline,
        "per_layer": {"tokens_per_s": round(wl.num_tokens / (step_ms * 1e-3), 1), "algorithmic_bytes": step_bytes,
                      "hbm_gbps": round(step_bytes / (step_ms * 1e-3) / 1e9, 1),
                      "hbm_frac": round(step_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                      **kernel_rates(wl, r, kv_elem)},
        "per_step_shared_ms": shared,
        "wall_ms_timed_region": round(r["wall_ms"], 2),
    }
    q, k, v, pool_k, pool_v = r["tensors"]
    line["rotary_append"] = rotary_append_times(wl, backend, meta, q, k, v, pool_k, pool_v)
    del r, q, k, v, pool_k, pool_v, meta, plan
    if not args.no_configs:
        # the other layer workloads, on the GPU in this run; each beside the same CPU baseline
        configs = {}
        subs = [(name, False) for name in ("decode_4", "mixed_128", "prefix_64") if name != wl.name]
        if not fp8 and wl.name == "decode_256":
            subs.append(("decode_256", True))
        for name, sub_fp8 in subs:
            swl = wl if name == wl.name else workloads.WORKLOADS[name]()
            sr = measure_layer(swl, backend, dev, args.steps, args.warmup, sub_fp8)
            entry = {"gpu": kernel_rates(swl, sr, 1 if sub_fp8 else 2)}
            del sr
            if not sub_fp8 and not args.no_cpu_baseline:
                t, times = cpu_step_seconds(swl, cpu_threads(args))
                entry["cpu"] = {"layer_ms": round(t * 1e3, 2), "runs_ms": [round(x * 1e3, 1) for x in times],
                                "threads": cpu_threads(args), "kind": "port (oracle, bf16, all rows)",
                                "tokens_per_s_32_layers": round(swl.num_tokens / (LAYERS * t), 2)}
            configs[f"{name}_fp8" if sub_fp8 else name] = entry
            torch.cuda.empty_cache()
        # the MFMA rate a library GEMM reaches on this GPU in the same run: the prefill launches' rates
        # against it as well as against the nominal peak
        gemm = gemm_rates()
        configs["gemm_8192"] = gemm
        for name in ("mixed_128", "prefix_64"):
            gpu = configs.get(name, {}).get("gpu", {})
            if gpu.get("prefill_tflops"):
                gpu["prefill_frac_of_gemm_random"] = round(gpu["prefill_tflops"] / gemm["random_tflops"], 4)
        configs["engine_8b"] = engine_subline()
        line["configs"] = configs
    if not args.no_cpu_baseline:  # the reference's own format: the oracle on the bf16 pool, every row
        line["cpu_baseline"] = cpu_baseline(wl, args)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
