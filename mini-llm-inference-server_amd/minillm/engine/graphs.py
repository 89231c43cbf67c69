"""HIP-graph capture of decode steps (the reference's planned M8, "CUDA graphs for decode":
docs/distributed_inference_plan.md:309; the plan-once/run-per-layer split it relies on is FlashInfer's,
src/minillm/attention/flashinfer_backend.py:44).

A decode step launches about fifteen kernels per layer; at small batch the host's work to launch them
exceeds the GPU's time.  For each batch bucket B, `DecodeGraphs` captures everything a decode step does
after the scheduler has picked its rows into one HIP graph over fixed device buffers:
  the metadata build (mllm_build_metadata), the work plan (a -1 fill and mllm_plan), the model forward
  (embedding, 32 x {RMSNorm, QKV GEMM, fused RoPE + KV append, split-KV decode + merge, o_proj, MLP}),
  lm_head on the B last positions and the greedy argmax.
A step then costs the host one packed upload of (num_cached, num_new, block tables), one input-id copy,
one graph launch and the read of B token ids.

The graph is captured with fixed sizes.  A row may hold up to ceil(max_model_len / block_size) blocks;
the decode plan's capacity of a B-row bucket covers every step of up to the fewer pages of B rows at that
length and the whole pool plus one page per row (without prefix sharing, a step's pages never exceed the
pool), each at the split size the host heuristic picks for its page count.  Each replay stages the split size an eager step of the same rows would
use (mllm_plan_dev reads it on the device), so a replayed step runs the same decode work as the eager
one; a step whose plan at that size exceeds the bucket's capacity (rows sharing prefix pages can) is
not replayed but run eagerly (`fits`).  Every replay fills the plan buffers with -1 before planning,
and the decode and merge launches cover the capacity: workgroups past the step's own bins and merges
exit at once.  Rows past the step's own are padding (see StaticDecodeMetadata).  All buckets share one decode
workspace, sized for the largest: replays run one at a time on the engine's stream.
Only pure decode steps run as graphs; prefill and mixed steps run eagerly.
"""

from __future__ import annotations

import torch

from ..attention.hip_backend import MAX_SPLIT_PAGES, decode_records_bound, device_cus, pages_per_split
from ..attention.metadata import DeviceBlockTables, SeqStep, StaticDecodeMetadata, decode_plan_size

DEFAULT_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128)


class _Captured:
    def __init__(self, static: StaticDecodeMetadata, ids: torch.Tensor, pinned_ids: torch.Tensor) -> None:
        self.static, self.ids, self.pinned_ids = static, ids, pinned_ids
        self.ids_uploaded = torch.cuda.Event()  # the last copy out of pinned_ids
        self.graph: torch.cuda.CUDAGraph | None = None
        self.workspace: torch.Tensor | None = None  # the decode workspace the graph recorded
        self.logits: torch.Tensor | None = None  # [B, V] of the last replay
        self.tokens: torch.Tensor | None = None  # [B] greedy ids of the last replay


class DecodeGraphs:
    """Captured decode steps of `model` over `cache`, one graph per bucket, captured on first use."""

    def __init__(self, model, cache, tables: DeviceBlockTables, block_size: int, buckets=DEFAULT_BUCKETS) -> None:
        backend = model.model.layers[0].self_attn.backend
        if not hasattr(backend, "invalidate_plan"):
            raise ValueError("decode graphs need the hip attention backend")
        self.model, self.cache, self.backend, self.tables = model, cache, backend, tables
        self.block_size = block_size
        self.buckets = tuple(sorted(set(int(b) for b in buckets)))
        self.device = next(model.parameters()).device
        self.num_kv_heads = model.config.num_key_value_heads
        self.num_heads = model.config.num_attention_heads
        self.head_dim = model.config.head_dim
        self._captured: dict[int, _Captured] = {}
        self._capacity: dict[int, int] = {}
        self._pool = None
        self._workspace: torch.Tensor | None = None  # shared by every bucket's graph
        self.replays = 0
        self.eager_fallbacks = 0
        self.last_bucket: int | None = None

    def supports(self, num_rows: int) -> bool:
        return 0 < num_rows <= self.buckets[-1]

    def bucket(self, num_rows: int) -> int:
        return next(b for b in self.buckets if b >= num_rows)

    def capacity(self, bucket: int) -> int:
        """Decode plan records the bucket's plan holds: the most any step of `bucket` rows needs (padding rows
        included) at the split size the heuristic picks for its pages, over steps of up to its rows at
        max_model_len or the whole pool plus one page per row, whichever is fewer pages.  The captured decode
        launch covers that many bins, so a bound tighter than every page count at the smallest split keeps
        the replays' grids small."""
        cap = self._capacity.get(bucket)
        if cap is None:
            pages = min(bucket * self.tables.max_blocks, self.cache.num_blocks + bucket)
            cap = self._capacity[bucket] = decode_records_bound(
                pages, bucket, self.num_kv_heads, self.num_heads, self.cache.quantized, device_cus(self.device),
                pad_pages=bucket)
        return cap

    def fits(self, seqs: list[SeqStep]) -> bool:
        """Whether the decode step `seqs` can replay a graph: a bucket holds its rows, and its decode plan at
        the split size it would stage fits that bucket's plan."""
        if not self.supports(len(seqs)):
            return False
        b = self.bucket(len(seqs))
        pages = sum(-(-(s.num_cached + 1) // self.block_size) for s in seqs)
        c = max(StaticDecodeMetadata.SPLIT_MIN, min(MAX_SPLIT_PAGES, self._split(pages)))
        records, _ = decode_plan_size(pages + (b - len(seqs)), b, c)  # padding rows hold one page each
        if records <= self.capacity(b):
            return True
        self.eager_fallbacks += 1
        return False

    def run(self, keys, seqs: list[SeqStep], token_ids: list[int]) -> tuple[torch.Tensor, torch.Tensor]:
        """One decode step: `seqs` are the rows (one new token each, its id in `token_ids`), `keys` their
        requests' keys in the resident tables.  Returns the rows' logits [rows, vocab] and greedy next
        tokens [rows], views of the graph's output buffers (valid until its next replay)."""
        n = len(seqs)
        b = self.bucket(n)
        c = self.captured(b)
        self._stage(c, keys, seqs, token_ids)
        c.graph.replay()
        self.replays += 1
        self.last_bucket = b
        return c.logits[:n], c.tokens[:n]

    def captured(self, bucket: int) -> _Captured:
        if bucket not in self._captured:
            self._captured[bucket] = self._capture(bucket)
        return self._captured[bucket]

    # ------------------------------------------------------------------ internals

    def _split(self, pages: int) -> int:
        """The split size an eager step over `pages` decode pages uses with this pool.  A replay cuts the same
        bins, so its output is the eager step's bit for bit; its decode launch, planned at the smallest
        split, runs 4-wavefront workgroups over them (the launch shape does not change a wavefront's
        arithmetic)."""
        return pages_per_split(pages, self.num_kv_heads, self.num_heads, self.cache.quantized,
                               device_cus(self.device))

    def _stage(self, c: _Captured, keys, seqs: list[SeqStep], token_ids: list[int]) -> None:
        bs = self.block_size
        pages = sum(-(-(s.num_cached + 1) // bs) for s in seqs)
        c.static.load(keys, seqs, self._split(pages))  # the eager step's split size
        # the previous step's copy out of the same pinned memory may still be queued behind its replay
        # (a sampler need not wait for the GPU): let it run before the host rewrites the ids
        c.ids_uploaded.synchronize()
        ids = c.pinned_ids.numpy()
        ids[:len(token_ids)] = token_ids
        ids[len(token_ids):] = 0
        c.ids.copy_(c.pinned_ids.view(1, -1), non_blocking=True)
        c.ids_uploaded.record()

    def _body(self, c: _Captured):
        """The captured work: metadata build, then the forward (whose first layer builds the plan)."""
        c.static.build()
        self.backend.invalidate_plan()
        meta = c.static.meta
        logits = self.model(c.ids, kv_cache=self.cache.step(meta), last_index=meta.logits_index)[:, -1]
        return logits, logits.argmax(dim=-1)

    @torch.inference_mode()
    def _capture(self, bucket: int) -> _Captured:
        static = StaticDecodeMetadata(bucket, self.tables, self.block_size, decode_records=self.capacity(bucket))
        c = _Captured(static, torch.zeros((1, bucket), dtype=torch.long, device=self.device),
                      torch.zeros(bucket, dtype=torch.long, pin_memory=True))
        self._stage(c, [], [], [])  # every row padding: a valid step that writes nothing to the pool
        if self._workspace is None:  # sized for the largest bucket's plan: no bucket ever grows it
            nbytes = self.backend._lib.workspace_bytes(self.capacity(self.buckets[-1]), self.num_heads,
                                                       self.head_dim)
            self._workspace = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=self.device)
        # warm-up on a side stream, then capture, with the shared workspace in the backend
        eager_ws = self.backend.detach_workspace()
        self.backend._workspace = self._workspace
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(2):
                self._body(c)
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        c.graph = torch.cuda.CUDAGraph()
        if self._pool is None:
            self._pool = torch.cuda.graph_pool_handle()
        with torch.cuda.graph(c.graph, pool=self._pool):
            c.logits, c.tokens = self._body(c)
        if self.backend.detach_workspace() is not self._workspace:
            raise RuntimeError("the decode workspace was reallocated during capture")
        c.workspace = self._workspace
        self.backend._workspace = eager_ws
        self.backend.invalidate_plan()  # eager steps must not reuse the captured plan buffers
        torch.cuda.synchronize(self.device)
        return c

    def eager_reference(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The last replayed step run again eagerly on the same staged inputs (for tests: the replay must
        equal it).  It appends the same k/v rows at the same slots again."""
        c = self._captured[self.last_bucket]
        with torch.inference_mode():
            eager_ws, self.backend._workspace = self.backend._workspace, c.workspace
            try:
                out = self._body(c)
            finally:
                self.backend._workspace = eager_ws
                self.backend.invalidate_plan()
            return out
