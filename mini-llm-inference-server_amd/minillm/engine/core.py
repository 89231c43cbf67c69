"""Engine core: scheduler + paged pool + model, one unit of GPU work per step
(reference src/minillm/engine/core.py:56-180; IPC, HTTP and text live outside this package).

`step()`: schedule -> build the step's AttentionMetadata on the GPU (shared by every layer) -> one
model forward over the ragged new tokens with the pool -> greedy argmax of each sequence's last
token -> bookkeeping.  The attention backend is whatever the model was built with (`hip` by default).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import torch

from ..attention.metadata import AttentionMetadata, DeviceBlockTables, SeqStep
from ..cache.paged import BLOCK_SIZE, PagedKVCache
from ..cache.prefix import PrefixCache, root_hash
from .block_manager import BlockManager
from .scheduler import Request, Scheduler

DEFAULT_MAX_NUM_BATCHED_TOKENS = 8192


@dataclass
class AddRequest:
    req_id: str
    prompt_token_ids: list[int]
    max_tokens: int
    stop_token_ids: list[int] = field(default_factory=list)
    ignore_eos: bool = False
    timeline: dict = field(default_factory=dict)
    cache_salt: str = ""


@dataclass
class RequestOutput:
    req_id: str
    new_token_ids: list[int]
    finished: bool = False
    finish_reason: str | None = None
    timeline: dict | None = None
    num_prompt_tokens: int = 0
    num_output_tokens: int = 0
    num_cached_tokens: int = 0


@dataclass
class EngineStats:
    num_waiting: int
    num_running: int
    kv_tokens_used: int
    kv_blocks_used: int = 0
    kv_blocks_total: int = 0
    num_preemptions: int = 0
    kv_blocks_cached: int = 0
    prefix_cache_queries: int = 0
    prefix_cache_hits: int = 0


@dataclass
class StepOutputs:
    outputs: list[RequestOutput]
    stats: EngineStats


@dataclass
class StepRecord:
    step: int
    t_start: int
    duration_ns: int
    num_seqs: int
    prefill_tokens: int
    decode_tokens: int
    kv_tokens_used: int
    queue_len: int
    kv_blocks_used: int = 0
    num_preempted: int = 0


def now_ns() -> int:
    return time.monotonic_ns()


class EngineCore:
    def __init__(self, model, max_model_len: int | None = None, step_log: bool = False, max_batch_size: int = 1,
                 max_num_batched_tokens: int | None = None, num_kv_blocks: int | None = None,
                 enable_prefix_caching: bool = True, model_id: str = "unknown", metadata_builder=None,
                 chunked_prefill: bool = False, kv_cache_dtype: torch.dtype | None = None,
                 kv_scales: tuple[float, float] = (1.0, 1.0), decode_graphs=None) -> None:
        """The step's metadata comes from a device-resident mirror of the block tables (DeviceBlockTables:
        only new block ids travel each step); `metadata_builder(seqs, block_size, device)` replaces that with
        another implementation of the same contract (AttentionMetadata.build uploads every table; a test
        passes the oracle's).  `chunked_prefill` mixes
        decode rows and prompt chunks in one step under the token budget (see Scheduler).
        `kv_cache_dtype` defaults to the model's dtype; torch.float8_e4m3fn gives an fp8 pool whose K and
        V tensors of every layer use the per-tensor scales `kv_scales` (k_scale, v_scale).
        `decode_graphs` (True, or a tuple of batch buckets) runs pure decode steps as captured HIP graphs
        (DecodeGraphs); prefill and mixed steps stay eager."""
        self.model = model
        self.build_metadata = metadata_builder
        p = next(model.parameters())
        self.device, self.dtype = p.device, p.dtype
        self.max_model_len = max_model_len or model.config.max_position_embeddings
        self.max_batch_size = max_batch_size
        if num_kv_blocks is None:
            num_kv_blocks = max_batch_size * -(-self.max_model_len // BLOCK_SIZE)
        self.kv_dtype = kv_cache_dtype or self.dtype
        self.cache = PagedKVCache(model.config, num_kv_blocks, self.device, self.kv_dtype, k_scale=kv_scales[0],
                                  v_scale=kv_scales[1])
        self.prefix = PrefixCache() if enable_prefix_caching else None
        self.blocks = BlockManager(num_kv_blocks, BLOCK_SIZE, self.prefix)
        self.scheduler = Scheduler(max_batch_size, max_num_batched_tokens or DEFAULT_MAX_NUM_BATCHED_TOKENS,
                                   self.blocks, self.prefix, chunked_prefill=chunked_prefill)
        self._salt_keys = {"block_size": BLOCK_SIZE, "kv_dtype": str(self.kv_dtype).removeprefix("torch."),
                           "layout": "NHD", "model": model_id}
        if self.cache.quantized:  # the stored bytes depend on the scales too
            self._salt_keys["kv_scales"] = [kv_scales[0], kv_scales[1]]
        self.tables = None
        if metadata_builder is None:
            self.tables = DeviceBlockTables(max_batch_size, -(-self.max_model_len // BLOCK_SIZE), self.device)
        self.graphs = None
        if decode_graphs:
            from .graphs import DEFAULT_BUCKETS, DecodeGraphs

            if self.tables is None:
                raise ValueError("decode graphs read the resident block tables: leave metadata_builder unset")
            buckets = DEFAULT_BUCKETS if decode_graphs is True else tuple(decode_graphs)
            self.graphs = DecodeGraphs(model, self.cache, self.tables, BLOCK_SIZE, buckets)
        self.step_log: list[StepRecord] | None = [] if step_log else None
        self._step = 0
        self._aborted: list[RequestOutput] = []

    def add_request(self, msg: AddRequest) -> None:
        if not msg.prompt_token_ids:
            raise ValueError("empty prompt")
        total = len(msg.prompt_token_ids) + msg.max_tokens
        if total > self.max_model_len:
            raise ValueError(f"prompt + max_tokens exceeds max_model_len {self.max_model_len}")
        if self.blocks.blocks_for(total) > self.blocks.num_blocks:
            raise ValueError(f"prompt + max_tokens needs more KV blocks than the pool has ({self.blocks.num_blocks})")
        timeline = dict(msg.timeline)
        timeline["queued"] = now_ns()
        stop = frozenset() if msg.ignore_eos else frozenset(msg.stop_token_ids)
        root = root_hash({**self._salt_keys, "salt": msg.cache_salt}) if self.prefix is not None else b""
        self.scheduler.add(Request(msg.req_id, list(msg.prompt_token_ids), msg.max_tokens, stop, timeline,
                                   root=root))

    def abort(self, req_id: str) -> None:
        req = next((r for r in self.scheduler.running if r.req_id == req_id), None)
        if req is not None:
            self.scheduler.finish([req])
            self._release(req)
        else:
            req = self.scheduler.remove_waiting(req_id)
            if req is None:
                return
        self._aborted.append(self._finish(req, [], "abort"))

    def has_work(self) -> bool:
        s = self.scheduler
        return bool(s.running or s.waiting or self._aborted)

    def stats(self) -> EngineStats:
        s = self.scheduler
        return EngineStats(num_waiting=len(s.waiting), num_running=len(s.running),
                           kv_tokens_used=sum(r.num_cached for r in s.running),
                           kv_blocks_used=self.blocks.num_blocks - self.blocks.num_free,
                           kv_blocks_total=self.blocks.num_blocks, num_preemptions=s.num_preemptions,
                           kv_blocks_cached=self.blocks.num_cached,
                           prefix_cache_queries=self.prefix.queries if self.prefix else 0,
                           prefix_cache_hits=self.prefix.hits if self.prefix else 0)

    def check_blocks(self) -> None:
        self.blocks.check([r.block_ids for r in self.scheduler.running])

    @torch.inference_mode()
    def step(self) -> StepOutputs:
        outputs, self._aborted = self._aborted, []
        t0 = now_ns()
        plan = self.scheduler.schedule()
        for r in plan.preempted:
            self._release(r)
        rows = plan.rows()
        if not rows:
            return StepOutputs(outputs, self.stats())
        reqs = [r for r, _ in rows]
        for r in plan.prefill:
            r.timeline.setdefault("scheduled", t0)
        new = [r.uncached()[:n] for r, n in rows]
        seqs = [SeqStep(r.num_cached, len(n), r.block_ids) for r, n in zip(reqs, new)]
        if self.graphs is not None and not plan.prefill and self.graphs.supports(len(seqs)):
            tokens = self.graphs.run(reqs, seqs, [n[0] for n in new])
        else:
            if self.tables is not None:
                meta = self.tables.build(reqs, seqs, BLOCK_SIZE)
            else:
                meta = self.build_metadata(seqs, BLOCK_SIZE, self.device)
            ids = torch.tensor([[t for n in new for t in n]], device=self.device)
            logits = self.model(ids, kv_cache=self.cache.step(meta), last_index=meta.logits_index)
            tokens = logits[:, -1].argmax(dim=-1).tolist()
        t_tok = now_ns()
        done = []
        for req, n, token in zip(reqs, new, tokens):
            if req.num_cached + len(n) < req.num_tokens:  # a prompt chunk short of the end: nothing sampled
                req.num_cached += len(n)
                continue
            req.num_cached = req.num_tokens
            req.output.append(token)
            req.timeline.setdefault("first_token", t_tok)
            if token in req.stop_ids or len(req.output) >= req.max_tokens:
                done.append(req)
                outputs.append(self._finish(req, [token], "stop" if token in req.stop_ids else "length"))
            else:
                outputs.append(RequestOutput(req.req_id, [token]))
        self.scheduler.name_full_blocks(reqs)
        self.scheduler.finish(done)
        for r in done:
            self._release(r)
        if self.step_log is not None:
            st = self.stats()
            self.step_log.append(StepRecord(self._step, t0, now_ns() - t0, len(reqs),
                                            sum(plan.chunks[r] for r in plan.prefill), len(plan.decode),
                                            st.kv_tokens_used, st.num_waiting, st.kv_blocks_used,
                                            len(plan.preempted)))
        self._step += 1
        return StepOutputs(outputs, self.stats())

    def _release(self, req: Request) -> None:
        """The request left the running set: its resident table row is free again."""
        if self.tables is not None:
            self.tables.release(req)

    def _finish(self, req: Request, new_tokens: list[int], reason: str) -> RequestOutput:
        req.timeline["finished"] = now_ns()
        return RequestOutput(req.req_id, new_tokens, finished=True, finish_reason=reason, timeline=req.timeline,
                             num_prompt_tokens=len(req.prompt), num_output_tokens=len(req.output),
                             num_cached_tokens=req.num_cached_tokens or 0)
