"""Engine core: scheduler + paged pool + model, one unit of GPU work per step.

The reference's engine core (src/minillm/engine/core.py:56-180) fixes what a caller sees: the request and
output messages below (its engine/protocol.py), the request timeline keys ("queued", "scheduled",
"first_token", "finished"), the step log rows, and one forward per step over the ragged new tokens of
every scheduled request.  The code is this build's own, in three phases per step:
  plan    the scheduler picks the rows (request, new tokens) and preempts when the pool is full;
  run     the step's AttentionMetadata is built on the GPU from the resident block tables (shared by
          every layer), the model runs once over the ragged tokens, and each row's last position is
          sampled (greedy argmax unless a `sampler` is given); pure decode steps may replay a captured
          HIP graph instead;
  commit  sampled tokens are appended, finished requests leave, filled blocks are named for the
          prefix cache before any block is released.
The attention backend is whatever the model was built with (`hip` by default).  IPC, HTTP and text
live outside this package.
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
                 kv_scales: tuple[float, float] = (1.0, 1.0), decode_graphs=None, sampler=None) -> None:
        """The step's metadata comes from a device-resident mirror of the block tables (DeviceBlockTables:
        only new block ids travel each step); `metadata_builder(seqs, block_size, device)` replaces that with
        another implementation of the same contract (AttentionMetadata.build uploads every table; a test
        passes the oracle's).  `chunked_prefill` mixes decode rows and prompt chunks in one step under the
        token budget (see Scheduler).  `kv_cache_dtype` defaults to the model's dtype; torch.float8_e4m3fn
        gives an fp8 pool whose K and V tensors of every layer use the per-tensor scales `kv_scales`
        (k_scale, v_scale).  `decode_graphs` (True, or a tuple of batch buckets) runs pure decode steps as
        captured HIP graphs (DecodeGraphs); prefill and mixed steps stay eager.  `sampler(requests,
        logits)` picks each row's next token from its logits [rows, vocab] (default: greedy argmax); a
        row whose prompt chunk stops short of its end ignores its pick."""
        self.model = model
        self.build_metadata = metadata_builder
        self.sampler = sampler
        p = next(model.parameters())
        self.device, self.dtype = p.device, p.dtype
        self.max_model_len = max_model_len or model.config.max_position_embeddings
        self.max_batch_size = max_batch_size
        blocks_per_seq = -(-self.max_model_len // BLOCK_SIZE)
        if num_kv_blocks is None:  # room for every sequence at full length
            num_kv_blocks = max_batch_size * blocks_per_seq
        self.kv_dtype = kv_cache_dtype or self.dtype
        self.cache = PagedKVCache(model.config, num_kv_blocks, self.device, self.kv_dtype, k_scale=kv_scales[0],
                                  v_scale=kv_scales[1])
        self.prefix = PrefixCache() if enable_prefix_caching else None
        self.blocks = BlockManager(num_kv_blocks, BLOCK_SIZE, self.prefix)
        self.scheduler = Scheduler(max_batch_size, max_num_batched_tokens or DEFAULT_MAX_NUM_BATCHED_TOKENS,
                                   self.blocks, self.prefix, chunked_prefill=chunked_prefill)
        # everything besides the tokens that shapes a block's K/V salts the prefix-cache names
        self._salt_keys = {"block_size": BLOCK_SIZE, "kv_dtype": str(self.kv_dtype).removeprefix("torch."),
                           "layout": "NHD", "model": model_id}
        if self.cache.quantized:  # the stored bytes depend on the scales too
            self._salt_keys["kv_scales"] = [kv_scales[0], kv_scales[1]]
        self.tables = DeviceBlockTables(max_batch_size, blocks_per_seq, self.device) if metadata_builder is None \
            else None
        self.graphs = None
        if decode_graphs:
            from .graphs import DEFAULT_BUCKETS, DecodeGraphs

            if self.tables is None:
                raise ValueError("decode graphs read the resident block tables: leave metadata_builder unset")
            buckets = DEFAULT_BUCKETS if decode_graphs is True else tuple(decode_graphs)
            self.graphs = DecodeGraphs(model, self.cache, self.tables, BLOCK_SIZE, buckets)
        self.step_log: list[StepRecord] | None = [] if step_log else None
        self._step = 0
        self._aborted: list[RequestOutput] = []  # reported by the next step

    # ------------------------------------------------------------------ requests in

    def add_request(self, msg: AddRequest) -> None:
        """Queues a request after checking that it can ever run (ValueError otherwise)."""
        n_prompt = len(msg.prompt_token_ids)
        if n_prompt == 0:
            raise ValueError("empty prompt")
        longest = n_prompt + msg.max_tokens
        if longest > self.max_model_len:
            raise ValueError(f"a request of {n_prompt} prompt tokens + max_tokens {msg.max_tokens} does not fit "
                             f"max_model_len {self.max_model_len}")
        if self.blocks.blocks_for(longest) > self.blocks.num_blocks:
            raise ValueError(f"a request of {longest} tokens needs {self.blocks.blocks_for(longest)} KV blocks; "
                             f"the pool has {self.blocks.num_blocks}")
        timeline = {**msg.timeline, "queued": now_ns()}
        root = b"" if self.prefix is None else root_hash({**self._salt_keys, "salt": msg.cache_salt})
        stops = frozenset(() if msg.ignore_eos else msg.stop_token_ids)
        self.scheduler.add(Request(msg.req_id, list(msg.prompt_token_ids), msg.max_tokens, stops, timeline,
                                   root=root))

    def abort(self, req_id: str) -> None:
        """Drops a request wherever it is (a running one releases its blocks now); an unknown id is a
        request that already finished."""
        sched = self.scheduler
        req = next((r for r in sched.running if r.req_id == req_id), None)
        if req is None:
            req = sched.remove_waiting(req_id)
        else:
            sched.finish([req])
            self._release_row(req)
        if req is not None:
            self._aborted.append(self._final_output(req, [], "abort"))

    # ------------------------------------------------------------------ state

    def has_work(self) -> bool:
        return bool(self._aborted) or bool(self.scheduler.running) or bool(self.scheduler.waiting)

    def stats(self) -> EngineStats:
        sched, blocks, prefix = self.scheduler, self.blocks, self.prefix
        return EngineStats(num_waiting=len(sched.waiting), num_running=len(sched.running),
                           kv_tokens_used=sum(r.num_cached for r in sched.running),
                           kv_blocks_used=blocks.num_blocks - blocks.num_free, kv_blocks_total=blocks.num_blocks,
                           num_preemptions=sched.num_preemptions, kv_blocks_cached=blocks.num_cached,
                           prefix_cache_queries=prefix.queries if prefix is not None else 0,
                           prefix_cache_hits=prefix.hits if prefix is not None else 0)

    def check_blocks(self) -> None:
        """Block accounting matches the running requests' tables (AssertionError otherwise)."""
        self.blocks.check([r.block_ids for r in self.scheduler.running])

    def clear_prefix_cache(self) -> None:
        """Names of blocks nobody holds are dropped: an idle engine then has every block free."""
        if self.prefix is not None:
            self.blocks.clear_cache()

    # ------------------------------------------------------------------ the step

    @torch.inference_mode()
    def step(self) -> StepOutputs:
        outputs, self._aborted = self._aborted, []
        t0 = now_ns()
        plan = self.scheduler.schedule()
        for r in plan.preempted:
            self._release_row(r)
        rows = plan.rows()
        if rows:
            for r in plan.prefill:
                r.timeline.setdefault("scheduled", t0)  # a readmitted request keeps its first admission
            tokens = self._run(rows, decode_only=not plan.prefill)
            outputs += self._commit(rows, tokens, now_ns())
            if self.step_log is not None:
                self._log_step(t0, plan, len(rows))
            self._step += 1
        return StepOutputs(outputs, self.stats())

    def _run(self, rows, decode_only: bool) -> list[int]:
        """One forward over the rows' new tokens; one sampled token per row."""
        reqs = [r for r, _ in rows]
        new = [r.uncached()[:n] for r, n in rows]
        seqs = [SeqStep(r.num_cached, len(t), r.block_ids) for r, t in zip(reqs, new)]
        if decode_only and self.graphs is not None and self.graphs.fits(seqs):
            logits, greedy = self.graphs.run(reqs, seqs, [t[0] for t in new])
        else:
            meta = self.tables.build(reqs, seqs, BLOCK_SIZE) if self.tables is not None \
                else self.build_metadata(seqs, BLOCK_SIZE, self.device)
            ids = torch.tensor([[tok for t in new for tok in t]], device=self.device)
            logits = self.model(ids, kv_cache=self.cache.step(meta), last_index=meta.logits_index)[:, -1]
            greedy = None
        if self.sampler is not None:
            return list(self.sampler(reqs, logits))
        return (greedy if greedy is not None else logits.argmax(dim=-1)).tolist()  # waits for the GPU

    def _commit(self, rows, tokens: list[int], t_tokens: int) -> list[RequestOutput]:
        outs: list[RequestOutput] = []
        finished: list[Request] = []
        for (req, n), tok in zip(rows, tokens):
            req.num_cached += n
            if req.num_cached < req.num_tokens:  # a prompt chunk short of its end samples nothing
                continue
            req.output.append(tok)
            req.timeline.setdefault("first_token", t_tokens)
            reason = "stop" if tok in req.stop_ids else "length" if len(req.output) >= req.max_tokens else None
            if reason is None:
                outs.append(RequestOutput(req.req_id, [tok]))
            else:
                finished.append(req)
                outs.append(self._final_output(req, [tok], reason))
        self.scheduler.name_full_blocks([r for r, _ in rows])  # before release: named blocks stay cached
        self.scheduler.finish(finished)
        for req in finished:
            self._release_row(req)
        return outs

    def _log_step(self, t0: int, plan, num_rows: int) -> None:
        st = self.stats()
        self.step_log.append(StepRecord(self._step, t0, now_ns() - t0, num_rows,
                                        sum(plan.chunks[r] for r in plan.prefill), len(plan.decode),
                                        st.kv_tokens_used, st.num_waiting, st.kv_blocks_used, len(plan.preempted)))

    def _release_row(self, req: Request) -> None:
        """The request left the running set: its resident table row is free again."""
        if self.tables is not None:
            self.tables.release(req)

    def _final_output(self, req: Request, new_tokens: list[int], reason: str) -> RequestOutput:
        req.timeline["finished"] = now_ns()
        return RequestOutput(req.req_id, new_tokens, finished=True, finish_reason=reason, timeline=req.timeline,
                             num_prompt_tokens=len(req.prompt), num_output_tokens=len(req.output),
                             num_cached_tokens=req.num_cached_tokens or 0)
