"""The `hip` attention backend: minillm's paged hot path on gfx950 kernels.

Drop-in for the reference's backends (src/minillm/attention/torch_ref.py:46-48,
flashinfer_backend.py:42-64, flash_attn_backend.py:107-115): same `forward(q, k, v, k_cache, v_cache,
meta)` and `prefill(q, k, v, key_valid)` contract, same pool layout, same metadata object.

Per layer, `forward` issues on the current stream:
1. `mllm_kv_append`     the step's k/v into the pool at `meta.slot_mapping` (bit-exact write_kv);
2. `mllm_paged_decode`  split-KV decode for rows with one new token, then `mllm_merge_splits`;
3. `mllm_paged_prefill` MFMA prefill for rows with several new tokens.
A work plan (`mllm_plan`) is built on the GPU the first time a given `meta` is seen and reused by the
other layers, like FlashInfer's plan()/run() split (flashinfer_backend.py:44).  Nothing synchronises
the host, and there is no fallback: a missing library raises RuntimeError at construction.

A pool of dtype torch.float8_e4m3fn (the reference's planned fp8 KV cache, M9b in
docs/distributed_inference_plan.md:310) selects the `_fp8` entry points: the append stores
e4m3fn(x * (1 / scale)) and attention reads value * scale, with per-tensor `k_scale` / `v_scale` passed
to `forward`; q, k, v and the output stay bf16 / fp16.
"""

from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass

import torch

from .. import _native
from .base import AttentionBackend
from .metadata import decode_plan_size

FULL_CHIP_CUS = 256  # MI355X: 8 XCDs x 32 CUs
MAX_SPLIT_PAGES = 192  # pages one decode bin may hold (the kernels keep a segment's page ids in 3 registers)
_CUS: dict = {}


def device_cus(device=None) -> int:
    """Compute units of the device the kernels run on (torch's multi_processor_count, read once per device):
    a partitioned or smaller device holds fewer resident wavefronts, so the decode bins grow to match."""
    if device is None or not torch.cuda.is_available():
        return FULL_CHIP_CUS
    index = torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    cus = _CUS.get(index)
    if cus is None:
        cus = _CUS[index] = int(torch.cuda.get_device_properties(index).multi_processor_count)
    return cus


WHOLE_PAGE_WAVES = 8  # KV heads per workgroup of the whole-page decode launch (one workgroup per CU)
WHOLE_PAGE_MIN_SPLIT = 24  # the library launches it from this split size up (kWholePageMinSplit)


def whole_page(kv_fp8: bool, num_kv_heads: int, split: int) -> bool:
    """Whether mllm_paged_decode runs its whole-page workgroups for this split size (the library's rule)."""
    return not kv_fp8 and num_kv_heads % WHOLE_PAGE_WAVES == 0 and split >= WHOLE_PAGE_MIN_SPLIT


def decode_waves(num_heads: int, num_kv_heads: int, kv_fp8: bool, num_cus: int = FULL_CHIP_CUS) -> tuple[int, int]:
    """(resident wavefronts of the decode kernel on the device, wavefronts one bin takes): CUs x 4 SIMDs x 3
    per SIMD for the 16-bit 4-wavefront kernel, one per KV head; 2 per SIMD for the fp8 kernels, one per two
    KV heads when they pair up (decode_kernel_name), else one per KV head.  The fp8 one-head kernel's bins
    are one round of these."""
    if not kv_fp8:
        return num_cus * 4 * 3, num_kv_heads
    if decode_kernel_name(True, num_heads, num_kv_heads) == "decode_pair_kernel":
        return num_cus * 4 * 2, num_kv_heads // 2
    return num_cus * 4 * 2, num_kv_heads


SMALL_BIN_PAGES = 16  # the 4-wavefront launch adds workgroups per CU before its bins grow past this
MIN_SPLIT_PAGES = 2  # the smallest bin the heuristic picks (16-bit pools)


def pages_per_split(decode_pages: int, num_kv_heads: int, num_heads: int | None = None, kv_fp8: bool = False,
                    num_cus: int = FULL_CHIP_CUS, whole_pages: bool = True) -> int:
    """Pages per decode bin for a step of `decode_pages` decode pages on a device of `num_cus` CUs.

    16-bit pools with KV heads in groups of 8 (`whole_pages`): one whole-page workgroup per CU, Hkv / 8 per
    bin, so bins of ceil(T / (rounds x bins per round)) pages, at most 192 (two rounds past 192 x 256 pages).
    That is 134 pages on the 256-row decode workload: 255 bins, 341.7 us against 349.6 us for 383 bins of 89
    pages in 4-wavefront workgroups (with 257 bins of 133 pages, one bin past a round, 554 us).

    Below WHOLE_PAGE_MIN_SPLIT the library runs 4-wavefront workgroups (4 KV heads each, up to 3 per CU).
    Their bins are sized so that no CU gets more than k workgroups: with B = CUs / ceil(Hkv / 4) bins per
    workgroup round, bins of ceil(T / (k B)) pages, k the fewest (at most 3, all resident) that keeps them
    within SMALL_BIN_PAGES, and at least MIN_SPLIT_PAGES.  A CU given one workgroup more than the others
    finishes a bin's time later, and more workgroups per CU than needed only add bins.  Measured on MI355X (append +
    decode + merge per layer, Llama-3.1-8B heads): 8 to 32 rows of 16-64 pages (T = 128-512) 11.6-14.7 us
    against 14.6-17.7 us with the previous floor of 8 pages; 256 rows of 16 pages and 64 of 64 (T = 4,096)
    46.5-48.8 us at 16 pages against 55.2-59.1 us at 11; 32 rows of U[128, 4096] tokens (T = 3,895) 50.8 us
    against 53.5 us.  Bins that give some CUs one workgroup more measured slower: T = 1,024 at 6 pages
    (342 workgroups) 24.0 us against 18.3 us at 8 (256).
    fp8 pools whose KV heads pair up run the pair kernel, whose workgroups (4 wavefronts of two KV heads)
    also cover 8 KV heads: their bins are sized like whole pages, one workgroup per CU and round, at least
    MIN_SPLIT_PAGES at any size.  One per CU measured faster than two (the previous rule): decode_256 177.7
    against 183.3 us (134 against 67 pages a bin), mixed_128's decode 166.4 against 172.6 us, ragged steps
    of 3,895-25,773 pages 4-13% faster, steps of 128-1,024 pages 12.2-16.9 against 16.6-18.5 us.  The fp8
    one-head kernel keeps one round of its resident wavefronts, at least 8 pages.  `whole_pages=False`
    gives the 4-wavefront sizing whatever the step (16-bit pools)."""
    forced = os.environ.get("MLLM_PAGES_PER_SPLIT")
    if forced:
        return max(1, min(MAX_SPLIT_PAGES, int(forced)))
    if whole_pages and not kv_fp8 and num_kv_heads % WHOLE_PAGE_WAVES == 0 and decode_pages > 0:
        per_round = max(1, num_cus // (num_kv_heads // WHOLE_PAGE_WAVES))
        rounds = math.ceil(decode_pages / (MAX_SPLIT_PAGES * per_round))
        split = math.ceil(decode_pages / (rounds * per_round))
        if split >= WHOLE_PAGE_MIN_SPLIT:
            return split
    if kv_fp8 and decode_kernel_name(True, num_heads or 4 * num_kv_heads, num_kv_heads) == "decode_pair_kernel":
        per_round = max(1, num_cus // -(-num_kv_heads // WHOLE_PAGE_WAVES))
        rounds = max(1, math.ceil(decode_pages / (MAX_SPLIT_PAGES * per_round)))
        return max(MIN_SPLIT_PAGES, min(MAX_SPLIT_PAGES, math.ceil(decode_pages / (rounds * per_round))))
    if not kv_fp8:
        per_round = max(1, num_cus // -(-num_kv_heads // 4))
        per_cu = min(3, max(1, math.ceil(decode_pages / (per_round * SMALL_BIN_PAGES))))
        return max(MIN_SPLIT_PAGES, min(MAX_SPLIT_PAGES, math.ceil(decode_pages / (per_round * per_cu))))
    slots, per_bin = decode_waves(num_heads or 4 * num_kv_heads, num_kv_heads, kv_fp8, num_cus)
    return max(8, min(MAX_SPLIT_PAGES, math.ceil(decode_pages * per_bin / slots)))


def decode_records_bound(max_pages: int, rows: int, num_kv_heads: int, num_heads: int | None = None,
                         kv_fp8: bool = False, num_cus: int = FULL_CHIP_CUS, pad_pages: int = 0) -> int:
    """The most decode plan records a step of `rows` rows and at most `max_pages` decode pages needs at the
    bin size pages_per_split picks for its page count (plus `pad_pages` pages of padding rows, which do not
    change that size)."""
    best = 0
    for t in range(1, max_pages + 1):
        c = pages_per_split(t, num_kv_heads, num_heads, kv_fp8, num_cus)
        best = max(best, decode_plan_size(t + pad_pages, rows, c)[0])
    return best


PREFILL_ROWS = 256  # (token, head) rows of a prefill workgroup of 8 wavefronts (one per CU)
PREFILL_ROWS_SMALL = 128  # rows of a 4-wavefront workgroup (two per CU: 16-bit pools)
SMALL_PREFILL_PER_CU = 4  # 8-wavefront workgroups per CU up to which 4-wavefront ones are used instead


def prefill_q_tile(num_new: list[int], group: int, num_kv_heads: int, kv_fp8: bool = False,
                   num_cus: int = FULL_CHIP_CUS) -> int:
    """New tokens per prefill work item: PREFILL_ROWS / group for 8-wavefront workgroups, or
    PREFILL_ROWS_SMALL / group for 4-wavefront ones, two of which share a CU so that one's prologue and
    output drain run under the other's main loop.  A step takes the small items when the large ones would
    give each CU at most SMALL_PREFILL_PER_CU workgroups.  Measured on MI355X (prefill launch,
    Llama-3.1-8B heads): mixed_128 (2.2 large workgroups per CU) 70.7 against 79.1-79.9 us, on an fp8
    pool 79.2 against 84.5-86.4 us; steps of 4-32 rows of 512-2048 new tokens at 1-4 per CU 2-15%
    faster; prefix_64 (9.8 per CU) 2% slower on either pool, and rows of 256 new tokens over 1,024
    cached at 8 and 16 per CU 11% and 26% slower (twice the K/V re-reads per FLOP).  MLLM_PREFILL_ROWS
    (256 or 128) forces either size.  Group sizes that do not divide 32 have no prefill kernel (the entry
    point rejects them)."""
    if 32 % group:
        return 1
    forced = os.environ.get("MLLM_PREFILL_ROWS")
    if forced:
        small = int(forced) == PREFILL_ROWS_SMALL
    else:
        items = sum(-(-nn // (PREFILL_ROWS // group)) for nn in num_new if nn > 1)
        small = items * num_kv_heads <= SMALL_PREFILL_PER_CU * num_cus
    return (PREFILL_ROWS_SMALL if small else PREFILL_ROWS) // group


class PlanOverflowError(RuntimeError):
    """A decode plan did not fit the capacities it was given (its header reads {0, records, merges, -1})."""


def check_plan_header(decode_work: torch.Tensor) -> None:
    """Reads a decode plan's header back (one host synchronisation) and raises PlanOverflowError when the
    step did not fit: the plan then holds no decode work, and the decode rows' outputs would stay unwritten."""
    if decode_work.numel() < 4:
        return
    nb, records, merges, flag = decode_work[:4].tolist()
    if flag == -1:
        raise PlanOverflowError(f"decode plan overflow: the step needs {records} records and {merges} merges, "
                                f"more than the capacities the plan was given")


@dataclass
class StepPlan:
    """Work lists of one step (device int32 buffers) and their sizes."""

    pages_per_split: int
    q_tile: int
    num_decode: int  # int4 records of the decode plan (its capacity)
    num_merge: int
    num_prefill: int
    decode_work: torch.Tensor
    merge_work: torch.Tensor
    prefill_work: torch.Tensor
    workspace_bytes: int
    # the step's fixed pointer arguments, taken once per plan instead of once per layer: the metadata's
    # qo_indptr, kv_indptr, kv_indices, seq_lens_i32, then the work lists and their sizes
    meta_ptrs: tuple = ()
    decode_args: tuple = ()
    # the mllm_layer_step of mllm_attention_forward, built on the plan's first layer call and rebuilt when
    # the pools' shape, the dtypes or the workspace change
    layer_key: tuple | None = None
    layer_step: object = None
    layer_addr: int = 0


def _ptr(t: torch.Tensor | None) -> int:
    return 0 if t is None or t.numel() == 0 else t.data_ptr()


FP8 = torch.float8_e4m3fn


def decode_kernel_name(kv_fp8: bool, num_heads: int, num_kv_heads: int) -> str:
    """The decode kernel mllm_paged_decode(_fp8) launches: fp8 pools pair adjacent KV heads in one wavefront
    when the KV heads are even and a pair's query heads fit 16 MFMA columns."""
    pair = kv_fp8 and num_kv_heads % 2 == 0 and 2 * (num_heads // num_kv_heads) <= 16
    return "decode_pair_kernel" if pair else "decode_kernel"


def prefill_kernel_name(kv_fp8: bool, q_tile_rows: int = 256) -> str:
    """The prefill kernel mllm_paged_prefill(_fp8) launches for items of `q_tile_rows` (token, head) rows:
    8-wavefront workgroups with phases of two 64-key tiles, or 4-wavefront workgroups, two per CU, for
    128-row items (on fp8 pools both pass tiles through registers to be widened on their way into LDS)."""
    del kv_fp8
    return "prefill4w_kernel" if q_tile_rows == PREFILL_ROWS_SMALL else "prefill128_kernel"


def is_fp8(pool: torch.Tensor) -> bool:
    return pool.dtype == FP8


class HipBackend(AttentionBackend):
    name = "hip"
    # The model hands q and k to `forward_rotary` before RoPE when this is set (LlamaAttention checks it),
    # so the rotation runs in the KV-append launch; False gives the reference call sequence.
    fuse_rotary = True
    # When set, a step with decode rows and multi-token rows runs the prefill launch on a second stream
    # beside the decode launch; their outputs are disjoint rows of `out`.  Off by default: the decode
    # launch is one round of equal bins that keeps every SIMD busy until it ends, so the prefill's
    # workgroups (a whole CU each) find no room beside it.  On mixed_128, one box: 410.8 us one after the
    # other, 412.8 us overlapped with decode enqueued first, 413.5 us with prefill first.
    overlap_mixed = False
    # When set, every plan build reads the plan's header back (one host synchronisation) and raises
    # PlanOverflowError if the decode plan did not fit its capacities; for tests and debugging.
    check_plan = os.environ.get("MLLM_CHECK_PLAN", "") not in ("", "0")

    def __init__(self) -> None:
        self._lib = _native.lib()
        self._attention_forward = self._lib.fn("mllm_attention_forward")
        self._planned = None  # the AttentionMetadata the plan was last built for
        self._planned_fp8 = False  # and the pool type it was built for
        self._plan: StepPlan | None = None
        self._workspace: torch.Tensor | None = None
        self._side: dict = {}  # device -> the stream mixed steps run their prefill launch on

    # ------------------------------------------------------------------ paged path

    def forward(self, q, k, v, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0):
        q, k, v = self._check(q, k, v, k_cache, v_cache, meta, k_scale, v_scale)
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        if self._split_launches(q, k_cache, meta):
            self.append(k, v, k_cache, v_cache, meta, k_scale, v_scale)
            self.attend(q, k_cache, v_cache, meta, out, k_scale, v_scale)
        else:
            self.run_layer(q, k, v, k_cache, v_cache, meta, out, k_scale=k_scale, v_scale=v_scale)
        return out

    def _split_launches(self, q, k_cache, meta) -> bool:
        """Whether this layer runs as separate calls: only a mixed step with `overlap_mixed` set, whose
        prefill goes to a second stream."""
        if not self.overlap_mixed:
            return False
        plan = self.plan(meta, q.shape[1], k_cache.shape[2], q.shape[2], q.device, is_fp8(k_cache))
        return bool(plan.num_decode and plan.num_prefill) and not torch.cuda.is_current_stream_capturing()

    def run_layer(self, q, k, v, k_cache, v_cache, meta, out, cos=None, sin=None, q_rot=None,
                  k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        """The layer's whole path in one host call (mllm_attention_forward): KV append (with cos and sin, the
        RoPE of q and k fused into it and the rotated q written to q_rot), decode + merge, prefill, on the
        current stream.  The arguments are the checked ones of `forward` / `forward_rotary`; q_rot and out
        are contiguous [N, H, Dh]."""
        fp8 = is_fp8(k_cache)
        plan = self.plan(meta, q.shape[1], k_cache.shape[2], q.shape[2], q.device, fp8)
        step = self._layer_step(plan, meta, q, k_cache, fp8)
        rot = cos is not None
        self._lib.check(self._attention_forward(
            step, q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(),
            v.stride(0), v.stride(1), cos.data_ptr() if rot else None, sin.data_ptr() if rot else None,
            cos.stride(0) if rot else 0, q_rot.data_ptr() if rot else None, k_cache.data_ptr(), v_cache.data_ptr(),
            k_scale, v_scale, out.data_ptr(), _native.stream_ptr(q.device)))

    def _layer_step(self, plan: StepPlan, meta, q, k_cache, fp8: bool) -> int:
        """Address of the plan's mllm_layer_step for these pools and this workspace."""
        ws = self._workspace
        key = (k_cache.shape[0], k_cache.shape[1], q.dtype, fp8, ws.data_ptr() if ws is not None else 0)
        if plan.layer_key == key:
            return plan.layer_addr
        ws = self._workspace_for(plan.workspace_bytes, q.device)
        num_blocks, bs, hkv, dh = k_cache.shape
        step = _native.LayerStep(
            num_blocks=num_blocks, num_tokens=q.shape[0], slot_mapping=meta.slot_mapping.data_ptr(),
            qo_indptr=plan.meta_ptrs[0], kv_indptr=plan.meta_ptrs[1], kv_indices=plan.meta_ptrs[2],
            seq_lens=plan.meta_ptrs[3], decode_work=_ptr(plan.decode_work), merge_work=_ptr(plan.merge_work),
            prefill_work=_ptr(plan.prefill_work), workspace=_ptr(ws), workspace_bytes=plan.workspace_bytes,
            num_decode_work=plan.num_decode, num_merge_work=plan.num_merge, num_prefill_work=plan.num_prefill,
            pages_per_split=plan.pages_per_split, q_tile_tokens=plan.q_tile, num_heads=q.shape[1],
            num_kv_heads=hkv, head_dim=dh, block_size=bs, dtype=_native.dtype_code(q.dtype), kv_fp8=int(fp8),
            softmax_scale=dh ** -0.5)
        plan.layer_step, plan.layer_addr = step, ctypes.addressof(step)
        plan.layer_key = (num_blocks, bs, q.dtype, fp8, ws.data_ptr() if ws is not None else 0)
        return plan.layer_addr

    def _check(self, q, k, v, k_cache, v_cache, meta, k_scale=1.0, v_scale=1.0):
        n, h, dh = q.shape
        if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
            raise ValueError("k_cache and v_cache must both be [num_blocks, block_size, Hkv, Dh]")
        _, bs, hkv, dh_c = k_cache.shape
        if k.shape != (n, hkv, dh) or v.shape != (n, hkv, dh) or dh_c != dh:
            raise ValueError(f"k/v must be [N, Hkv, Dh] = [{n}, {hkv}, {dh}] to match q and the pool")
        if bs != meta.block_size:
            raise ValueError(f"pool block size {bs} != metadata block size {meta.block_size}")
        if h % hkv:
            raise ValueError("num_heads must be a multiple of num_kv_heads")
        if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
            raise ValueError("the KV pools must be contiguous")
        if v_cache.dtype != k_cache.dtype:
            raise ValueError("k_cache and v_cache must share one dtype")
        if is_fp8(k_cache):
            if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
                raise ValueError("with an fp8 pool, q, k and v must share one dtype, bfloat16 or float16")
            if not (0 < k_scale < math.inf and 0 < v_scale < math.inf):
                raise ValueError("k_scale and v_scale must be positive and finite")
        else:
            if q.dtype != k_cache.dtype:
                raise ValueError("q and the pools must share one dtype")
            if k_scale != 1.0 or v_scale != 1.0:
                raise ValueError("k_scale / v_scale apply to fp8 pools only")
        if n != meta.query_start_loc[-1]:
            raise ValueError(f"q has {n} tokens, the metadata describes {meta.query_start_loc[-1]}")
        return tuple(t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))

    def forward_rotary(self, q, k, v, cos, sin, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0):
        """`forward` with the model's RoPE folded in: q and k arrive before the rotation (reference
        src/minillm/model/llama.py:110 applies it right before the backend call), with the step's
        cos / sin rows [N, Dh].  One launch rotates q and k, appends the rotated k and v to the pool and
        writes the rotated q, bit for bit what apply_rotary followed by `forward` produces."""
        q, k, v = self._check(q, k, v, k_cache, v_cache, meta, k_scale, v_scale)
        if self._split_launches(q, k_cache, meta):
            q_rot = self.rope_append(q, k, v, cos, sin, k_cache, v_cache, meta, k_scale, v_scale)
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
            self.attend(q_rot, k_cache, v_cache, meta, out, k_scale, v_scale)
            return out
        n, h, dh = q.shape
        if cos.shape != (n, dh) or sin.shape != (n, dh):
            raise ValueError(f"cos and sin must be [N, Dh] = [{n}, {dh}]")
        if cos.dtype != q.dtype or sin.dtype != q.dtype:
            raise ValueError("q, cos, sin and the pools must share one dtype (or the pools be fp8)")
        if cos.stride(-1) != 1 or sin.stride() != cos.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        q_rot = torch.empty((n, h, dh), dtype=q.dtype, device=q.device)
        out = torch.empty((n, h, dh), dtype=q.dtype, device=q.device)
        self.run_layer(q, k, v, k_cache, v_cache, meta, out, cos, sin, q_rot, k_scale, v_scale)
        return out

    def rope_append(self, q, k, v, cos, sin, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0):
        """Rotary embedding of q and k plus the KV append (`mllm_rope_kv_append`); returns the rotated q."""
        n, h, dh = q.shape
        num_blocks, bs, hkv, _ = k_cache.shape
        if cos.shape != (n, dh) or sin.shape != (n, dh):
            raise ValueError(f"cos and sin must be [N, Dh] = [{n}, {dh}]")
        if cos.dtype != q.dtype or sin.dtype != q.dtype or not (k_cache.dtype == q.dtype or is_fp8(k_cache)):
            raise ValueError("q, cos, sin and the pools must share one dtype (or the pools be fp8)")
        if cos.stride(-1) != 1 or sin.stride() != cos.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        q_rot = torch.empty((n, h, dh), dtype=q.dtype, device=q.device)
        args = (q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(),
                v.stride(0), v.stride(1), cos.data_ptr(), sin.data_ptr(), cos.stride(0), h, hkv, dh,
                _native.dtype_code(q.dtype), q_rot.data_ptr(), q_rot.stride(0), q_rot.stride(1), k_cache.data_ptr(),
                v_cache.data_ptr(), num_blocks * bs, meta.slot_mapping.data_ptr(), n)
        if is_fp8(k_cache):
            self._lib.call("mllm_rope_kv_append_fp8", *args, k_scale, v_scale, _native.stream_ptr(q.device))
        else:
            self._lib.call("mllm_rope_kv_append", *args, _native.stream_ptr(q.device))
        return q_rot

    def append(self, k, v, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        """KV append (reference write_kv, paged_torch_ref.py:23-28): one launch for K and V."""
        num_blocks, bs, hkv, dh = k_cache.shape
        if is_fp8(k_cache):
            self._lib.call("mllm_kv_append_fp8", k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                           v.stride(1), _native.dtype_code(k.dtype), k_cache.data_ptr(), v_cache.data_ptr(),
                           num_blocks * bs, hkv, dh, meta.slot_mapping.data_ptr(), k.shape[0], k_scale, v_scale,
                           _native.stream_ptr(k_cache.device))
            return
        self._lib.call("mllm_kv_append", k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0),
                       v.stride(1), _native.dtype_code(k.dtype), k_cache.data_ptr(), v_cache.data_ptr(),
                       _native.dtype_code(k_cache.dtype), num_blocks * bs, hkv, dh, meta.slot_mapping.data_ptr(),
                       k.shape[0], _native.stream_ptr(k_cache.device))

    def detach_workspace(self) -> torch.Tensor | None:
        """Hands the decode workspace to the caller and starts a new one on the next use (a captured HIP
        graph keeps the buffer it recorded, whatever later eager steps allocate)."""
        ws, self._workspace = self._workspace, None
        return ws

    def invalidate_plan(self) -> None:
        """Forget the cached plan: the next layer builds one even for a `meta` it has seen (HIP-graph
        capture records that build, so every replay re-plans from the staged metadata)."""
        self._planned = None

    def plan(self, meta, num_heads: int, num_kv_heads: int, head_dim: int, device, kv_fp8: bool = False) -> StepPlan:
        """The step's work plan, built on the GPU once per `meta` object (and pool type) and reused after."""
        if self._planned is not meta or self._planned_fp8 != kv_fp8:
            self._make_plan(meta, num_heads, num_kv_heads, head_dim, device, _native.stream_ptr(device), kv_fp8)
        return self._plan

    def attend(self, q, k_cache, v_cache, meta, out, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        """Attention of every new token over its row's context in the pool, written into `out`."""
        plan = self.plan(meta, q.shape[1], k_cache.shape[2], q.shape[2], q.device, is_fp8(k_cache))
        if plan.num_decode and plan.num_prefill and self.overlap_mixed and not torch.cuda.is_current_stream_capturing():
            # decode is enqueued first; the prefill's workgroups take CUs as the decode's free up
            cur = torch.cuda.current_stream(q.device)
            side = self._side.get(q.device)
            if side is None:
                side = self._side[q.device] = torch.cuda.Stream(q.device)  # default priority
            ready = cur.record_event()  # the append (and everything before it) has landed
            self.run_decode(q, k_cache, v_cache, meta, out, k_scale, v_scale)
            self.run_merge(q, meta, out)
            side.wait_event(ready)
            with torch.cuda.stream(side):
                self.run_prefill(q, k_cache, v_cache, meta, out, k_scale, v_scale)
            cur.wait_stream(side)  # nothing after attend runs before the prefill rows are written
            return
        if plan.num_decode:
            self.run_decode(q, k_cache, v_cache, meta, out, k_scale, v_scale)
            self.run_merge(q, meta, out)
        if plan.num_prefill:
            self.run_prefill(q, k_cache, v_cache, meta, out, k_scale, v_scale)

    def run_decode(self, q, k_cache, v_cache, meta, out, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        """Split-KV decode of the rows with one new token (reference paged_torch_ref.py:47-59)."""
        plan = self._plan
        num_blocks, bs, hkv, dh = k_cache.shape
        ws = self._workspace_for(plan.workspace_bytes, q.device)
        args = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, bs,
                q.shape[1], hkv, dh, *plan.decode_args, dh ** -0.5, _native.dtype_code(q.dtype))
        tail = (out.data_ptr(), out.stride(0), out.stride(1), _ptr(ws), plan.workspace_bytes,
                _native.stream_ptr(q.device))
        if is_fp8(k_cache):
            self._lib.call("mllm_paged_decode_fp8", *args, k_scale, v_scale, *tail)
        else:
            self._lib.call("mllm_paged_decode", *args, *tail)

    def run_merge(self, q, meta, out) -> None:
        """Log-sum-exp merge of the decode rows that were split."""
        plan = self._plan
        if not plan.num_merge:
            return
        self._lib.call("mllm_merge_splits", _ptr(plan.merge_work), plan.num_merge, plan.num_decode, q.shape[1],
                       q.shape[2], plan.meta_ptrs[0], _native.dtype_code(q.dtype), out.data_ptr(),
                       out.stride(0), out.stride(1), _ptr(self._workspace), plan.workspace_bytes,
                       _native.stream_ptr(q.device))

    def run_prefill(self, q, k_cache, v_cache, meta, out, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
        """MFMA attention of the rows with several new tokens (reference paged_torch_ref.py:61-73)."""
        plan = self._plan
        num_blocks, bs, hkv, dh = k_cache.shape
        args = (q.data_ptr(), q.stride(0), q.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), num_blocks, bs,
                q.shape[1], hkv, dh, *plan.meta_ptrs, _ptr(plan.prefill_work), plan.num_prefill, plan.q_tile,
                dh ** -0.5, _native.dtype_code(q.dtype))
        tail = (out.data_ptr(), out.stride(0), out.stride(1), _native.stream_ptr(q.device))
        if is_fp8(k_cache):
            self._lib.call("mllm_paged_prefill_fp8", *args, k_scale, v_scale, *tail)
        else:
            self._lib.call("mllm_paged_prefill", *args, *tail)

    def _make_plan(self, meta, h: int, hkv: int, dh: int, dev, stream: int, kv_fp8: bool = False) -> None:
        news, lens, bs = meta.num_new, meta.seq_lens, meta.block_size
        pages = [-(-length // bs) for length in lens]
        decode_pages = sum(p for p, nn in zip(pages, news) if nn == 1)
        # a graph-captured step (StaticDecodeMetadata) stages its split size on the device; the
        # capacities then cover the smallest split it may stage
        split_dev = getattr(meta, "split_dev", None)
        c = meta.split_min if split_dev is not None else pages_per_split(decode_pages, hkv, h, kv_fp8, device_cus(dev))
        g = h // hkv
        q_tile = prefill_q_tile(news, g, hkv, kv_fp8, device_cus(dev))
        decode_rows = sum(1 for nn in news if nn == 1)
        n_dec, n_merge = decode_plan_size(decode_pages, decode_rows, c)
        if split_dev is not None:  # a captured step sized for fewer records than its worst case
            n_dec = min(n_dec, meta.decode_records_cap)
        n_pf = sum(-(-nn // q_tile) for nn in news if nn > 1)
        buf = torch.full((4 * n_dec + 4 * n_merge + 8 * n_pf,), -1, dtype=torch.int32, device=dev)
        dec, mrg, pf = buf[:4 * n_dec], buf[4 * n_dec:4 * (n_dec + n_merge)], buf[4 * (n_dec + n_merge):]
        if split_dev is not None:
            self._lib.call("mllm_plan_dev", meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(),
                           meta.seq_lens_i32.data_ptr(), meta.num_seqs, split_dev.data_ptr(), c, q_tile, _ptr(dec),
                           n_dec, _ptr(mrg), n_merge, _ptr(pf), n_pf, stream)
        else:
            self._lib.call("mllm_plan", meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(),
                           meta.seq_lens_i32.data_ptr(), meta.num_seqs, c, q_tile, _ptr(dec), n_dec, _ptr(mrg), n_merge,
                           _ptr(pf), n_pf, stream)
        ws = self._lib.workspace_bytes(n_dec, h, dh) if n_merge else 0
        meta_ptrs = (meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(), meta.kv_indices.data_ptr(),
                     meta.seq_lens_i32.data_ptr())
        self._plan = StepPlan(c, q_tile, n_dec, n_merge, n_pf, dec, mrg, pf, ws, meta_ptrs,
                              (*meta_ptrs, _ptr(dec), n_dec, _ptr(mrg), n_merge, c))
        self._planned, self._planned_fp8 = meta, kv_fp8
        if self.check_plan and n_dec and not torch.cuda.is_current_stream_capturing():
            check_plan_header(dec)

    def _workspace_for(self, nbytes: int, dev) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        if self._workspace is None or self._workspace.numel() < nbytes or self._workspace.device != dev:
            self._workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        return self._workspace

    # ------------------------------------------------------------------ contiguous path

    def prefill(self, q, k, v, key_valid=None, **kwargs):
        b, h, tq, dh = q.shape
        bk, hkv, tk, dhk = k.shape
        if v.shape != k.shape or bk != b or dhk != dh:
            raise ValueError("k and v must be [B, Hkv, Tk, Dh] matching q [B, H, Tq, Dh]")
        if tk < tq:
            raise ValueError("Tk must be >= Tq")
        if not (q.dtype == k.dtype == v.dtype):
            raise ValueError("q, k and v must share one dtype")
        q, k, v = (t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v))
        out = torch.empty((b, h, tq, dh), dtype=q.dtype, device=q.device)
        kv_ptr, kv_sb, kv_st = 0, 0, 0
        if key_valid is not None:
            if key_valid.shape != (b, tk):
                raise ValueError(f"key_valid must be [B, Tk] = [{b}, {tk}]")
            key_valid = key_valid.to(device=q.device, dtype=torch.bool).contiguous().view(torch.uint8)
            kv_ptr, kv_sb, kv_st = key_valid.data_ptr(), key_valid.stride(0), key_valid.stride(1)
        self._lib.call("mllm_dense_attention", q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), k.data_ptr(),
                       k.stride(0), k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
                       kv_ptr, kv_sb, kv_st, b, h, hkv, tq, tk, dh, dh ** -0.5, _native.dtype_code(q.dtype),
                       out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), _native.stream_ptr(q.device))
        return out
