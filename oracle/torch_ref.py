"""Oracle: the torch reference attention, restated.  TEST INFRASTRUCTURE ONLY.

Follows reference `src/minillm/attention/paged_torch_ref.py:23-74` and
`src/minillm/attention/torch_ref.py:20-48` step for step, calling the same torch library routines
(`index_copy_`, advanced-index gather, `F.scaled_dot_product_attention` with `enable_gqa=True`) on the
same shapes, so that its rounding is the reference's own:

- decode rows (one new token) are attended together, gathered to the longest context and masked
  past each row's length (`paged_torch_ref.py:47-59`);
- rows with several new tokens run one at a time, `is_causal=True` when the row is a fresh prompt and
  a bottom-right aligned `tril(length - n)` mask otherwise (`paged_torch_ref.py:61-73`).

Runs on any torch device.  On a GPU, callers pass float32 tensors (the bf16 batched-matmul path of
torch is avoided there), or bf16 tensors with `fused=True`, which pins SDPA to torch's fused
memory-efficient kernel (the reference's torch_ref arithmetic in bf16 on a GPU); on the CPU it runs in
the caller's dtype, exactly as the reference does.

fp8 pools (torch.float8_e4m3fn, the reference's planned fp8 KV cache: docs/distributed_inference_plan.md:310)
hold e4m3fn(x * (1 / scale)) with one scale per tensor: `write_kv` quantizes with torch's own cast and
`paged_attention` reads value * scale.  This part has no reference code to follow; it is pinned by
hand-checked encodings and the e4m3fn grid properties in tests/test_oracle.py.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn.functional as F

from .metadata import OracleMetadata


def torch_meta(meta: OracleMetadata, device) -> SimpleNamespace:
    """The host lists plus the int64 block table on `device`: all `paged_attention` reads."""
    return SimpleNamespace(
        query_start_loc=list(meta.query_start_loc),
        seq_lens=list(meta.seq_lens),
        num_new=meta.num_new,
        block_tables=torch.as_tensor(meta.block_tables, dtype=torch.long, device=device),
        slot_mapping=torch.as_tensor(meta.slot_mapping, dtype=torch.long, device=device),
    )


FP8 = torch.float8_e4m3fn


def inv_scale(scale: float) -> float:
    """1 / scale evaluated in float32 (the value the quantizer multiplies by)."""
    return (torch.tensor(1.0, dtype=torch.float32) / torch.tensor(scale, dtype=torch.float32)).item()


def quantize_fp8(x: torch.Tensor, scale: float) -> torch.Tensor:
    """e4m3fn(float(x) * (1 / scale)): torch's cast rounds to nearest even and stores NaN for magnitudes
    above 464 and for non-finite values."""
    return (x.float() * inv_scale(scale)).to(FP8)


def dequantize_fp8(q: torch.Tensor, scale: float, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    return q.to(dtype) * scale


def write_kv(k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor, k: torch.Tensor,
             v: torch.Tensor, k_scale: float = 1.0, v_scale: float = 1.0) -> None:
    """Reference `paged_torch_ref.py:23-28`: k, v [N, Hkv, Dh] scattered into the flat pool view at
    `slot_mapping` [N] (int64), after a cast to the pool's dtype (the quantizing cast for an fp8 pool)."""
    hkv, dh = k_cache.shape[-2:]
    if k_cache.dtype == FP8:  # torch has no index_copy_ for float8: move the bytes
        k_cache.view(torch.uint8).view(-1, hkv, dh).index_copy_(0, slot_mapping, quantize_fp8(k, k_scale).view(torch.uint8))
        v_cache.view(torch.uint8).view(-1, hkv, dh).index_copy_(0, slot_mapping, quantize_fp8(v, v_scale).view(torch.uint8))
        return
    k_cache.view(-1, hkv, dh).index_copy_(0, slot_mapping, k.to(k_cache.dtype))
    v_cache.view(-1, hkv, dh).index_copy_(0, slot_mapping, v.to(v_cache.dtype))


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Reference `model/llama.py:58-61`: cat(-x2, x1) of the last dim's halves."""
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([-x2, x1], dim=-1)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Reference `model/llama.py:64-72` on the backend's token-major layout: x [N, heads, Dh],
    cos / sin [N, Dh] broadcast over the heads.  Eager torch ops, so on 16-bit tensors each product
    and the sum are rounded to the tensor dtype in turn."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    return x * cos + rotate_half(x) * sin


def rope_then_write_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                       k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                       k_scale: float = 1.0, v_scale: float = 1.0) -> torch.Tensor:
    """The two steps the fused rotary + append replaces: the model's RoPE of q and k
    (`model/llama.py:110`) and `write_kv` of the rotated k and of v.  Returns the rotated q."""
    write_kv(k_cache, v_cache, slot_mapping, apply_rotary(k, cos, sin), v, k_scale, v_scale)
    return apply_rotary(q, cos, sin)


class _Converted:
    """A pool whose gathered rows are converted on the way out (the pool itself is not copied)."""

    def __init__(self, cache: torch.Tensor, conv) -> None:
        self.cache, self.conv, self.shape = cache, conv, cache.shape

    def __getitem__(self, idx):
        return self.conv(self.cache[idx])


def gather(cache: torch.Tensor, block_tables: torch.Tensor, length: int) -> torch.Tensor:
    """Reference `paged_torch_ref.py:31-37`: [num_blocks, bs, Hkv, Dh] through tables [B, nb] ->
    [B, Hkv, length, Dh], the first `length` tokens of every row."""
    b = block_tables.shape[0]
    bs, hkv, dh = cache.shape[1:]
    nb = math.ceil(length / bs)
    tokens = cache[block_tables[:, :nb]].reshape(b, nb * bs, hkv, dh)[:, :length]
    return tokens.transpose(1, 2)


def sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, attn_mask: torch.Tensor | None = None,
         is_causal: bool = False, p_round: torch.dtype | None = None, fused: bool = False) -> torch.Tensor:
    """`F.scaled_dot_product_attention(..., enable_gqa=True)` (scale 1/sqrt(Dh), bottom-right causal
    when `is_causal`: the reference only sets it when Tq == Tk).  With `p_round`, the same mathematics
    written out in q's dtype, with the softmax probabilities rounded to `p_round` before the product with
    V, which is how flash-style bf16 kernels form P.  That variant is not the reference's computation:
    it is the noise-floor reference of bf16 attention arithmetic for end-to-end comparisons.

    With `fused` (GPU tensors), the library SDPA pinned to torch's fused memory-efficient kernel, with
    K/V expanded to one head per query head (that kernel takes no grouped heads; each query head still
    reads its own KV head's values): the reference's torch_ref arithmetic on a GPU in bf16, without the
    math path, whose bf16 batched products are not used here."""
    if fused:
        from torch.nn.attention import SDPBackend, sdpa_kernel

        g = q.shape[1] // k.shape[1]
        k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
        with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal)
    if p_round is None:
        return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal, enable_gqa=True)
    g = q.shape[1] // k.shape[1]
    k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    s = torch.matmul(q, k.transpose(-2, -1)) * (q.shape[-1] ** -0.5)
    tq, tk = s.shape[-2:]
    if is_causal:
        attn_mask = torch.ones(tq, tk, dtype=torch.bool, device=q.device).tril(diagonal=tk - tq)
    if attn_mask is not None:
        s = s.masked_fill(~attn_mask, -math.inf)
    p = torch.softmax(s, dim=-1).to(p_round).to(s.dtype)
    return torch.matmul(p, v)


def paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, meta,
                    compute_dtype: torch.dtype | None = None, k_scale: float = 1.0,
                    v_scale: float = 1.0, p_round: torch.dtype | None = None, fused: bool = False) -> torch.Tensor:
    """Reference `paged_torch_ref.py:40-74`.  q [N, H, Dh] -> [N, H, Dh]; the step's own k/v must
    already be in the pool.  Scale 1/sqrt(Dh); GQA through `enable_gqa`.  With `compute_dtype` the
    gathered context and q are converted to it before SDPA (and the result back to q's dtype): how the
    oracle runs on a GPU, in float32.  An fp8 pool's gathered rows are dequantized (value * scale, in
    `compute_dtype` or q's dtype).  `p_round` selects the rounded-P variant of `sdpa`, `fused` its
    fused-kernel variant."""
    if getattr(k_cache, "dtype", None) == FP8:
        cd = compute_dtype or q.dtype

        def deq(scale):
            return lambda t: dequantize_fp8(t.view(FP8), scale, cd)

        kb, vb = k_cache.view(torch.uint8), v_cache.view(torch.uint8)  # gathered as bytes (no float8 indexing)
        out = paged_attention(q.to(cd), _Converted(kb, deq(k_scale)), _Converted(vb, deq(v_scale)), meta,
                              p_round=p_round, fused=fused)
        return out.to(q.dtype)
    if compute_dtype is not None and compute_dtype != q.dtype:
        orig = q.dtype

        def conv(t):
            return t.to(compute_dtype)

        out = paged_attention(conv(q), _Converted(k_cache, conv), _Converted(v_cache, conv), meta, p_round=p_round,
                              fused=fused)
        return out.to(orig)
    out = torch.empty_like(q)
    starts, lens, news = meta.query_start_loc, meta.seq_lens, meta.num_new

    decode = [i for i, n in enumerate(news) if n == 1]
    if decode:
        rows = torch.tensor(decode, device=q.device)
        longest = max(lens[i] for i in decode)
        k = gather(k_cache, meta.block_tables[rows], longest)
        v = gather(v_cache, meta.block_tables[rows], longest)
        token_idx = torch.tensor([starts[i] for i in decode], device=q.device)
        qd = q[token_idx][:, :, None]
        mask = None
        if any(lens[i] != longest for i in decode):
            ends = torch.tensor([lens[i] for i in decode], device=q.device)
            mask = (torch.arange(longest, device=q.device)[None, :] < ends[:, None])[:, None, None, :]
        out[token_idx] = sdpa(qd, k, v, attn_mask=mask, p_round=p_round, fused=fused)[:, :, 0]

    for i, n in enumerate(news):
        if n == 1:
            continue
        s, length = starts[i], lens[i]
        k = gather(k_cache, meta.block_tables[i:i + 1], length)
        v = gather(v_cache, meta.block_tables[i:i + 1], length)
        qi = q[s:s + n].transpose(0, 1)[None]
        if n == length:
            o = sdpa(qi, k, v, is_causal=True, p_round=p_round, fused=fused)
        else:
            mask = torch.ones(n, length, dtype=torch.bool, device=q.device).tril(diagonal=length - n)
            o = sdpa(qi, k, v, attn_mask=mask, p_round=p_round, fused=fused)
        out[s:s + n] = o[0].transpose(0, 1)
    return out


def forward(q, k, v, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0) -> torch.Tensor:
    """Reference `torch_ref.py:46-48`: write the step's k/v into the pool, then attend."""
    write_kv(k_cache, v_cache, meta.slot_mapping, k, v, k_scale, v_scale)
    return paged_attention(q, k_cache, v_cache, meta, k_scale=k_scale, v_scale=v_scale)


def prefill(q, k, v, key_valid=None) -> torch.Tensor:
    """Reference `torch_ref.py:20-44`: contiguous attention.  q [B, H, Tq, Dh], k/v [B, Hkv, Tk, Dh];
    the queries are the last Tq of the Tk positions.  With `key_valid` [B, Tk] (bool) the mask is
    bottom-right causal AND key-is-real, and a query with no real key may see its own position."""
    tq, tk = q.shape[2], k.shape[2]
    if key_valid is not None:
        causal = torch.ones(tq, tk, dtype=torch.bool, device=q.device).tril(diagonal=tk - tq)
        mask = causal & key_valid[:, None, None, :]
        own = torch.zeros(tq, tk, dtype=torch.bool, device=q.device)
        own[torch.arange(tq), torch.arange(tq) + tk - tq] = True
        mask = mask | (own & ~mask.any(dim=-1, keepdim=True))
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
    if tq == tk:
        return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)
    if tq == 1:
        return F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
    mask = torch.ones(tq, tk, dtype=torch.bool, device=q.device).tril(diagonal=tk - tq)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
