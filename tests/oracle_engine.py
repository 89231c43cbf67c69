"""The oracle as a drop-in attention backend and metadata builder, for end-to-end comparisons of the
engine on the GPU: same model, same weights, same engine code, only the hot path swapped."""

from __future__ import annotations

from types import SimpleNamespace

import torch

from oracle import torch_ref
from oracle.metadata import OracleSeq, build_metadata


def oracle_metadata(seqs, block_size, device):
    """The oracle's metadata build, as device tensors with the contract's field names."""
    om = build_metadata([OracleSeq(s.num_cached, s.num_new, list(s.block_ids)) for s in seqs], block_size)
    t = {name: torch.from_numpy(getattr(om, name)).to(device) for name in om.TENSOR_FIELDS}
    return SimpleNamespace(block_size=block_size, query_start_loc=om.query_start_loc, seq_lens=om.seq_lens,
                           num_new=om.num_new, max_query_len=om.max_query_len, max_seq_len=om.max_seq_len,
                           num_seqs=om.num_seqs, **t)


class OracleBackend:
    """write_kv + gather/SDPA restated from the reference; attention computed in float32.  With
    `p_round` (torch.bfloat16) the softmax probabilities are rounded before the product with V: bf16
    attention arithmetic, the noise-floor reference of end-to-end comparisons.  With `fused` and
    compute_dtype torch.bfloat16, SDPA runs in bf16 on torch's fused memory-efficient kernel: the
    reference's torch_ref backend as it computes on a GPU in bf16."""

    name = "oracle"

    def __init__(self, compute_dtype=torch.float32, p_round=None, fused: bool = False) -> None:
        self.compute_dtype = compute_dtype
        self.p_round = p_round
        self.fused = fused

    def forward(self, q, k, v, k_cache, v_cache, meta, k_scale: float = 1.0, v_scale: float = 1.0):
        torch_ref.write_kv(k_cache, v_cache, meta.slot_mapping, k, v, k_scale, v_scale)
        return torch_ref.paged_attention(q, k_cache, v_cache, meta, compute_dtype=self.compute_dtype,
                                         k_scale=k_scale, v_scale=v_scale, p_round=self.p_round, fused=self.fused)

    def prefill(self, q, k, v, key_valid=None, **kwargs):
        dt = q.dtype
        c = self.compute_dtype
        return torch_ref.prefill(q.to(c), k.to(c), v.to(c), key_valid=key_valid).to(dt)
