"""Runs one layer of a ragged paged step through the HIP backend and through the CPU oracle's
algorithm on identical inputs (shared by the GPU parity tests, smoke() and bench.py)."""

from __future__ import annotations

import torch

from oracle import torch_ref
from oracle.metadata import OracleSeq, build_metadata

ATOL, RTOL = 2e-2, 1e-2  # bf16 outputs vs the fp32 oracle (fp32 accumulation in the kernels)


def hip_step(wl, device, backend=None, pool_fill=None):
    """Metadata build + backend.forward on `device`; returns (out, pool_k, pool_v, meta)."""
    from minillm.attention import get_backend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, device)
    pk = wl.pool_k.to(device)
    pv = wl.pool_v.to(device)
    if pool_fill is not None:
        pool_fill(pk, pv, wl)
    backend = backend or get_backend("hip")
    out = backend.forward(wl.q.to(device), wl.k.to(device), wl.v.to(device), pk, pv, meta)
    return out, pk, pv, meta


def oracle_step(wl, device, dtype=torch.float32, pool_fill=None):
    """The oracle (gather + SDPA restated from the reference) on `device` in `dtype`; returns
    (out, pool_k, pool_v) where the pools hold the step's k/v after write_kv."""
    om = build_metadata([OracleSeq(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size)
    tm = torch_ref.torch_meta(om, device)
    pk = wl.pool_k.to(device)
    pv = wl.pool_v.to(device)
    if pool_fill is not None:
        pool_fill(pk, pv, wl)
    torch_ref.write_kv(pk, pv, tm.slot_mapping, wl.k.to(device), wl.v.to(device))
    out = torch_ref.paged_attention(wl.q.to(device=device, dtype=dtype), pk.to(dtype), pv.to(dtype), tm)
    return out, pk, pv


def bits(t: torch.Tensor) -> torch.Tensor:
    """Bit pattern view for exact comparisons (NaN payloads included)."""
    return t.view({2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])
