"""The oracle's GPU-only mode, pinned on the GPU: `fused=True` runs the reference's SDPA call in bf16 on
torch's fused memory-efficient kernel (the reference's torch_ref arithmetic on a GPU), the comparison
run of the end-to-end test.  It is checked against the float64 textbook (tests/naive.py) on every row
kind of the reference's kernel harness, at the bf16 tolerance, and against the CPU oracle in bf16."""

import pytest
import torch

from naive import causal_allowed, naive_attention
from oracle import torch_ref
from test_oracle import build_step, cases

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("name", ["kernel_mixed_step", "paged_equals_dense"])
def test_fused_bf16_sdpa_matches_the_textbook(hip, name):
    case = cases()[name]
    q, k, v, pool_k, pool_v, meta, seqs, ctx_k, ctx_v = build_step(case, dtype=torch.bfloat16)
    cpu_pk, cpu_pv = pool_k.clone(), pool_v.clone()
    tm = torch_ref.torch_meta(meta, DEV)
    pk, pv = pool_k.to(DEV), pool_v.to(DEV)
    torch_ref.write_kv(pk, pv, tm.slot_mapping, k.to(DEV), v.to(DEV))
    out = torch_ref.paged_attention(q.to(DEV), pk, pv, tm, fused=True)
    assert out.dtype == torch.bfloat16
    out = out.cpu()
    for i, s in enumerate(seqs):
        st, n, length = meta.query_start_loc[i], s.num_new, meta.seq_lens[i]
        exp = naive_attention(q[st:st + n].transpose(0, 1), ctx_k[i].transpose(0, 1), ctx_v[i].transpose(0, 1),
                              causal_allowed(n, length))
        torch.testing.assert_close(out[st:st + n].double(), exp.transpose(0, 1), atol=2e-2, rtol=1e-2)
    cpu = torch_ref.forward(q, k, v, cpu_pk, cpu_pv, torch_ref.torch_meta(meta, "cpu"))
    torch.testing.assert_close(out.float(), cpu.float(), atol=2e-2, rtol=1e-2)
    # the fused mode is a different kernel from the float32 path, not the same numbers
    f32 = torch_ref.paged_attention(q.to(DEV).float(), pk.float(), pv.float(), tm).cpu()
    assert not torch.equal(out.float(), f32.to(torch.bfloat16).float())
