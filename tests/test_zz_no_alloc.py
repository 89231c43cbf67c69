"""mllm_paged_decode_noalloc (decode + merge with the split partials in the library's own scratch array)
against the existing entry points mllm_paged_decode + mllm_merge_splits with a caller workspace.

Called through the C ABI on two steps in a row, the second smaller than the first (the scratch keeps
the first call's partials, which must not leak into the second), and on a step whose partials exceed
the scratch (rejected before any launch).  Outputs must be bit-identical: the same kernels run.
"""

import pytest
import torch

from harness import bits

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ptr(t):
    return 0 if t is None or t.numel() == 0 else t.data_ptr()


def _decode_both(hip, wl):
    from minillm import _native
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, SeqStep

    print(f"no-alloc decode: workload {wl.name}, {len(wl.seqs)} rows", flush=True)
    backend = HipBackend()
    meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, DEV)
    q, k, v = wl.q.to(DEV), wl.k.to(DEV), wl.v.to(DEV)
    pk, pv = wl.pool_k.to(DEV), wl.pool_v.to(DEV)
    backend.append(k, v, pk, pv, meta)
    plan = backend.plan(meta, wl.h, wl.hkv, wl.dh, q.device)
    slots = int(plan.decode_work[2])  # the plan header: {bins, segments, partial slots, 0}
    assert slots > 0 and plan.num_merge > 0, "the case must cut rows, or the scratch is unused"
    want = torch.full_like(q, float("nan"))
    backend.run_decode(q, pk, pv, meta, want)
    backend.run_merge(q, meta, want)
    got = torch.full_like(q, float("nan"))
    num_blocks, bs, hkv, dh = pk.shape
    hip.call("mllm_paged_decode_noalloc", q.data_ptr(), q.stride(0), q.stride(1), pk.data_ptr(), pv.data_ptr(),
             num_blocks, bs, q.shape[1], hkv, dh, meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(),
             meta.kv_indices.data_ptr(), meta.seq_lens_i32.data_ptr(), _ptr(plan.decode_work), plan.num_decode,
             _ptr(plan.merge_work), plan.num_merge, plan.pages_per_split, dh ** -0.5, _native.dtype_code(q.dtype),
             got.data_ptr(), got.stride(0), got.stride(1), _native.stream_ptr(q.device))
    torch.cuda.synchronize()
    return want, got, plan


def test_noalloc_decode_matches_workspace_decode_twice(hip):
    from minillm import workloads

    big = workloads.decode_256()
    want, got, plan = _decode_both(hip, big)
    assert int(plan.decode_work[2]) > len(big.seqs)  # more partial slots than rows: the scratch is well used
    assert torch.equal(bits(got), bits(want))
    small = workloads.decode_4()  # a smaller step right after: the scratch still holds the first one's partials
    want, got, _ = _decode_both(hip, small)
    assert torch.equal(bits(got), bits(want))


def test_noalloc_decode_rejects_steps_beyond_the_scratch(hip):
    # a plan of 9,000 records can need 4,499 partial slots of 32 heads, 75 MB, more than the 64 MiB scratch:
    # refused with the reason, before any pointer is read or kernel launched; so is 8,067 (4,033 slots)
    for records in (9000, 8067):
        with pytest.raises(ValueError, match="scratch"):
            hip.call("mllm_paged_decode_noalloc", 0, 0, 0, 0, 0, 0, 16, 32, 8, 128, 0, 0, 0, 0, 0, records, 1, 1, 8,
                     1.0, 2, 0, 0, 0, 0)
    # at the limit itself (8,066 records: 4,032 slots at H = 32) the size check passes and the pointer check fires
    with pytest.raises(ValueError, match="null pointer"):
        hip.call("mllm_paged_decode_noalloc", 0, 0, 0, 0, 0, 0, 16, 32, 8, 128, 0, 0, 0, 0, 0, 8066, 1, 1, 8, 1.0,
                 2, 0, 0, 0, 0)


CAPTURE_FIRST_CALL = r"""
import sys
sys.path[:0] = sys.argv[1:]
import torch
from harness import bits
from minillm import _native, workloads
from minillm.attention.hip_backend import HipBackend, _ptr
from minillm.attention.metadata import AttentionMetadata, SeqStep

dev = torch.device("cuda:0")
wl = workloads.decode_256()
be = HipBackend()
meta = AttentionMetadata.build([SeqStep(c, n, list(b)) for c, n, b in wl.seqs], wl.block_size, dev)
q, k, v = wl.q.to(dev), wl.k.to(dev), wl.v.to(dev)
pk, pv = wl.pool_k.to(dev), wl.pool_v.to(dev)
be.append(k, v, pk, pv, meta)
plan = be.plan(meta, wl.h, wl.hkv, wl.dh, dev)
want = torch.full_like(q, float("nan"))
be.run_decode(q, pk, pv, meta, want)
be.run_merge(q, meta, want)
got = torch.full_like(q, float("nan"))
lib = _native.lib()
nb, bs, hkv, dh = pk.shape
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
side = torch.cuda.Stream()
with torch.cuda.graph(g, stream=side):  # the process's first no-alloc call happens under capture
    lib.call("mllm_paged_decode_noalloc", q.data_ptr(), q.stride(0), q.stride(1), pk.data_ptr(), pv.data_ptr(), nb,
             bs, q.shape[1], hkv, dh, meta.qo_indptr.data_ptr(), meta.kv_indptr.data_ptr(),
             meta.kv_indices.data_ptr(), meta.seq_lens_i32.data_ptr(), _ptr(plan.decode_work), plan.num_decode,
             _ptr(plan.merge_work), plan.num_merge, plan.pages_per_split, dh ** -0.5, _native.dtype_code(q.dtype),
             got.data_ptr(), got.stride(0), got.stride(1), _native.stream_ptr(dev))
for i in range(3):
    got.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(bits(got), bits(want)), f"replay {i}"
print("capture ok", flush=True)
"""


def test_noalloc_decode_first_call_under_graph_capture(hip, tmp_path):
    # a fresh process whose first no-alloc call is recorded into a HIP graph (the scratch address is looked
    # up during capture); three replays, each bit-identical to the workspace path
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parent.parent
    script = tmp_path / "capture_first_call.py"
    script.write_text(CAPTURE_FIRST_CALL)
    paths = [str(root / "mini-llm-inference-server_amd"), str(root / "tests"), str(root)]
    print("no-alloc decode: first call under graph capture, fresh process, decode_256", flush=True)
    res = subprocess.run([sys.executable, str(script), *paths], capture_output=True, text=True, timeout=240)
    assert res.returncode == 0 and "capture ok" in res.stdout, res.stdout[-2000:] + res.stderr[-3000:]
