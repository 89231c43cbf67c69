"""GPU parity of the backend's contiguous `prefill` (reference torch_ref.py:20-44) with the oracle's
restatement, for the reference's own test shapes (tests/test_attention.py:22-55) and the key_valid
padding rule, in float32, float16 and bfloat16."""

import pytest
import torch

from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (2e-3, 1e-3), torch.bfloat16: (2e-2, 1e-2)}


def _check(q, k, v, key_valid=None):
    from minillm.attention import get_backend

    out = get_backend("hip").prefill(q.to(DEV), k.to(DEV), v.to(DEV),
                                     key_valid=None if key_valid is None else key_valid.to(DEV))
    ref = torch_ref.prefill(q.double(), k.double(), v.double(), key_valid=key_valid)
    atol, rtol = TOL[q.dtype]
    torch.testing.assert_close(out.cpu().double(), ref, atol=atol, rtol=rtol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("h,hkv", [(4, 4), (4, 2), (8, 1)], ids=["mha", "gqa", "mqa"])
def test_prefill_matches(hip, dtype, h, hkv):
    g = torch.Generator().manual_seed(0)
    b, t, dh = 2, 7, 16
    q, k, v = (torch.randn(b, n, t, dh, generator=g).to(dtype) for n in (h, hkv, hkv))
    _check(q, k, v)


@pytest.mark.parametrize("tq,tk", [(1, 9), (4, 9), (9, 9), (300, 700), (1, 1000)])
def test_prefill_on_top_of_cache(hip, tq, tk):
    g = torch.Generator().manual_seed(2)
    q_all, k, v = (torch.randn(1, n, tk, 128, generator=g) for n in (8, 2, 2))
    _check(q_all[:, :, -tq:].contiguous(), k, v)


def test_prefill_key_valid(hip):
    g = torch.Generator().manual_seed(3)
    b, tq, tk = 3, 5, 12
    q = torch.randn(b, 4, tq, 32, generator=g)
    k = torch.randn(b, 2, tk, 32, generator=g)
    v = torch.randn(b, 2, tk, 32, generator=g)
    key_valid = torch.ones(b, tk, dtype=torch.bool)
    key_valid[0, :9] = False  # left padding: row 0's first query sees no real key but its own slot
    key_valid[1, 10:] = False  # a shorter row (M4 slot batch)
    _check(q, k, v, key_valid)


def test_prefill_strided_views(hip):
    # [B, T, H, Dh] storage seen as [B, H, T, Dh], as llama.py's view + transpose produces
    g = torch.Generator().manual_seed(4)
    q = torch.randn(2, 11, 8, 64, generator=g).transpose(1, 2)
    k = torch.randn(2, 11, 4, 64, generator=g).transpose(1, 2)
    v = torch.randn(2, 11, 4, 64, generator=g).transpose(1, 2)
    _check(q, k, v)
