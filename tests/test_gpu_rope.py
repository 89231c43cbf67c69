"""GPU parity of the fused rotary embedding + KV append (`mllm_rope_kv_append`) against the oracle's
`rope_then_write_kv` (the model's apply_rotary followed by write_kv, torch ops on the CPU):
the rotated q and both pools bit-identical, for bf16 and fp16, contiguous and strided inputs; and the
fused backend path giving the same attention output, bit for bit, as RoPE in torch plus `forward`."""

import pytest
import torch

from harness import ATOL, RTOL, bits
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(n, h, hkv, dh, dtype, seed, nb=64, bs=16, fused_qkv=False):
    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import RotaryEmbedding

    gen = torch.Generator().manual_seed(seed)
    if fused_qkv:  # q, k, v as column slices of one projection output (token stride (h + 2 hkv) dh)
        qkv = torch.randn(n, (h + 2 * hkv) * dh, generator=gen).to(dtype)
        q = qkv[:, : h * dh].view(n, h, dh)
        k = qkv[:, h * dh: (h + hkv) * dh].view(n, hkv, dh)
        v = qkv[:, (h + hkv) * dh:].view(n, hkv, dh)
    else:
        q, k, v = (torch.randn(n, x, dh, generator=gen).to(dtype) for x in (h, hkv, hkv))
    cfg = LlamaConfig(**{**LLAMA_3_1_8B, "head_dim": dh})
    pos = torch.randint(0, 131072, (1, n), generator=gen)
    cos, sin = RotaryEmbedding(cfg)(pos, dtype)
    pool = [torch.randn(nb, bs, hkv, dh, generator=gen).to(dtype) for _ in range(2)]
    slots = torch.randperm(nb * bs, generator=gen)[:n]
    return q, k, v, cos[0], sin[0], pool, slots


class _Meta:
    def __init__(self, slots):
        self.slot_mapping = slots


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,seed", [(1, 0), (37, 1), (300, 2), (4096, 3)])
def test_rope_append_bit_exact(hip, dtype, n, seed):
    from minillm.attention.hip_backend import HipBackend

    h, hkv, dh = 32, 8, 128
    q, k, v, cos, sin, (pk, pv), slots = _inputs(n, h, hkv, dh, dtype, seed, nb=max(64, n // 8))
    exp_k, exp_v = pk.clone(), pv.clone()
    exp_q = torch_ref.rope_then_write_kv(q, k, v, cos, sin, exp_k, exp_v, slots)
    gk, gv = pk.to(DEV), pv.to(DEV)
    got_q = HipBackend().rope_append(q.to(DEV), k.to(DEV), v.to(DEV), cos.to(DEV), sin.to(DEV), gk, gv,
                                     _Meta(slots.to(DEV)))
    assert torch.equal(bits(got_q.cpu()), bits(exp_q))
    assert torch.equal(bits(gk.cpu()), bits(exp_k)) and torch.equal(bits(gv.cpu()), bits(exp_v))


def test_rope_append_strided_views_and_other_shapes(hip):
    from minillm.attention.hip_backend import HipBackend

    for h, hkv, dh, seed in [(32, 8, 128, 4), (8, 8, 64, 5), (16, 2, 256, 6)]:
        q, k, v, cos, sin, (pk, pv), slots = _inputs(53, h, hkv, dh, torch.bfloat16, seed, fused_qkv=True)
        exp_k, exp_v = pk.clone(), pv.clone()
        exp_q = torch_ref.rope_then_write_kv(q, k, v, cos, sin, exp_k, exp_v, slots)
        qd = torch.cat([q.reshape(53, -1), k.reshape(53, -1), v.reshape(53, -1)], 1).to(DEV)
        gq = qd[:, : h * dh].view(53, h, dh)
        gk_in = qd[:, h * dh: (h + hkv) * dh].view(53, hkv, dh)
        gv_in = qd[:, (h + hkv) * dh:].view(53, hkv, dh)
        gk, gv = pk.to(DEV), pv.to(DEV)
        got_q = HipBackend().rope_append(gq, gk_in, gv_in, cos.to(DEV), sin.to(DEV), gk, gv, _Meta(slots.to(DEV)))
        assert torch.equal(bits(got_q.cpu()), bits(exp_q)), (h, hkv, dh)
        assert torch.equal(bits(gk.cpu()), bits(exp_k)) and torch.equal(bits(gv.cpu()), bits(exp_v)), (h, hkv, dh)


def test_forward_rotary_equals_rope_then_forward(hip):
    # the fused path and the reference call sequence (RoPE in torch, then forward) on one mixed step
    from minillm.attention.hip_backend import HipBackend
    from minillm.attention.metadata import AttentionMetadata, SeqStep
    from minillm.model.config import LLAMA_3_1_8B, LlamaConfig
    from minillm.model.llama import RotaryEmbedding

    h, hkv, dh, bs, nb = 32, 8, 128, 16, 160
    gen = torch.Generator().manual_seed(7)
    steps = [(0, 37), (90, 1), (40, 25), (0, 1), (300, 1), (700, 1), (1000, 300)]
    free = torch.randperm(nb, generator=gen).tolist()
    seqs = [SeqStep(c, n, [free.pop() for _ in range(-(-(c + n) // bs))]) for c, n in steps]
    n = sum(s for _, s in steps)
    q, k, v = (torch.randn(n, x, dh, generator=gen).to(torch.bfloat16).to(DEV) for x in (h, hkv, hkv))
    pk0 = torch.randn(nb, bs, hkv, dh, generator=gen).to(torch.bfloat16).to(DEV)
    pv0 = torch.randn(nb, bs, hkv, dh, generator=gen).to(torch.bfloat16).to(DEV)
    meta = AttentionMetadata.build(seqs, bs, DEV)
    cos, sin = RotaryEmbedding(LlamaConfig(**LLAMA_3_1_8B))(meta.positions[None], torch.bfloat16)
    be = HipBackend()
    pk1, pv1 = pk0.clone(), pv0.clone()
    fused = be.forward_rotary(q, k, v, cos[0], sin[0], pk1, pv1, meta)
    qr = torch_ref.apply_rotary(q, cos[0], sin[0])
    kr = torch_ref.apply_rotary(k, cos[0], sin[0])
    pk2, pv2 = pk0.clone(), pv0.clone()
    plain = HipBackend().forward(qr, kr, v, pk2, pv2, meta)
    assert torch.equal(bits(pk1), bits(pk2)) and torch.equal(bits(pv1), bits(pv2))
    assert torch.equal(bits(fused), bits(plain))
    assert torch.isfinite(fused.float()).all()


def test_rope_append_rejects_bad_arguments(hip):
    from minillm.attention.hip_backend import HipBackend

    q, k, v, cos, sin, (pk, pv), slots = _inputs(8, 32, 8, 128, torch.bfloat16, 8)
    be = HipBackend()
    args = [t.to(DEV) for t in (q, k, v)]
    with pytest.raises(ValueError):
        be.rope_append(*args, cos[:4].to(DEV), sin[:4].to(DEV), pk.to(DEV), pv.to(DEV), _Meta(slots.to(DEV)))
    with pytest.raises(ValueError):
        be.rope_append(*args, cos.float().to(DEV), sin.float().to(DEV), pk.to(DEV), pv.to(DEV), _Meta(slots.to(DEV)))
