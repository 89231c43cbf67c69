"""Llama decoder, as the engine's caller of the attention backend
(reference src/minillm/model/llama.py:22-237; module and parameter names follow Hugging Face so
checkpoints load by name).

The hot path's call site is `LlamaAttention.forward` on a ragged paged step: q/k/v of the N new tokens
go to `backend.forward(q[N,H,Dh], k[N,Hkv,Dh], v[N,Hkv,Dh], k_pool[layer], v_pool[layer], meta)`,
which appends k/v to the pool and returns the attention output.  GEMMs, RMSNorm, RoPE and SwiGLU stay
in PyTorch.  Without a cache (kv_cache None) the contiguous `backend.prefill` path runs instead.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from ..attention import AttentionBackend, get_backend
from .config import LlamaConfig
from .rope import compute_inv_freq


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float) -> None:
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x * rsqrt(mean(x^2) + eps) computed in float32, cast back, then scaled by the weight."""
        h = x.float()
        h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + self.eps)
        return self.weight * h.to(x.dtype)


class RotaryEmbedding(nn.Module):
    """The frequency table is derived from the config and kept in float32 on every device it is used on
    (not a module buffer, so casting the model to bf16 never rounds it)."""

    def __init__(self, config: LlamaConfig) -> None:
        super().__init__()
        self._inv_freq = compute_inv_freq(config)
        self._on_device: dict[torch.device, torch.Tensor] = {}

    def inv_freq(self, device: torch.device) -> torch.Tensor:
        t = self._on_device.get(device)
        if t is None:
            t = self._on_device[device] = self._inv_freq.to(device)
        return t

    def forward(self, positions: torch.Tensor, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
        """positions [B, T] -> cos, sin [B, T, Dh]: float32 angles, the half-size table repeated."""
        ang = positions[..., None].float() * self.inv_freq(positions.device)
        ang = torch.cat([ang, ang], dim=-1)
        return ang.cos().to(dtype), ang.sin().to(dtype)


def apply_rotary(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, heads, T, Dh]: pairs (i, i + Dh/2) rotated by their angle ("rotate half" convention)."""
    cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
    half = x.shape[-1] // 2
    rot = torch.cat([-x[..., half:], x[..., :half]], dim=-1)
    return x * cos + rot * sin


class LlamaAttention(nn.Module):
    def __init__(self, config: LlamaConfig, backend: AttentionBackend, layer_idx: int) -> None:
        super().__init__()
        self.config = config
        self.backend = backend
        self.layer_idx = layer_idx
        h, hkv, dh, d = config.num_attention_heads, config.num_key_value_heads, config.head_dim, config.hidden_size
        self.q_proj = nn.Linear(d, h * dh, bias=False)
        self.k_proj = nn.Linear(d, hkv * dh, bias=False)
        self.v_proj = nn.Linear(d, hkv * dh, bias=False)
        self.o_proj = nn.Linear(h * dh, d, bias=False)

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, kv_cache=None,
                key_valid: torch.Tensor | None = None) -> torch.Tensor:
        b, t, _ = x.shape
        dh = self.config.head_dim
        q = self.q_proj(x).view(b, t, -1, dh).transpose(1, 2)
        k = self.k_proj(x).view(b, t, -1, dh).transpose(1, 2)
        v = self.v_proj(x).view(b, t, -1, dh).transpose(1, 2)
        if getattr(kv_cache, "ragged", False):
            # ragged step: one row of every sequence's new tokens -> [N, heads, Dh] views for the backend
            layer = self.layer_idx
            pools = (kv_cache.cache.k[layer], kv_cache.cache.v[layer], kv_cache.meta)
            scales = kv_cache.cache.scales(layer)  # fp8 pools only
            if getattr(self.backend, "fuse_rotary", False) and b == 1:
                # the backend rotates q and k itself, in the launch that appends k and v
                out = self.backend.forward_rotary(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1),
                                                  cos[0], sin[0], *pools, **scales)
            else:
                q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
                out = self.backend.forward(q[0].transpose(0, 1), k[0].transpose(0, 1), v[0].transpose(0, 1), *pools,
                                           **scales)
            return self.o_proj(out.reshape(b, t, -1))
        q, k = apply_rotary(q, cos, sin), apply_rotary(k, cos, sin)
        if kv_cache is not None:
            raise ValueError("only paged ragged caches (PagedStep) are supported")
        out = self.backend.prefill(q, k, v, key_valid=key_valid)
        return self.o_proj(out.transpose(1, 2).reshape(b, t, -1))


class LlamaMLP(nn.Module):
    def __init__(self, config: LlamaConfig) -> None:
        super().__init__()
        d, f = config.hidden_size, config.intermediate_size
        self.gate_proj = nn.Linear(d, f, bias=False)
        self.up_proj = nn.Linear(d, f, bias=False)
        self.down_proj = nn.Linear(f, d, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class LlamaDecoderLayer(nn.Module):
    def __init__(self, config: LlamaConfig, backend: AttentionBackend, layer_idx: int) -> None:
        super().__init__()
        self.input_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.self_attn = LlamaAttention(config, backend, layer_idx)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = LlamaMLP(config)

    def forward(self, x, cos, sin, kv_cache=None, key_valid=None):
        x = x + self.self_attn(self.input_layernorm(x), cos, sin, kv_cache, key_valid)
        return x + self.mlp(self.post_attention_layernorm(x))


class LlamaModel(nn.Module):
    def __init__(self, config: LlamaConfig, backend: AttentionBackend) -> None:
        super().__init__()
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(LlamaDecoderLayer(config, backend, i) for i in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.rotary_emb = RotaryEmbedding(config)

    def forward(self, input_ids, positions, kv_cache=None, attention_mask=None):
        if kv_cache is not None:
            kv_cache.mark(attention_mask, input_ids.shape[1])
            key_valid = kv_cache.key_valid(input_ids.shape[1])
        else:
            key_valid = None if attention_mask is None else attention_mask.to(torch.bool)
        x = self.embed_tokens(input_ids)
        cos, sin = self.rotary_emb(positions, x.dtype)  # shared by every layer
        for layer in self.layers:
            x = layer(x, cos, sin, kv_cache, key_valid)
        if kv_cache is not None:
            kv_cache.advance(input_ids.shape[1])
        return self.norm(x)


class LlamaForCausalLM(nn.Module):
    def __init__(self, config: LlamaConfig, backend: AttentionBackend | None = None) -> None:
        super().__init__()
        self.config = config
        self.model = LlamaModel(config, backend or get_backend("hip"))
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    def set_backend(self, backend: AttentionBackend) -> None:
        for layer in self.model.layers:
            layer.self_attn.backend = backend

    def forward(self, input_ids, positions=None, kv_cache=None, last_only: bool = False, attention_mask=None,
                last_index=None):
        """input_ids [B, T] -> logits [B, T, V]; with a ragged paged step and `last_index` (the metadata's
        logits_index) only each sequence's last new token reaches lm_head: [S, 1, V]."""
        if positions is None:
            if kv_cache is not None:
                positions = kv_cache.positions(input_ids, attention_mask)
            elif attention_mask is not None:
                positions = (attention_mask.long().cumsum(dim=1) - 1).clamp_min(0)
            else:
                positions = torch.arange(input_ids.shape[1], device=input_ids.device).expand_as(input_ids)
        hidden = self.model(input_ids, positions, kv_cache, attention_mask)
        if last_index is not None and getattr(kv_cache, "ragged", False):
            hidden = hidden[0, last_index.to(hidden.device)][:, None]
        elif last_index is not None:
            rows = torch.arange(hidden.shape[0], device=hidden.device)
            hidden = hidden[rows, last_index.to(hidden.device)][:, None]
        elif last_only:
            hidden = hidden[:, -1:]
        return self.lm_head(hidden)


@torch.no_grad()
def random_init_(model: LlamaForCausalLM, std: float = 0.02, seed: int = 0) -> LlamaForCausalLM:
    """Seeded N(0, std) weights (norms stay 1), drawn on the model's device."""
    dev = next(model.parameters()).device
    g = torch.Generator(device=dev).manual_seed(seed)
    for name, p in model.named_parameters():
        if name.endswith("layernorm.weight") or name.endswith("norm.weight"):
            p.fill_(1.0)
        else:
            p.copy_(torch.randn(p.shape, generator=g, device=dev, dtype=torch.float32).to(p.dtype) * std)
    return model
