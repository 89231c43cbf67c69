"""Rotary-embedding frequencies, with Llama 3's long-context scaling
(reference src/minillm/model/rope.py:16-42).

inv_freq[i] = theta^(-2i / Dh).  With rope_type "llama3": wavelengths 2*pi / inv_freq longer than
original_len / low_freq_factor are divided by `factor`, those shorter than original_len /
high_freq_factor are kept, and the band between is a linear blend in original_len / wavelength.
"""

from __future__ import annotations

import math

import torch


def compute_inv_freq(config) -> torch.Tensor:
    dim = config.head_dim
    exponents = torch.arange(0, dim, 2, dtype=torch.int64, device="cpu").float() / dim
    inv_freq = 1.0 / (config.rope_theta ** exponents)
    sc = config.rope_scaling
    if sc is None:
        return inv_freq
    if sc["rope_type"] != "llama3":
        raise NotImplementedError(f"rope_type {sc['rope_type']!r}")
    factor, lo, hi = sc["factor"], sc["low_freq_factor"], sc["high_freq_factor"]
    orig = sc["original_max_position_embeddings"]
    wavelen = 2 * math.pi / inv_freq
    long_wave = wavelen > orig / lo
    short_wave = wavelen < orig / hi
    blend = (orig / wavelen - lo) / (hi - lo)
    mid = (1 - blend) * inv_freq / factor + blend * inv_freq
    out = torch.where(long_wave, inv_freq / factor, mid)
    return torch.where(short_wave, inv_freq, out)
