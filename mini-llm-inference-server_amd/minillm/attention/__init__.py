"""Attention backends for the paged hot path (reference src/minillm/attention/__init__.py:15-28).

- `hip`: the gfx950 kernels of libminillm_hip.so (metadata build, KV append, split-KV decode,
  MFMA prefill), in `hip_backend.py`.
- `metadata.py`: the per-step description of a ragged batch on paged KV, built on the GPU.

Pick one with `get_backend(name)`; an unknown name raises ValueError, and a backend whose library
is unavailable raises RuntimeError at construction.
"""

from .base import AttentionBackend

BACKENDS = ("hip",)


def get_backend(name: str) -> AttentionBackend:
    if name == "hip":
        from .hip_backend import HipBackend

        return HipBackend()
    raise ValueError(f"unknown attention backend: {name!r} (available: {', '.join(BACKENDS)})")


__all__ = ["AttentionBackend", "get_backend", "BACKENDS"]
