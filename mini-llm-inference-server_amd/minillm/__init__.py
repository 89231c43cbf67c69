"""minillm's paged-attention hot path, MI355X-native (gfx950 HIP kernels behind a C ABI).

Mirrors the reference package's interfaces for this path (reference src/minillm/attention/,
src/minillm/cache/paged.py): `attention.get_backend("hip")`, `attention.metadata.{SeqStep,
AttentionMetadata}` and `cache.paged.PagedKVCache`.
"""
