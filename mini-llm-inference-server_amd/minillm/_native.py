"""ctypes binding of libminillm_hip.so (the C ABI in include/minillm_hip.h).

The library is loaded once per process.  Every call passes raw device pointers and the current HIP
stream; a nonzero status becomes ValueError (argument or unsupported-shape errors) or RuntimeError
(HIP errors) carrying the library's message.  A missing library raises RuntimeError: there is no
fallback path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("MLLM_HIP_LIB", Path(__file__).resolve().parent / "_lib" / "libminillm_hip.so"))

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, -1, -2, -3
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
ABI_VERSION = 4

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class LayerStep(ctypes.Structure):
    """mllm_layer_step: the step-constant arguments of mllm_attention_forward (same fields, same order)."""

    _fields_ = [("num_blocks", _i64), ("num_tokens", _i64), ("slot_mapping", _p), ("qo_indptr", _p),
                ("kv_indptr", _p), ("kv_indices", _p), ("seq_lens", _p), ("decode_work", _p), ("merge_work", _p),
                ("prefill_work", _p), ("workspace", _p), ("workspace_bytes", _i64), ("num_decode_work", _i32),
                ("num_merge_work", _i32), ("num_prefill_work", _i32), ("pages_per_split", _i32),
                ("q_tile_tokens", _i32), ("num_heads", _i32), ("num_kv_heads", _i32), ("head_dim", _i32),
                ("block_size", _i32), ("dtype", _i32), ("kv_fp8", _i32), ("softmax_scale", _f32)]

# symbol -> (restype, argtypes); the exact list include/minillm_hip.h declares
SIGNATURES = {
    "mllm_abi_version": (ctypes.c_int, []),
    "mllm_last_error": (ctypes.c_char_p, []),
    "mllm_build_metadata": (ctypes.c_int, [_p, _p, _p, _p, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p,
                                           _p]),
    "mllm_build_metadata_rows": (ctypes.c_int, [_p, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p, _p,
                                                _p, _p, _p, _p, _p]),
    "mllm_update_block_tables": (ctypes.c_int, [_p, _i64, _p, _i32, _p]),
    "mllm_kv_append": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _p, _i32, _i64, _i32, _i32, _p, _i64,
                                      _p]),
    "mllm_rope_kv_append": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i32, _i32,
                                           _i32, _i32, _p, _i64, _i64, _p, _p, _i64, _p, _i64, _p]),
    "mllm_plan": (ctypes.c_int, [_p, _p, _p, _i32, _i32, _i32, _p, _i32, _p, _i32, _p, _i32, _p]),
    "mllm_plan_dev": (ctypes.c_int, [_p, _p, _p, _i32, _p, _i32, _i32, _p, _i32, _p, _i32, _p, _i32, _p]),
    "mllm_decode_workspace_bytes": (ctypes.c_int64, [_i32, _i32, _i32]),
    "mllm_paged_decode": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                         _i32, _p, _i32, _i32, _f32, _i32, _p, _i64, _i64, _p, _i64, _p]),
    "mllm_merge_splits": (ctypes.c_int, [_p, _i32, _i32, _i32, _i32, _p, _i32, _p, _i64, _i64, _p, _i64, _p]),
    # decode + merge with the partials in the library's own scratch array (no allocation)
    "mllm_paged_decode_noalloc": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p,
                                                 _p, _i32, _p, _i32, _i32, _f32, _i32, _p, _i64, _i64, _p]),
    # one layer: append (RoPE optionally fused), decode + merge, prefill
    "mllm_attention_forward": (ctypes.c_int, [_p, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p,
                                              _p, _p, _f32, _f32, _p, _p]),
    "mllm_paged_prefill": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                          _i32, _i32, _f32, _i32, _p, _i64, _i64, _p]),
    "mllm_dense_attention": (ctypes.c_int, [_p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64,
                                            _i64, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _p, _i64, _i64, _i64,
                                            _p]),
    # fp8 (e4m3fn) pools with per-tensor k_scale / v_scale
    "mllm_kv_append_fp8": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _i32, _p, _p, _i64, _i32, _i32, _p, _i64, _f32,
                                          _f32, _p]),
    "mllm_rope_kv_append_fp8": (ctypes.c_int, [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _i32,
                                               _i32, _i32, _i32, _p, _i64, _i64, _p, _p, _i64, _p, _i64, _f32, _f32,
                                               _p]),
    "mllm_paged_decode_fp8": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                             _i32, _p, _i32, _i32, _f32, _i32, _f32, _f32, _p, _i64, _i64, _p, _i64,
                                             _p]),
    "mllm_paged_prefill_fp8": (ctypes.c_int, [_p, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _p, _p, _p, _p,
                                              _i32, _i32, _f32, _i32, _f32, _f32, _p, _i64, _i64, _p]),
}


class NativeLib:
    """The loaded library with typed entry points that raise on a nonzero status."""

    def __init__(self, path: Path) -> None:
        if not path.exists():
            raise RuntimeError(f"HIP library not built: {path} is missing (run __graft_entry__.build() or "
                               f"python build_hip.py)")
        self.path = path
        self._cdll = ctypes.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self._cdll, name)
            fn.restype = res
            fn.argtypes = args
        version = self._cdll.mllm_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")

    def last_error(self) -> str:
        return (self._cdll.mllm_last_error() or b"").decode()

    def fn(self, name: str):
        """The typed foreign function itself, for callers that check its status with `check`."""
        return getattr(self._cdll, name)

    def check(self, status: int) -> None:
        self._check(status)

    def _check(self, status: int) -> None:
        if status == OK:
            return
        msg = self.last_error()
        if status in (ERR_INVALID, ERR_UNSUPPORTED):
            raise ValueError(msg)
        raise RuntimeError(msg or f"HIP library error {status}")

    def call(self, name: str, *args) -> None:
        self._check(getattr(self._cdll, name)(*args))

    def workspace_bytes(self, num_work: int, num_heads: int, head_dim: int) -> int:
        return int(self._cdll.mllm_decode_workspace_bytes(num_work, num_heads, head_dim))


_LIB: NativeLib | None = None


def lib() -> NativeLib:
    global _LIB
    if _LIB is None:
        _LIB = NativeLib(LIB_PATH)
    return _LIB


_DTYPE_CODES: dict = {}


def dtype_code(dtype) -> int:
    if not _DTYPE_CODES:
        import torch

        _DTYPE_CODES.update({torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16})
    code = _DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"unsupported dtype {dtype}")
    return code


def stream_ptr(device) -> int:
    """The raw hipStream_t of the device's current stream (what `torch.cuda.current_stream(device).cuda_stream`
    returns, without building a Stream object: 0.08 against 1.9 us per call, paid by every launch)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:  # a torch without the raw accessor: the same handle through the public API
        return torch.cuda.current_stream(device).cuda_stream
    index = device if isinstance(device, int) else torch.device(device).index
    if index is None:
        index = torch.cuda.current_device()
    return raw(index)
