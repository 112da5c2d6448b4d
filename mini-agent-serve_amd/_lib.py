"""ctypes binding of libmas_kernels.so (the C ABI declared in include/mas_kernels.h).

The library is loaded after ``import torch``: torch maps its bundled HIP runtime
(``libamdhip64.so.7``) first and the kernel library, which needs the same soname, binds to that
runtime, so torch's streams and device pointers are valid in both. There is no fallback: on a
machine without the built library every op raises.
"""
from __future__ import annotations

import ctypes
import threading

import torch  # noqa: F401  (must precede the CDLL load, see above)

from . import _build

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_u32p = ctypes.POINTER(ctypes.c_uint32)

# name -> argtypes, in the order of include/mas_kernels.h
_SIGNATURES: dict[str, list] = {
    "mas_version": [],
    "mas_status_string": [_i32],
    "mas_fused_add_rmsnorm_bf16": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _f32, _c_void_p],
    "mas_fused_add_rmsnorm_quant_fp8": [_c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p,
                                        _f32, _i64, _i64, _f32, _c_void_p],
    "mas_silu_and_mul_bf16": [_c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p],
    "mas_silu_and_mul_quant_fp8": [_c_void_p, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _f32, _c_void_p],
    "mas_rope_cos_sin_cache_bf16": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _i32,
                                    _c_void_p, _i64, _i64, _i64, _i64, _i64, _i32, _c_void_p, _c_void_p],
    "mas_append_paged_kv_cache_bf16": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64,
                                       _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
                                       _i64, _i64, _i64, _i64, _c_void_p, _c_void_p],
    "mas_store_kv_slots_bf16": [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64,
                                _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64, _c_void_p, _c_void_p],
    "mas_rope_append_paged_kv_cache_bf16": [_c_void_p, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                            _i64, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i32,
                                            _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _c_void_p,
                                            _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p,
                                            _c_void_p],
    "mas_embedding_bf16": [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "mas_embedding_fill_placeholders_bf16": [_c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64,
                                             _c_void_p, _i64, _c_void_p, _c_void_p],
    "mas_paged_decode_attention_bf16": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                        _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _i64,
                                        _i64, ctypes.c_float, ctypes.c_float, _i32, _c_void_p, ctypes.c_float,
                                        _c_void_p, _i64, _c_void_p, _c_void_p],
    "mas_paged_decode_attention_bf16_noalloc": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p,
                                                _i64, _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _i64,
                                                _i64, _i64, _i64, ctypes.c_float, ctypes.c_float, _i32, _c_void_p,
                                                ctypes.c_float, _c_void_p, _c_void_p],
    "mas_paged_decode_attention_workspace_bytes": [_i64, _i64, _i64, _i64, _i64, _i64],
    "mas_paged_context_attention_workspace_bytes": [_i64, _i64, _i64, _i64, _i64],
    "mas_paged_context_attention_bf16": [_c_void_p, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                         _i64, _i64, _i64, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _i64,
                                         _i64, _i64, _i64, _i64, _i64, ctypes.c_float, ctypes.c_float, _i32, _c_void_p,
                                         ctypes.c_float, _c_void_p, _i64, _c_void_p, _c_void_p],
}
_RESTYPES = {"mas_status_string": ctypes.c_char_p, "mas_paged_decode_attention_workspace_bytes": ctypes.c_int64,
             "mas_paged_context_attention_workspace_bytes": ctypes.c_int64}

ERROR_BITS = {
    1: "token id outside [0, vocab)",
    2: "position outside the table / negative position",
    4: "batch index outside [0, batch)",
    8: "page slot past kv_indices or page id outside the cache",
    16: "slot past the end of the cache",
    32: "placeholder -1 - r past the previous step's samples",
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class KernelError(RuntimeError):
    """A nonzero status returned by the kernel library."""


def load() -> ctypes.CDLL:
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            path = _build.LIBRARY_PATH
            if not path.exists():
                raise RuntimeError(
                    f"{path.name} is not built (expected at {path}); build it with "
                    "`python -c 'import __graft_entry__ as g; g.build()'` from the repository root")
            lib = ctypes.CDLL(str(path))
            for name, argtypes in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def check(status: int, what: str) -> None:
    if status != 0:
        text = load().mas_status_string(status).decode()
        raise KernelError(f"{what}: status {status} ({text})")


def describe_error_bits(bits: int) -> str:
    return "; ".join(text for bit, text in ERROR_BITS.items() if bits & bit) or "none"


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device` (torch's raw-stream query when it has
    one: 0.1 us per call on MI355X hosts, against 1.9 us for building a Stream object)."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream
