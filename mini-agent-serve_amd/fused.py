"""RoPE + paged KV append (+ the llama-4 query scale) in one kernel: the call sequence at
miniagentserve/models/devstral2/devstral2.py:163-179 (``apply_rope_with_cos_sin_cache_inplace``, then
``append_paged_kv_cache`` on the same token rows and positions, then
``q * (1 + beta * log1p(floor(pos / original_max)))``) as one launch.

The results equal those of the separate calls: q and k are rotated in place, the rotated k and the
v rows land in the cache pages, and with a nonzero beta q is then scaled in place with the
reference's two roundings (bf16 rotate, then a bf16 multiply by the bf16 scale). Each k row is read
once instead of twice, q once instead of twice, and a decode step launches one kernel instead of
two (three with the scale).
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device
from .page import _cache_geometry, _index_vector, _source_view
from .rope import _head_view

__all__ = ["apply_rope_and_append_paged_kv_cache", "llama_4_q_scale_table"]

SUPPORTED_HEAD_DIMS = (32, 64, 128, 256, 512)

_Q_SCALE_TABLES: dict = {}


def llama_4_q_scale_table(beta: float, original_max_position: int, rows: int, device) -> torch.Tensor:
    """bf16 ``[rows]``: row k is the llama-4 query scale of every position in
    ``[k * original_max_position, (k + 1) * original_max_position)``, made with the reference's own
    torch expression (devstral2.py:176-179) on ``floor(pos / original_max)`` = k (exact for
    positions below 2^24, where ``pos.float() / original_max`` is an exact or correctly rounded
    fp32 quotient whose floor is the integer quotient). Cached per (beta, interval, rows, device);
    the first call for a key must happen outside HIP graph capture."""
    device = torch.device(device)
    key = (float(beta), int(original_max_position), int(rows), device)
    table = _Q_SCALE_TABLES.get(key)
    if table is None:
        if device.type == "cuda" and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("the llama-4 q-scale table is built on first use; make one call outside graph "
                               "capture first (the model runner's warm-up does)")
        k = torch.arange(int(rows), dtype=torch.float32, device=device)
        table = (1 + float(beta) * torch.log1p(torch.floor(k))).to(torch.bfloat16)
        _Q_SCALE_TABLES[key] = table
    return table


def _fused(positions, query, key, value, head_size, cos_sin_cache, is_neox, batch_indices, paged_kv_cache,
           kv_indices, kv_indptr, kv_layout, error_flags, llama_4_scaling_beta=0.0,
           original_max_position_embeddings=0) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, heads, dim = _cache_geometry(paged_kv_cache,
                                                                                                kv_layout)
    if dim != head_size:
        raise ValueError(f"cache head_dim {dim} != head_size {head_size}")
    if head_size not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_size must be one of {SUPPORTED_HEAD_DIMS} for the fused op, got {head_size}")
    for name, t in (("query", query), ("key", key), ("cos_sin_cache", cos_sin_cache)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(key, "key", torch.bfloat16)
    require_dtype(cos_sin_cache, "cos_sin_cache", torch.float32)
    if cos_sin_cache.dim() != 2 or cos_sin_cache.shape[1] != head_size or cos_sin_cache.stride(1) != 1:
        raise ValueError("cos_sin_cache must be [max_position, head_size] with a contiguous last dimension "
                         "(the fused op rotates the whole head)")
    q_rows, q_stride, q_hstride, hq = _head_view(query, "query", head_size)
    k_rows, k_stride, k_hstride, hk = _head_view(key, "key", head_size)
    v_rows, v_stride, v_hstride = _source_view(value, "value", heads, dim)
    if hk != heads:
        raise ValueError(f"key has {hk} heads, the cache {heads}")
    for name, t in (("positions", positions), ("batch_indices", batch_indices), ("kv_indices", kv_indices),
                    ("kv_indptr", kv_indptr)):
        _index_vector(t, name, torch.int32)
    device = require_same_device(("query", query), ("key", key), ("value", value), ("k_cache", k_cache),
                                 ("positions", positions), ("batch_indices", batch_indices),
                                 ("kv_indices", kv_indices), ("kv_indptr", kv_indptr),
                                 ("cos_sin_cache", cos_sin_cache))
    if not (q_rows == k_rows == v_rows == positions.shape[0] == batch_indices.shape[0]):
        raise ValueError("query, key, value, positions and batch_indices must have the same number of rows")
    if kv_indptr.shape[0] < 1:
        raise ValueError("kv_indptr needs batch + 1 entries")
    if cos_sin_cache.shape[0] == 0 and q_rows > 0 and hq + heads > 0:
        raise ValueError("cos_sin_cache has no rows (the fused op loads each token's row before judging its position)")
    q_scale_ptr, q_scale_rows, interval = None, 0, 0
    if llama_4_scaling_beta:
        interval = int(original_max_position_embeddings)
        if interval < 1:
            raise ValueError("llama-4 query scaling needs original_max_position_embeddings >= 1")
        q_scale_rows = -(-cos_sin_cache.shape[0] // interval)
        q_scale = llama_4_q_scale_table(llama_4_scaling_beta, interval, max(q_scale_rows, 1), device)
        q_scale_ptr, q_scale_rows = q_scale.data_ptr(), q_scale.shape[0]
    st = _lib.load().mas_rope_append_paged_kv_cache_bf16(
        query.data_ptr(), q_stride, q_hstride, hq, key.data_ptr(), k_stride, k_hstride, value.data_ptr(), v_stride,
        v_hstride, heads, positions.data_ptr(), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0),
        cos_sin_cache.shape[0], q_rows, head_size, int(bool(is_neox)), k_cache.data_ptr(), v_cache.data_ptr(),
        pstride, estride, hstride, pages, page_size, batch_indices.data_ptr(), kv_indices.data_ptr(),
        kv_indices.shape[0], kv_indptr.data_ptr(), kv_indptr.shape[0] - 1, q_scale_ptr, q_scale_rows, interval,
        error_word(error_flags, device), _lib.stream_handle(device))
    _lib.check(st, "apply_rope_and_append_paged_kv_cache")


def apply_rope_and_append_paged_kv_cache(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                                         value: torch.Tensor, head_size: int, cos_sin_cache: torch.Tensor,
                                         is_neox: bool, batch_indices: torch.Tensor, paged_kv_cache,
                                         kv_indices: torch.Tensor, kv_indptr: torch.Tensor,
                                         kv_last_page_len: torch.Tensor | None = None, kv_layout: str = "NHD", *,
                                         llama_4_scaling_beta: float = 0.0,
                                         original_max_position_embeddings: int = 0,
                                         error_flags: torch.Tensor | None = None) -> None:
    """``apply_rope_with_cos_sin_cache_inplace(positions, query, key, head_size, cos_sin_cache, is_neox)``
    followed by ``append_paged_kv_cache(key, value, batch_indices, positions, paged_kv_cache, kv_indices,
    kv_indptr, kv_last_page_len, kv_layout)``, in one kernel. The table must cover the whole head
    (rotary_dim = head_size); positions are int32, as the model runner packs them.

    With a nonzero ``llama_4_scaling_beta`` the kernel also applies the reference's llama-4 query
    scale (devstral2.py:175-179) to q in place: afterwards ``query`` holds what the reference's
    ``query_states`` holds after line 179, bit for bit."""
    if torch.compiler.is_compiling():
        k_cache, v_cache = (paged_kv_cache if isinstance(paged_kv_cache, (tuple, list)) else (paged_kv_cache, None))
        torch.ops.mas.apply_rope_and_append_paged_kv_cache(positions, query, key, value, int(head_size),
                                                           cos_sin_cache, bool(is_neox), batch_indices, k_cache,
                                                           v_cache, kv_indices, kv_indptr, kv_layout,
                                                           float(llama_4_scaling_beta),
                                                           int(original_max_position_embeddings), error_flags)
        return
    _fused(positions, query, key, value, head_size, cos_sin_cache, is_neox, batch_indices, paged_kv_cache,
           kv_indices, kv_indptr, kv_layout, error_flags, llama_4_scaling_beta, original_max_position_embeddings)
