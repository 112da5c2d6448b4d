"""Paged KV-cache append, mirroring ``flashinfer.page.append_paged_kv_cache`` as called at
miniagentserve/models/devstral2/devstral2.py:170-173, plus the equivalent slot-mapping store.

Cache layout (miniagentserve/engine/model_runner.py:83-85): per layer ``[num_pages, page_size,
kv_heads, head_dim]`` for "NHD", ``[num_pages, kv_heads, page_size, head_dim]`` for "HND". The
model runner keeps one extra page as a sink for padding rows (model_runner.py:82), so duplicate
destinations within one call are legal; the kernel lets one writer win.
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device

__all__ = ["append_paged_kv_cache", "store_kv_slots", "slot_mapping_from_block_tables"]


def _cache_geometry(paged_kv_cache, kv_layout: str):
    """(k_cache, v_cache, page_stride, entry_stride, head_stride, num_pages, page_size, heads, dim)."""
    if kv_layout not in ("NHD", "HND"):
        raise ValueError(f"kv_layout must be 'NHD' or 'HND', got {kv_layout!r}")
    if isinstance(paged_kv_cache, (tuple, list)):
        if len(paged_kv_cache) != 2:
            raise ValueError("paged_kv_cache tuple must be (k_cache, v_cache)")
        k_cache, v_cache = paged_kv_cache
    else:
        t = paged_kv_cache
        if t.dim() != 5 or t.shape[1] != 2:
            raise ValueError("a single paged_kv_cache tensor must be [num_pages, 2, ...] (k at index 0, v at 1)")
        k_cache, v_cache = t[:, 0], t[:, 1]
    for name, c in (("k_cache", k_cache), ("v_cache", v_cache)):
        require_gpu(c, name)
        require_dtype(c, name, torch.bfloat16)
        if c.dim() != 4:
            raise ValueError(f"{name} must be 4-D, got shape {tuple(c.shape)}")
        if c.shape[3] > 1 and c.stride(3) != 1:
            raise ValueError(f"{name} must be contiguous in head_dim")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise ValueError("k_cache and v_cache must have the same shape and strides")
    if kv_layout == "NHD":
        num_pages, page_size, heads, dim = k_cache.shape
        page_stride, entry_stride, head_stride = k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)
    else:
        num_pages, heads, page_size, dim = k_cache.shape
        page_stride, entry_stride, head_stride = k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)
    return k_cache, v_cache, page_stride, entry_stride, head_stride, num_pages, page_size, heads, dim


def _source_view(t: torch.Tensor, name: str, heads: int, dim: int) -> tuple[int, int, int]:
    """(rows, row_stride, head_stride) of [nnz, heads, dim] or [nnz, heads * dim] k/v rows."""
    require_gpu(t, name)
    require_dtype(t, name, torch.bfloat16)
    if t.dim() == 3:
        if tuple(t.shape[1:]) != (heads, dim):
            raise ValueError(f"{name} shape {tuple(t.shape)} does not match the cache's ({heads}, {dim}) heads")
        if dim > 1 and t.stride(2) != 1:
            raise ValueError(f"{name} must be contiguous in head_dim")
        return t.shape[0], t.stride(0), t.stride(1)
    if t.dim() == 2:
        if t.shape[1] != heads * dim:
            raise ValueError(f"{name} width {t.shape[1]} != kv_heads * head_dim = {heads * dim}")
        if t.shape[1] > 1 and t.stride(1) != 1:
            raise ValueError(f"{name} must be contiguous in its last dimension")
        return t.shape[0], t.stride(0), dim
    raise ValueError(f"{name} must be [nnz, kv_heads, head_dim] or [nnz, kv_heads * head_dim]")


def _index_vector(t: torch.Tensor, name: str, dtype: torch.dtype) -> None:
    require_gpu(t, name)
    require_dtype(t, name, dtype)
    if t.dim() != 1 or (t.numel() > 1 and t.stride(0) != 1):
        raise ValueError(f"{name} must be a contiguous 1-D tensor")


def _append(append_key, append_value, batch_indices, positions, paged_kv_cache, kv_indices, kv_indptr,
            kv_layout: str, error_flags: torch.Tensor | None) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, heads, dim = _cache_geometry(paged_kv_cache,
                                                                                                kv_layout)
    rows, ks, khs = _source_view(append_key, "append_key", heads, dim)
    vrows, vs, vhs = _source_view(append_value, "append_value", heads, dim)
    for name, t in (("batch_indices", batch_indices), ("positions", positions), ("kv_indices", kv_indices),
                    ("kv_indptr", kv_indptr)):
        _index_vector(t, name, torch.int32)
    device = require_same_device(("append_key", append_key), ("append_value", append_value), ("k_cache", k_cache),
                                 ("batch_indices", batch_indices), ("positions", positions),
                                 ("kv_indices", kv_indices), ("kv_indptr", kv_indptr))
    if not (vrows == rows == batch_indices.shape[0] == positions.shape[0]):
        raise ValueError("append_key, append_value, batch_indices and positions must have the same length")
    if kv_indptr.shape[0] < 1:
        raise ValueError("kv_indptr needs batch + 1 entries")
    st = _lib.load().mas_append_paged_kv_cache_bf16(
        k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, append_key.data_ptr(),
        ks, khs, append_value.data_ptr(), vs, vhs, batch_indices.data_ptr(), positions.data_ptr(),
        kv_indices.data_ptr(), kv_indices.shape[0], kv_indptr.data_ptr(), kv_indptr.shape[0] - 1, rows, heads, dim,
        error_word(error_flags, device), _lib.stream_handle(device))
    _lib.check(st, "append_paged_kv_cache")


def append_paged_kv_cache(append_key: torch.Tensor, append_value: torch.Tensor, batch_indices: torch.Tensor,
                          positions: torch.Tensor, paged_kv_cache, kv_indices: torch.Tensor,
                          kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor | None = None,
                          kv_layout: str = "NHD", *, error_flags: torch.Tensor | None = None) -> None:
    """Writes token t's k/v rows to page ``kv_indices[kv_indptr[b] + p // page_size]``, entry
    ``p % page_size``, where ``b = batch_indices[t]`` and ``p = positions[t]``.

    append_key/append_value: bf16 ``[nnz, kv_heads, head_dim]`` (any row stride, e.g. views of a
    fused qkv output); paged_kv_cache: ``(k_cache, v_cache)`` or one ``[num_pages, 2, ...]``
    tensor; index tensors int32. ``kv_last_page_len`` is accepted for signature compatibility
    and not needed by the store. Tokens whose destination is out of range are skipped; with
    ``error_flags`` (a 1-element int32 device tensor) the kernel records why (bits 2/4/8).
    """
    if torch.compiler.is_compiling():
        k_cache, v_cache = (paged_kv_cache if isinstance(paged_kv_cache, (tuple, list)) else (paged_kv_cache, None))
        torch.ops.mas.append_paged_kv_cache(append_key, append_value, batch_indices, positions, k_cache, v_cache,
                                            kv_indices, kv_indptr, kv_layout, error_flags)
        return
    _append(append_key, append_value, batch_indices, positions, paged_kv_cache, kv_indices, kv_indptr, kv_layout,
            error_flags)


def _store_slots(key, value, k_cache, v_cache, slot_mapping, kv_layout: str, error_flags) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, heads, dim = _cache_geometry((k_cache, v_cache),
                                                                                                kv_layout)
    rows, ks, khs = _source_view(key, "key", heads, dim)
    vrows, vs, vhs = _source_view(value, "value", heads, dim)
    _index_vector(slot_mapping, "slot_mapping", torch.int64)
    device = require_same_device(("key", key), ("value", value), ("k_cache", k_cache), ("slot_mapping", slot_mapping))
    if not (vrows == rows == slot_mapping.shape[0]):
        raise ValueError("key, value and slot_mapping must have the same length")
    st = _lib.load().mas_store_kv_slots_bf16(
        k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, key.data_ptr(), ks, khs,
        value.data_ptr(), vs, vhs, slot_mapping.data_ptr(), rows, heads, dim, error_word(error_flags, device),
        _lib.stream_handle(device))
    _lib.check(st, "store_kv_slots")


def store_kv_slots(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                   slot_mapping: torch.Tensor, kv_layout: str = "NHD", *,
                   error_flags: torch.Tensor | None = None) -> None:
    """Slot-mapping form of the store: token t goes to page ``slot // page_size``, entry
    ``slot % page_size`` with ``slot = slot_mapping[t]`` (int64); a negative slot is skipped."""
    if torch.compiler.is_compiling():
        torch.ops.mas.store_kv_slots(key, value, k_cache, v_cache, slot_mapping, kv_layout, error_flags)
        return
    _store_slots(key, value, k_cache, v_cache, slot_mapping, kv_layout, error_flags)


def slot_mapping_from_block_tables(block_tables: torch.Tensor, batch_indices: torch.Tensor, positions: torch.Tensor,
                                   page_size: int) -> torch.Tensor:
    """``slot[t] = block_tables[b, p // page_size] * page_size + p % page_size`` (int64), the slot
    that the block-table form of the store resolves for token t (devstral2.py:170-173,289)."""
    b = batch_indices.long()
    p = positions.long()
    return block_tables[b, p // page_size].long() * page_size + p % page_size
