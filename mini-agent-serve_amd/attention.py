"""Paged attention over the KV cache the append kernels write: the drop-ins for
``flashinfer.decode.trtllm_batch_decode_with_kv_cache`` and
``flashinfer.prefill.trtllm_batch_context_with_kv_cache`` as called at
miniagentserve/models/devstral2/devstral2.py:184-196 and :198-213.

For decode row ``b`` and query head ``h`` (kv head ``h // (Hq // Hk)``), over the positions
``p < seq_lens[b]`` whose rows sit at page ``block_tables[b, p // page_size]``, entry
``p % page_size``::

    out[b, h] = bmm2_scale * sum_p softmax_p(bmm1_scale * q[b, h] . k_p) * v_p

computed in fp32 from the bf16 inputs and rounded once to bf16. The work is split over the
sequence (split-KV); the per-split partials live in the caller's ``workspace_buffer``, as with
flashinfer (the reference passes a 128 MiB buffer, devstral2.py:36-42).
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device
from .page import _cache_geometry

__all__ = ["trtllm_batch_decode_with_kv_cache", "trtllm_batch_context_with_kv_cache", "decode_workspace_bytes"]

SUPPORTED_HEAD_DIMS = (64, 128, 256)


def decode_workspace_bytes(batch: int, num_q_heads: int, head_dim: int, max_blocks: int, page_size: int,
                           chunks_per_split: int = 1) -> int:
    """Workspace bytes the kernel needs for splits of ``chunks_per_split`` chunks of 256 positions
    (1: the most parallel split; a smaller workspace makes the kernel pick longer splits)."""
    n = _lib.load().mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size,
                                                                chunks_per_split)
    if n < 0:
        raise ValueError("invalid attention shape")
    return n


def _decode(query, kv_cache, workspace_buffer, block_tables, seq_lens, bmm1_scale, bmm2_scale, out, kv_layout,
            error_flags) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, hk, dim = _cache_geometry(kv_cache, kv_layout)
    for name, t in (("query", query), ("out", out), ("block_tables", block_tables), ("seq_lens", seq_lens),
                    ("workspace_buffer", workspace_buffer)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16)
    require_dtype(block_tables, "block_tables", torch.int32)
    require_dtype(seq_lens, "seq_lens", torch.int32)
    device = require_same_device(("query", query), ("k_cache", k_cache), ("out", out),
                                 ("block_tables", block_tables), ("seq_lens", seq_lens),
                                 ("workspace_buffer", workspace_buffer))
    if query.dim() != 3 or query.shape[2] != dim or (dim > 1 and query.stride(2) != 1):
        raise ValueError(f"query must be [batch, num_q_heads, {dim}] with a contiguous last dimension, "
                         f"got {tuple(query.shape)}")
    batch, hq = query.shape[0], query.shape[1]
    if tuple(out.shape) != tuple(query.shape) or (dim > 1 and out.stride(2) != 1):
        raise ValueError(f"out must be {tuple(query.shape)} with a contiguous last dimension")
    if dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {SUPPORTED_HEAD_DIMS}, got {dim}")
    if hk == 0 or hq % hk != 0 or hq // hk > 16:
        raise ValueError(f"num_q_heads {hq} must be a multiple of num_kv_heads {hk}, at most 16 per kv head")
    if page_size & (page_size - 1):
        raise ValueError(f"page_size must be a power of two, got {page_size}")
    if block_tables.dim() != 2 or block_tables.shape[0] < batch or (block_tables.shape[1] > 1 and
                                                                    block_tables.stride(1) != 1):
        raise ValueError("block_tables must be [batch, max_blocks] int32 with a contiguous last dimension")
    if seq_lens.dim() != 1 or seq_lens.shape[0] < batch or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 [batch] tensor")
    nbytes = workspace_buffer.numel() * workspace_buffer.element_size()
    st = _lib.load().mas_paged_decode_attention_bf16(
        out.data_ptr(), out.stride(0), out.stride(1), query.data_ptr(), query.stride(0), query.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, block_tables.data_ptr(),
        block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(), batch, hq, hk, dim, float(bmm1_scale),
        float(bmm2_scale), workspace_buffer.data_ptr(), nbytes, error_word(error_flags, device),
        _lib.stream_handle(device))
    _lib.check(st, "trtllm_batch_decode_with_kv_cache")


def trtllm_batch_decode_with_kv_cache(query: torch.Tensor, kv_cache, workspace_buffer: torch.Tensor,
                                      block_tables: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int,
                                      bmm1_scale: float = 1.0, bmm2_scale: float = 1.0, window_left: int = -1,
                                      out: torch.Tensor | None = None, out_dtype=None, o_sf_scale=None,
                                      o_sf_vec_size=None, sinks=None, kv_layout: str = "NHD",
                                      enable_pdl: bool | None = None, *,
                                      error_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of one query token per row over its paged KV. Returns ``out`` (allocated when
    not given), bf16 ``[batch, num_q_heads, head_dim]``.

    ``kv_cache`` is ``(k_cache, v_cache)`` or one ``[pages, 2, ...]`` tensor, in ``kv_layout``.
    ``max_seq_len`` is accepted and unused: the reach of ``block_tables`` bounds the positions.
    Not supported (raise): a sliding window, attention sinks, non-bf16 or block-scaled outputs.
    ``enable_pdl`` is ignored. ``error_flags`` as for the other ops (page 8, seq_len 2).
    """
    if window_left != -1:
        raise ValueError("sliding-window attention (window_left != -1) is not supported")
    if sinks is not None or o_sf_scale is not None or o_sf_vec_size is not None:
        raise ValueError("attention sinks and block-scaled outputs are not supported")
    if out_dtype not in (None, torch.bfloat16):
        raise ValueError(f"out_dtype must be bfloat16, got {out_dtype}")
    if isinstance(bmm1_scale, torch.Tensor) or isinstance(bmm2_scale, torch.Tensor):
        raise TypeError("bmm1_scale and bmm2_scale must be Python floats")
    del max_seq_len, enable_pdl
    if torch.compiler.is_compiling():
        k_cache, v_cache = (kv_cache if isinstance(kv_cache, (tuple, list)) else (kv_cache[:, 0], kv_cache[:, 1]))
        if out is None:
            out = torch.empty_like(query)
        torch.ops.mas.paged_decode_attention(query, k_cache, v_cache, workspace_buffer, block_tables, seq_lens,
                                             float(bmm1_scale), float(bmm2_scale), out, kv_layout)
        return out
    if out is None:
        out = torch.empty(query.shape, dtype=torch.bfloat16, device=query.device)
    _decode(query, kv_cache, workspace_buffer, block_tables, seq_lens, bmm1_scale, bmm2_scale, out, kv_layout,
            error_flags)
    return out


def _context(query, kv_cache, block_tables, seq_lens, cu_seqlens_q, max_q_len, bmm1_scale, bmm2_scale, out,
             kv_layout, error_flags) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, hk, dim = _cache_geometry(kv_cache, kv_layout)
    for name, t in (("query", query), ("out", out), ("block_tables", block_tables), ("seq_lens", seq_lens),
                    ("cum_seq_lens_q", cu_seqlens_q)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16)
    for name, t in (("block_tables", block_tables), ("seq_lens", seq_lens), ("cum_seq_lens_q", cu_seqlens_q)):
        require_dtype(t, name, torch.int32)
    device = require_same_device(("query", query), ("k_cache", k_cache), ("out", out),
                                 ("block_tables", block_tables), ("seq_lens", seq_lens),
                                 ("cum_seq_lens_q", cu_seqlens_q))
    if query.dim() != 3 or query.shape[2] != dim or (dim > 1 and query.stride(2) != 1):
        raise ValueError(f"query must be [tokens, num_q_heads, {dim}] with a contiguous last dimension, "
                         f"got {tuple(query.shape)}")
    hq = query.shape[1]
    if tuple(out.shape) != tuple(query.shape) or (dim > 1 and out.stride(2) != 1):
        raise ValueError(f"out must be {tuple(query.shape)} with a contiguous last dimension")
    if dim not in (64, 128):
        raise ValueError(f"head_dim must be 64 or 128 for context attention, got {dim}")
    if hk == 0 or hq % hk != 0:
        raise ValueError(f"num_q_heads {hq} must be a multiple of num_kv_heads {hk}")
    if page_size & (page_size - 1):
        raise ValueError(f"page_size must be a power of two, got {page_size}")
    rows = cu_seqlens_q.shape[0] - 1
    if cu_seqlens_q.dim() != 1 or rows < 0 or not cu_seqlens_q.is_contiguous():
        raise ValueError("cum_seq_lens_q must be a contiguous int32 [rows + 1] tensor")
    if block_tables.dim() != 2 or block_tables.shape[0] < rows or (block_tables.shape[1] > 1 and
                                                                   block_tables.stride(1) != 1):
        raise ValueError("block_tables must be [rows, max_blocks] int32 with a contiguous last dimension")
    if seq_lens.dim() != 1 or seq_lens.shape[0] < rows or not seq_lens.is_contiguous():
        raise ValueError("seq_lens must be a contiguous int32 [rows] tensor")
    st = _lib.load().mas_paged_context_attention_bf16(
        out.data_ptr(), out.stride(0), out.stride(1), query.data_ptr(), query.stride(0), query.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, block_tables.data_ptr(),
        block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(), cu_seqlens_q.data_ptr(), rows,
        int(max_q_len), hq, hk, dim, float(bmm1_scale), float(bmm2_scale), error_word(error_flags, device),
        _lib.stream_handle(device))
    _lib.check(st, "trtllm_batch_context_with_kv_cache")


def trtllm_batch_context_with_kv_cache(query: torch.Tensor, kv_cache, workspace_buffer: torch.Tensor,
                                       block_tables: torch.Tensor, seq_lens: torch.Tensor, max_q_len: int,
                                       max_kv_len: int, bmm1_scale: float, bmm2_scale: float, batch_size: int,
                                       cum_seq_lens_q: torch.Tensor, cum_seq_lens_kv: torch.Tensor | None = None,
                                       window_left: int = -1, out: torch.Tensor | None = None, out_dtype=None,
                                       o_sf_scale=None, o_sf_vec_size=None, kv_layout: str = "NHD",
                                       enable_pdl: bool | None = None, sinks=None, *,
                                       error_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Causal attention of ``batch_size`` prompt rows (row j: query tokens
    ``cum_seq_lens_q[j]:cum_seq_lens_q[j + 1]``, the last ``q_len`` of its ``seq_lens[j]`` cached
    positions) over their paged KV. Returns ``out`` (allocated when not given), bf16
    ``[tokens, num_q_heads, head_dim]``.

    ``max_q_len`` must bound every row's query length (it sizes the grid); ``max_kv_len``,
    ``cum_seq_lens_kv`` and ``workspace_buffer`` are accepted and unused (the kernel needs no
    workspace). Not supported (raise): a sliding window, attention sinks, non-bf16 or block-scaled
    outputs. ``enable_pdl`` is ignored.
    """
    if window_left != -1:
        raise ValueError("sliding-window attention (window_left != -1) is not supported")
    if sinks is not None or o_sf_scale is not None or o_sf_vec_size is not None:
        raise ValueError("attention sinks and block-scaled outputs are not supported")
    if out_dtype not in (None, torch.bfloat16):
        raise ValueError(f"out_dtype must be bfloat16, got {out_dtype}")
    if isinstance(bmm1_scale, torch.Tensor) or isinstance(bmm2_scale, torch.Tensor):
        raise TypeError("bmm1_scale and bmm2_scale must be Python floats")
    if cum_seq_lens_q.shape[0] != batch_size + 1:
        raise ValueError(f"cum_seq_lens_q has {cum_seq_lens_q.shape[0]} entries, expected batch_size + 1")
    del workspace_buffer, max_kv_len, cum_seq_lens_kv, enable_pdl
    if torch.compiler.is_compiling():
        k_cache, v_cache = (kv_cache if isinstance(kv_cache, (tuple, list)) else (kv_cache[:, 0], kv_cache[:, 1]))
        if out is None:
            out = torch.empty_like(query)
        torch.ops.mas.paged_context_attention(query, k_cache, v_cache, block_tables, seq_lens, cum_seq_lens_q,
                                              int(max_q_len), float(bmm1_scale), float(bmm2_scale), out, kv_layout)
        return out
    if out is None:
        out = torch.empty(query.shape, dtype=torch.bfloat16, device=query.device)
    _context(query, kv_cache, block_tables, seq_lens, cum_seq_lens_q, max_q_len, bmm1_scale, bmm2_scale, out,
             kv_layout, error_flags)
    return out
