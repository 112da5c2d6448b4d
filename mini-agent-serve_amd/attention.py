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

Both functions can also write the o_proj input directly: with ``out_quant_scale`` (the o_proj
``activation_scale``, a one-element fp32 device tensor or a Python float), ``out`` is
``float8_e4m3fn`` and holds ``fp8(clamp(bf16(out) / out_quant_scale, -448, 448))``, the quantize
``FP8Linear.forward`` applies to the attention output (devstral2.py:93-95,110-111).
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device
from .page import _cache_geometry

__all__ = ["trtllm_batch_decode_with_kv_cache", "trtllm_batch_context_with_kv_cache", "decode_workspace_bytes",
           "context_workspace_bytes"]

SUPPORTED_HEAD_DIMS = (64, 128, 256)
FP8 = torch.float8_e4m3fn


def _quant_args(quant_scale, device) -> tuple[int, int | None, float]:
    """(out_fp8, scale pointer, host scale) for the C entry points."""
    if quant_scale is None:
        return 0, None, 0.0
    if isinstance(quant_scale, torch.Tensor):
        require_gpu(quant_scale, "out_quant_scale")
        require_dtype(quant_scale, "out_quant_scale", torch.float32)
        if quant_scale.device != device:
            raise ValueError(f"out_quant_scale is on {quant_scale.device}, expected {device}")
        if quant_scale.numel() != 1:
            raise ValueError(f"out_quant_scale must hold one value, got shape {tuple(quant_scale.shape)}")
        return 1, quant_scale.data_ptr(), 0.0
    value = float(quant_scale)
    if not value > 0.0:
        raise ValueError(f"out_quant_scale must be positive, got {value}")
    return 1, None, value


def _out_dtype(out_dtype, quant_scale) -> torch.dtype:
    if out_dtype is None:
        return torch.bfloat16 if quant_scale is None else FP8
    if out_dtype not in (torch.bfloat16, FP8):
        raise ValueError(f"out_dtype must be bfloat16 or float8_e4m3fn, got {out_dtype}")
    if (out_dtype == FP8) != (quant_scale is not None):
        raise ValueError("a float8_e4m3fn output needs out_quant_scale, and out_quant_scale needs one")
    return out_dtype


def _custom_op_scale(quant_scale) -> tuple[torch.Tensor | None, float]:
    if isinstance(quant_scale, torch.Tensor):
        return quant_scale, 0.0
    return None, (0.0 if quant_scale is None else float(quant_scale))


def decode_workspace_bytes(batch: int, num_q_heads: int, head_dim: int, max_blocks: int, page_size: int,
                           chunks_per_split: int = 1) -> int:
    """Workspace bytes the kernel needs for splits of ``chunks_per_split`` chunks of 256 positions
    (1: the most parallel split; a smaller workspace, more than 64 splits per row or more than
    16384 (row, kv head, split) work items make the kernel pick longer splits)."""
    n = _lib.load().mas_paged_decode_attention_workspace_bytes(batch, num_q_heads, head_dim, max_blocks, page_size,
                                                                chunks_per_split)
    if n < 0:
        raise ValueError("invalid attention shape")
    return n


def context_workspace_bytes(num_rows: int, max_q_len: int, num_q_heads: int, num_kv_heads: int,
                            head_dim: int) -> int:
    """Workspace bytes with which context attention splits every small grid of these sizes the
    most (32 splits per token tile); a smaller workspace gets fewer splits or none."""
    n = _lib.load().mas_paged_context_attention_workspace_bytes(num_rows, max_q_len, num_q_heads, num_kv_heads,
                                                                 head_dim)
    if n < 0:
        raise ValueError("invalid attention shape")
    return n


def _decode(query, kv_cache, workspace_buffer, block_tables, seq_lens, bmm1_scale, bmm2_scale, out, kv_layout,
            error_flags, quant_scale=None) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, hk, dim = _cache_geometry(kv_cache, kv_layout)
    for name, t in (("query", query), ("out", out), ("block_tables", block_tables), ("seq_lens", seq_lens)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16 if quant_scale is None else FP8)
    require_dtype(block_tables, "block_tables", torch.int32)
    require_dtype(seq_lens, "seq_lens", torch.int32)
    device = require_same_device(("query", query), ("k_cache", k_cache), ("out", out),
                                 ("block_tables", block_tables), ("seq_lens", seq_lens))
    if workspace_buffer is not None:
        require_gpu(workspace_buffer, "workspace_buffer")
        require_same_device(("query", query), ("workspace_buffer", workspace_buffer))
    out_fp8, scale_ptr, scale_host = _quant_args(quant_scale, device)
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
    args = (out.data_ptr(), out.stride(0), out.stride(1), query.data_ptr(), query.stride(0), query.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, block_tables.data_ptr(),
            block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(), batch, hq, hk, dim, float(bmm1_scale),
            float(bmm2_scale), out_fp8, scale_ptr, scale_host)
    if workspace_buffer is None:
        # the library's own scratch: no allocation in the call (graph capture, allocation-free loops)
        st = _lib.load().mas_paged_decode_attention_bf16_noalloc(*args, error_word(error_flags, device),
                                                                 _lib.stream_handle(device))
    else:
        nbytes = workspace_buffer.numel() * workspace_buffer.element_size()
        st = _lib.load().mas_paged_decode_attention_bf16(*args, workspace_buffer.data_ptr(), nbytes,
                                                         error_word(error_flags, device), _lib.stream_handle(device))
    _lib.check(st, "trtllm_batch_decode_with_kv_cache")


def trtllm_batch_decode_with_kv_cache(query: torch.Tensor, kv_cache, workspace_buffer: torch.Tensor | None,
                                      block_tables: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int,
                                      bmm1_scale: float = 1.0, bmm2_scale: float = 1.0, window_left: int = -1,
                                      out: torch.Tensor | None = None, out_dtype=None, o_sf_scale=None,
                                      o_sf_vec_size=None, sinks=None, kv_layout: str = "NHD",
                                      enable_pdl: bool | None = None, *,
                                      out_quant_scale: torch.Tensor | float | None = None,
                                      error_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Decode attention of one query token per row over its paged KV. Returns ``out`` (allocated when
    not given), bf16 ``[batch, num_q_heads, head_dim]``, or its fp8 quantize with ``out_quant_scale``.

    ``kv_cache`` is ``(k_cache, v_cache)`` or one ``[pages, 2, ...]`` tensor, in ``kv_layout``.
    ``workspace_buffer=None`` uses the library's own scratch instead (no allocation in the call;
    at most ``MAS_DECODE_ATTENTION_SCRATCH_BYTES`` of partials, one buffer per GPU shared by every
    such call, so such calls must not overlap on two streams of one GPU).
    ``max_seq_len`` is accepted and unused: the reach of ``block_tables`` bounds the positions.
    Not supported (raise): a sliding window, attention sinks, block-scaled outputs.
    ``enable_pdl`` is ignored. ``error_flags`` as for the other ops (page 8, seq_len 2).
    """
    if window_left != -1:
        raise ValueError("sliding-window attention (window_left != -1) is not supported")
    if sinks is not None or o_sf_scale is not None or o_sf_vec_size is not None:
        raise ValueError("attention sinks and block-scaled outputs are not supported")
    dtype = _out_dtype(out_dtype, out_quant_scale)
    if isinstance(bmm1_scale, torch.Tensor) or isinstance(bmm2_scale, torch.Tensor):
        raise TypeError("bmm1_scale and bmm2_scale must be Python floats")
    del max_seq_len, enable_pdl
    if out is None:
        out = torch.empty(query.shape, dtype=dtype, device=query.device)
    if torch.compiler.is_compiling():
        k_cache, v_cache = (kv_cache if isinstance(kv_cache, (tuple, list)) else (kv_cache, None))
        qs, qs_host = _custom_op_scale(out_quant_scale)
        torch.ops.mas.paged_decode_attention(query, k_cache, v_cache, workspace_buffer, block_tables, seq_lens,
                                             float(bmm1_scale), float(bmm2_scale), out, kv_layout, qs, qs_host,
                                             error_flags)
        return out
    _decode(query, kv_cache, workspace_buffer, block_tables, seq_lens, bmm1_scale, bmm2_scale, out, kv_layout,
            error_flags, out_quant_scale)
    return out


def _context(query, kv_cache, block_tables, seq_lens, cu_seqlens_q, max_q_len, bmm1_scale, bmm2_scale, out,
             kv_layout, error_flags, quant_scale=None, workspace=None, max_kv_len=0) -> None:
    k_cache, v_cache, pstride, estride, hstride, pages, page_size, hk, dim = _cache_geometry(kv_cache, kv_layout)
    for name, t in (("query", query), ("out", out), ("block_tables", block_tables), ("seq_lens", seq_lens),
                    ("cum_seq_lens_q", cu_seqlens_q)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16 if quant_scale is None else FP8)
    for name, t in (("block_tables", block_tables), ("seq_lens", seq_lens), ("cum_seq_lens_q", cu_seqlens_q)):
        require_dtype(t, name, torch.int32)
    device = require_same_device(("query", query), ("k_cache", k_cache), ("out", out),
                                 ("block_tables", block_tables), ("seq_lens", seq_lens),
                                 ("cum_seq_lens_q", cu_seqlens_q))
    out_fp8, scale_ptr, scale_host = _quant_args(quant_scale, device)
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
    ws_ptr, ws_bytes = None, 0
    if workspace is not None:
        require_gpu(workspace, "workspace_buffer")
        require_same_device(("query", query), ("workspace_buffer", workspace))
        if not workspace.is_contiguous():
            raise ValueError("workspace_buffer must be contiguous")
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    st = _lib.load().mas_paged_context_attention_bf16(
        out.data_ptr(), out.stride(0), out.stride(1), query.data_ptr(), query.stride(0), query.stride(1),
        k_cache.data_ptr(), v_cache.data_ptr(), pstride, estride, hstride, pages, page_size, block_tables.data_ptr(),
        block_tables.stride(0), block_tables.shape[1], seq_lens.data_ptr(), cu_seqlens_q.data_ptr(), rows,
        int(max_q_len), int(max_kv_len), hq, hk, dim, float(bmm1_scale), float(bmm2_scale), out_fp8, scale_ptr, scale_host, ws_ptr,
        ws_bytes, error_word(error_flags, device), _lib.stream_handle(device))
    _lib.check(st, "trtllm_batch_context_with_kv_cache")


def trtllm_batch_context_with_kv_cache(query: torch.Tensor, kv_cache, workspace_buffer: torch.Tensor,
                                       block_tables: torch.Tensor, seq_lens: torch.Tensor, max_q_len: int,
                                       max_kv_len: int, bmm1_scale: float, bmm2_scale: float, batch_size: int,
                                       cum_seq_lens_q: torch.Tensor, cum_seq_lens_kv: torch.Tensor | None = None,
                                       window_left: int = -1, out: torch.Tensor | None = None, out_dtype=None,
                                       o_sf_scale=None, o_sf_vec_size=None, kv_layout: str = "NHD",
                                       enable_pdl: bool | None = None, sinks=None, *,
                                       out_quant_scale: torch.Tensor | float | None = None,
                                       error_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Causal attention of ``batch_size`` prompt rows (row j: query tokens
    ``cum_seq_lens_q[j]:cum_seq_lens_q[j + 1]``, the last ``q_len`` of its ``seq_lens[j]`` cached
    positions) over their paged KV. Returns ``out`` (allocated when not given), bf16
    ``[tokens, num_q_heads, head_dim]``, or its fp8 quantize with ``out_quant_scale``.

    ``max_q_len`` must bound every row's query length (it sizes the grid); ``cum_seq_lens_kv`` is
    accepted and unused. ``workspace_buffer`` (or None) holds split-KV partials when the grid is
    small (few new tokens after a long cached prefix): each token tile's key range is then split
    over several workgroups and merged by a second kernel; its contents on entry do not matter, and
    with too little of it the kernel splits less or not at all. ``max_kv_len`` is a hint for the
    choice of the split count (each row divides its own positions among the splits). Not
    supported (raise): a sliding window, attention sinks, block-scaled outputs. ``enable_pdl`` is
    ignored.
    """
    if window_left != -1:
        raise ValueError("sliding-window attention (window_left != -1) is not supported")
    if sinks is not None or o_sf_scale is not None or o_sf_vec_size is not None:
        raise ValueError("attention sinks and block-scaled outputs are not supported")
    dtype = _out_dtype(out_dtype, out_quant_scale)
    if isinstance(bmm1_scale, torch.Tensor) or isinstance(bmm2_scale, torch.Tensor):
        raise TypeError("bmm1_scale and bmm2_scale must be Python floats")
    if cum_seq_lens_q.shape[0] != batch_size + 1:
        raise ValueError(f"cum_seq_lens_q has {cum_seq_lens_q.shape[0]} entries, expected batch_size + 1")
    del cum_seq_lens_kv, enable_pdl
    if out is None:
        out = torch.empty(query.shape, dtype=dtype, device=query.device)
    if torch.compiler.is_compiling():
        k_cache, v_cache = (kv_cache if isinstance(kv_cache, (tuple, list)) else (kv_cache, None))
        qs, qs_host = _custom_op_scale(out_quant_scale)
        torch.ops.mas.paged_context_attention(query, k_cache, v_cache, workspace_buffer, block_tables, seq_lens,
                                              cum_seq_lens_q, int(max_q_len), int(max_kv_len), float(bmm1_scale),
                                              float(bmm2_scale), out, kv_layout, qs, qs_host, error_flags)
        return out
    _context(query, kv_cache, block_tables, seq_lens, cum_seq_lens_q, max_q_len, bmm1_scale, bmm2_scale, out,
             kv_layout, error_flags, out_quant_scale, workspace_buffer, max_kv_len)
    return out
