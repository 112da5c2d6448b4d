"""torch.library registrations of the ops under the ``mas`` namespace.

The public wrappers call the kernels directly in eager mode (one ctypes call, no dispatcher hop)
and route through these ops only while ``torch.compile`` traces, so a compiled model, like the
reference's ``torch.compile(model, dynamic=True)`` at miniagentserve/engine/model_runner.py:98,
keeps each kernel as one opaque node instead of breaking its graph at a ctypes call.

Every op whose kernel reports out-of-range indices takes the caller's ``error_flags`` word as a
mutated optional argument, so a compiled model reports them as an eager one does. Optional
arguments are passed explicitly by the wrappers (no defaults: the dispatcher's in-place bookkeeping
indexes mutated arguments by position).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch.library import custom_op

from . import activation, attention, embedding, fused, norm, page, rope

Tensor = torch.Tensor


def _cache(k_cache: Tensor, v_cache: Optional[Tensor]):
    """The ops' cache arguments: separate k / v caches, or (v_cache None) one combined
    ``[pages, 2, ...]`` tensor, passed whole so that the compiled graph holds no sub-view of it."""
    return (k_cache, v_cache) if v_cache is not None else k_cache


def _quant_scale(tensor: Optional[Tensor], host: float):
    """The attention ops' fp8 output scale: a device scalar, a positive host float, or none (0)."""
    if tensor is not None:
        return tensor
    return host if host > 0.0 else None


@custom_op("mas::fused_add_rmsnorm", mutates_args=("input", "residual"))
def _fused_add_rmsnorm(input: Tensor, residual: Tensor, weight: Tensor, eps: float) -> None:
    norm._fused_add_rmsnorm(input, residual, weight, eps)


@_fused_add_rmsnorm.register_fake
def _(input, residual, weight, eps):
    return None


@custom_op("mas::fused_add_rmsnorm_quant", mutates_args=("out", "residual"))
def _fused_add_rmsnorm_quant(out: Tensor, input: Tensor, residual: Tensor, weight: Tensor, scale: Tensor,
                             eps: float) -> None:
    norm._fused_add_rmsnorm_quant(out, input, residual, weight, scale, eps)


@_fused_add_rmsnorm_quant.register_fake
def _(out, input, residual, weight, scale, eps):
    return None


@custom_op("mas::fused_add_rmsnorm_quant_hs", mutates_args=("out", "residual"))
def _fused_add_rmsnorm_quant_hs(out: Tensor, input: Tensor, residual: Tensor, weight: Tensor, scale: float,
                                eps: float) -> None:
    norm._fused_add_rmsnorm_quant(out, input, residual, weight, scale, eps)


@_fused_add_rmsnorm_quant_hs.register_fake
def _(out, input, residual, weight, scale, eps):
    return None


@custom_op("mas::silu_and_mul", mutates_args=())
def _silu_and_mul(input: Tensor) -> Tensor:
    out = torch.empty(tuple(input.shape[:-1]) + (input.shape[-1] // 2,), dtype=input.dtype, device=input.device)
    activation._silu_and_mul(input, out)
    return out


@_silu_and_mul.register_fake
def _(input):
    return input.new_empty(tuple(input.shape[:-1]) + (input.shape[-1] // 2,))


@custom_op("mas::silu_and_mul_out", mutates_args=("out",))
def _silu_and_mul_out(input: Tensor, out: Tensor) -> None:
    activation._silu_and_mul(input, out)


@_silu_and_mul_out.register_fake
def _(input, out):
    return None


@custom_op("mas::apply_rope_with_cos_sin_cache_inplace", mutates_args=("query", "key", "error_flags"))
def _apply_rope(positions: Tensor, query: Tensor, key: Tensor, head_size: int, cos_sin_cache: Tensor,
                is_neox: bool, error_flags: Optional[Tensor]) -> None:
    rope._apply_rope(positions, query, key, head_size, cos_sin_cache, is_neox, error_flags)


@_apply_rope.register_fake
def _(positions, query, key, head_size, cos_sin_cache, is_neox, error_flags):
    return None


@custom_op("mas::append_paged_kv_cache", mutates_args=("k_cache", "v_cache", "error_flags"))
def _append_paged_kv_cache(append_key: Tensor, append_value: Tensor, batch_indices: Tensor, positions: Tensor,
                           k_cache: Tensor, v_cache: Optional[Tensor], kv_indices: Tensor, kv_indptr: Tensor,
                           kv_layout: str, error_flags: Optional[Tensor]) -> None:
    page._append(append_key, append_value, batch_indices, positions, _cache(k_cache, v_cache), kv_indices, kv_indptr,
                 kv_layout, error_flags)


@_append_paged_kv_cache.register_fake
def _(append_key, append_value, batch_indices, positions, k_cache, v_cache, kv_indices, kv_indptr, kv_layout,
      error_flags):
    return None


@custom_op("mas::store_kv_slots", mutates_args=("k_cache", "v_cache", "error_flags"))
def _store_kv_slots(key: Tensor, value: Tensor, k_cache: Tensor, v_cache: Tensor, slot_mapping: Tensor,
                    kv_layout: str, error_flags: Optional[Tensor]) -> None:
    page._store_slots(key, value, k_cache, v_cache, slot_mapping, kv_layout, error_flags)


@_store_kv_slots.register_fake
def _(key, value, k_cache, v_cache, slot_mapping, kv_layout, error_flags):
    return None


def _embedding_shape(input_ids: Tensor, weight: Tensor) -> tuple:
    return tuple(input_ids.shape) + (weight.shape[1],)


@custom_op("mas::embedding", mutates_args=("error_flags",))
def _embedding(input_ids: Tensor, weight: Tensor, error_flags: Optional[Tensor]) -> Tensor:
    out = torch.empty(_embedding_shape(input_ids, weight), dtype=weight.dtype, device=weight.device)
    embedding._embedding(input_ids, weight, out, error_flags)
    return out


@_embedding.register_fake
def _(input_ids, weight, error_flags):
    return weight.new_empty(_embedding_shape(input_ids, weight))


@custom_op("mas::embedding_out", mutates_args=("out", "error_flags"))
def _embedding_out(input_ids: Tensor, weight: Tensor, out: Tensor, error_flags: Optional[Tensor]) -> None:
    embedding._embedding(input_ids, weight, out, error_flags)


@_embedding_out.register_fake
def _(input_ids, weight, out, error_flags):
    return None


@custom_op("mas::embedding_fill_placeholders", mutates_args=("input_ids", "error_flags"))
def _embedding_fill(input_ids: Tensor, weight: Tensor, last_tokens: Tensor, error_flags: Optional[Tensor]) -> Tensor:
    out = torch.empty(_embedding_shape(input_ids, weight), dtype=weight.dtype, device=weight.device)
    embedding._embedding(input_ids, weight, out, error_flags, last_tokens)
    return out


@_embedding_fill.register_fake
def _(input_ids, weight, last_tokens, error_flags):
    return weight.new_empty(_embedding_shape(input_ids, weight))


@custom_op("mas::embedding_fill_placeholders_out", mutates_args=("input_ids", "out", "error_flags"))
def _embedding_fill_out(input_ids: Tensor, weight: Tensor, last_tokens: Tensor, out: Tensor,
                        error_flags: Optional[Tensor]) -> None:
    embedding._embedding(input_ids, weight, out, error_flags, last_tokens)


@_embedding_fill_out.register_fake
def _(input_ids, weight, last_tokens, out, error_flags):
    return None


@custom_op("mas::fill_placeholders", mutates_args=("input_ids", "error_flags"))
def _fill(input_ids: Tensor, last_tokens: Tensor, error_flags: Optional[Tensor]) -> None:
    embedding._fill_placeholders(input_ids, last_tokens, error_flags)


@_fill.register_fake
def _(input_ids, last_tokens, error_flags):
    return None


@custom_op("mas::paged_decode_attention", mutates_args=("workspace", "out", "error_flags"))
def _paged_decode_attention(query: Tensor, k_cache: Tensor, v_cache: Optional[Tensor], workspace: Optional[Tensor],
                            block_tables: Tensor,
                            seq_lens: Tensor, bmm1_scale: float, bmm2_scale: float, out: Tensor, kv_layout: str,
                            quant_scale: Optional[Tensor], quant_scale_host: float,
                            error_flags: Optional[Tensor]) -> None:
    attention._decode(query, _cache(k_cache, v_cache), workspace, block_tables, seq_lens, bmm1_scale, bmm2_scale, out,
                      kv_layout, error_flags, _quant_scale(quant_scale, quant_scale_host))


@_paged_decode_attention.register_fake
def _(query, k_cache, v_cache, workspace, block_tables, seq_lens, bmm1_scale, bmm2_scale, out, kv_layout,
      quant_scale, quant_scale_host, error_flags):
    return None


@custom_op("mas::paged_context_attention", mutates_args=("workspace", "out", "error_flags"))
def _paged_context_attention(query: Tensor, k_cache: Tensor, v_cache: Optional[Tensor], workspace: Optional[Tensor],
                             block_tables: Tensor, seq_lens: Tensor,
                             cu_seqlens_q: Tensor, max_q_len: int, max_kv_len: int, bmm1_scale: float,
                             bmm2_scale: float, out: Tensor, kv_layout: str, quant_scale: Optional[Tensor],
                             quant_scale_host: float, error_flags: Optional[Tensor]) -> None:
    attention._context(query, _cache(k_cache, v_cache), block_tables, seq_lens, cu_seqlens_q, max_q_len, bmm1_scale,
                       bmm2_scale, out, kv_layout, error_flags, _quant_scale(quant_scale, quant_scale_host),
                       workspace, max_kv_len)


@_paged_context_attention.register_fake
def _(query, k_cache, v_cache, workspace, block_tables, seq_lens, cu_seqlens_q, max_q_len, max_kv_len, bmm1_scale,
      bmm2_scale, out, kv_layout, quant_scale, quant_scale_host, error_flags):
    return None


@custom_op("mas::apply_rope_and_append_paged_kv_cache",
           mutates_args=("query", "key", "k_cache", "v_cache", "error_flags"))
def _rope_append(positions: Tensor, query: Tensor, key: Tensor, value: Tensor, head_size: int, cos_sin_cache: Tensor,
                 is_neox: bool, batch_indices: Tensor, k_cache: Tensor, v_cache: Optional[Tensor], kv_indices: Tensor,
                 kv_indptr: Tensor, kv_layout: str, llama_4_scaling_beta: float, original_max_position_embeddings: int,
                 error_flags: Optional[Tensor]) -> None:
    fused._fused(positions, query, key, value, head_size, cos_sin_cache, is_neox, batch_indices, _cache(k_cache, v_cache),
                 kv_indices, kv_indptr, kv_layout, error_flags, llama_4_scaling_beta, original_max_position_embeddings)


@_rope_append.register_fake
def _(positions, query, key, value, head_size, cos_sin_cache, is_neox, batch_indices, k_cache, v_cache, kv_indices,
      kv_indptr, kv_layout, llama_4_scaling_beta, original_max_position_embeddings, error_flags):
    return None


@custom_op("mas::silu_and_mul_quant", mutates_args=("out",))
def _silu_and_mul_quant(input: Tensor, out: Tensor, scale: Tensor) -> None:
    activation._silu_and_mul_quant(input, out, scale)


@_silu_and_mul_quant.register_fake
def _(input, out, scale):
    return None


@custom_op("mas::silu_and_mul_quant_hs", mutates_args=("out",))
def _silu_and_mul_quant_hs(input: Tensor, out: Tensor, scale: float) -> None:
    activation._silu_and_mul_quant(input, out, scale)


@_silu_and_mul_quant_hs.register_fake
def _(input, out, scale):
    return None
