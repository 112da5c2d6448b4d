"""Token-embedding gather, the drop-in for ``nn.Embedding`` at
miniagentserve/models/devstral2/devstral2.py:260,282.

``out[t, :] = weight[input_ids[t], :]``, a bit copy. With tied embeddings the table is shared with
lm_head (devstral2.py:317-318), so the op only reads it.

With ``last_tokens`` the gather also does the step-input path's placeholder resolution
(``ModelRunner.fill_placeholders``, miniagentserve/engine/model_runner.py:149-154): an id ``-1 - r``
stands for ``last_tokens[r]``, the previous step's sample still on the GPU, and is replaced by it in
``input_ids`` before its row is gathered - one launch for what the reference does in six.
"""
from __future__ import annotations

import torch
from torch import nn

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device

__all__ = ["embedding", "fill_placeholders", "Embedding"]


def _check_last_tokens(last_tokens: torch.Tensor, input_ids: torch.Tensor) -> None:
    require_gpu(last_tokens, "last_tokens")
    require_dtype(last_tokens, "last_tokens", torch.int32)
    require_same_device(("input_ids", input_ids), ("last_tokens", last_tokens))
    if not last_tokens.is_contiguous():
        raise ValueError("last_tokens must be contiguous")


def _fill_placeholders(input_ids: torch.Tensor, last_tokens: torch.Tensor,
                       error_flags: torch.Tensor | None = None) -> None:
    require_gpu(input_ids, "input_ids")
    require_dtype(input_ids, "input_ids", torch.int64)
    _check_last_tokens(last_tokens, input_ids)
    if not input_ids.is_contiguous():
        raise ValueError("input_ids must be contiguous")
    device = input_ids.device
    st = _lib.load().mas_embedding_fill_placeholders_bf16(None, 0, None, 0, 0, input_ids.data_ptr(), input_ids.numel(),
                                                          0, last_tokens.data_ptr(), last_tokens.numel(),
                                                          error_word(error_flags, device), _lib.stream_handle(device))
    _lib.check(st, "fill_placeholders")


def fill_placeholders(input_ids: torch.Tensor, last_tokens: torch.Tensor, *,
                      error_flags: torch.Tensor | None = None) -> None:
    """``ModelRunner.fill_placeholders`` (model_runner.py:149-154) in one launch: every id ``-1 - r``
    in int64 ``input_ids`` becomes ``last_tokens[r]`` (int32 samples), in place. A placeholder with
    ``r >= len(last_tokens)`` is left as is and sets bit 32 of ``error_flags``."""
    if torch.compiler.is_compiling():
        torch.ops.mas.fill_placeholders(input_ids, last_tokens, error_flags)
        return
    _fill_placeholders(input_ids, last_tokens, error_flags)


def _embedding(input_ids: torch.Tensor, weight: torch.Tensor, out: torch.Tensor,
               error_flags: torch.Tensor | None = None, last_tokens: torch.Tensor | None = None) -> None:
    require_gpu(input_ids, "input_ids")
    require_gpu(weight, "weight")
    require_gpu(out, "out")
    require_dtype(input_ids, "input_ids", torch.int64)
    require_dtype(weight, "weight", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16)
    device = require_same_device(("input_ids", input_ids), ("weight", weight), ("out", out))
    if weight.dim() != 2 or (weight.shape[1] > 1 and weight.stride(1) != 1):
        raise ValueError(f"weight must be [vocab, hidden] with a contiguous last dimension, got {tuple(weight.shape)}")
    vocab, hidden = weight.shape
    if not input_ids.is_contiguous():
        raise ValueError("input_ids must be contiguous")
    rows = input_ids.numel()
    if tuple(out.shape) != tuple(input_ids.shape) + (hidden,) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {tuple(input_ids.shape) + (hidden,)} tensor")
    if last_tokens is not None:
        _check_last_tokens(last_tokens, input_ids)
        st = _lib.load().mas_embedding_fill_placeholders_bf16(
            out.data_ptr(), hidden, weight.data_ptr(), weight.stride(0), vocab, input_ids.data_ptr(), rows, hidden,
            last_tokens.data_ptr(), last_tokens.numel(), error_word(error_flags, device), _lib.stream_handle(device))
    else:
        st = _lib.load().mas_embedding_bf16(out.data_ptr(), hidden, weight.data_ptr(), weight.stride(0), vocab,
                                            input_ids.data_ptr(), rows, hidden, error_word(error_flags, device),
                                            _lib.stream_handle(device))
    _lib.check(st, "embedding")


def embedding(input_ids: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None, *,
              last_tokens: torch.Tensor | None = None, error_flags: torch.Tensor | None = None) -> torch.Tensor:
    """Rows of ``weight`` (bf16 ``[vocab, hidden]``) selected by int64 ``input_ids``.

    An id outside ``[0, vocab)`` yields a zero row instead of reading out of bounds; with
    ``error_flags`` (a 1-element int32 device tensor) the kernel also sets bit 1 in it.
    With ``last_tokens`` (int32 samples of the previous step) placeholders ``-1 - r`` are first
    resolved to ``last_tokens[r]`` and written back into ``input_ids``, as ``fill_placeholders``.
    """
    if torch.compiler.is_compiling():
        if out is None:
            if last_tokens is not None:
                return torch.ops.mas.embedding_fill_placeholders(input_ids, weight, last_tokens, error_flags)
            return torch.ops.mas.embedding(input_ids, weight, error_flags)
        if last_tokens is not None:
            torch.ops.mas.embedding_fill_placeholders_out(input_ids, weight, last_tokens, out, error_flags)
        else:
            torch.ops.mas.embedding_out(input_ids, weight, out, error_flags)
        return out
    if out is None:
        out = torch.empty(tuple(input_ids.shape) + (weight.shape[1],), dtype=weight.dtype, device=weight.device)
    _embedding(input_ids, weight, out, error_flags, last_tokens)
    return out


class Embedding(nn.Module):
    """``nn.Embedding(num_embeddings, embedding_dim)`` whose forward is the HIP gather."""

    def __init__(self, num_embeddings: int, embedding_dim: int, device=None, dtype=torch.bfloat16):
        super().__init__()
        self.num_embeddings = num_embeddings
        self.embedding_dim = embedding_dim
        self.weight = nn.Parameter(torch.empty(num_embeddings, embedding_dim, device=device, dtype=dtype),
                                   requires_grad=False)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return embedding(input_ids, self.weight)

    def extra_repr(self) -> str:
        return f"{self.num_embeddings}, {self.embedding_dim}"
