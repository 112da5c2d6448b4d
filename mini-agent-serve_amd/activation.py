"""SiluAndMul, mirroring ``flashinfer.activation.silu_and_mul`` as called at
miniagentserve/models/devstral2/devstral2.py:224.

``out[..., i] = silu(input[..., i]) * input[..., d + i]`` for ``i < d``, ``2d = input.shape[-1]``:
the gate half comes first and the up half second (the concat order at devstral2.py:364).
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import require_dtype, require_gpu, require_same_device, rows_view

__all__ = ["silu_and_mul"]


def _silu_and_mul(input: torch.Tensor, out: torch.Tensor) -> None:
    require_gpu(input, "input")
    require_gpu(out, "out")
    require_dtype(input, "input", torch.bfloat16)
    require_dtype(out, "out", torch.bfloat16)
    device = require_same_device(("input", input), ("out", out))
    width = input.shape[-1]
    if width % 2 != 0:
        raise ValueError(f"input last dimension must be even, got {width}")
    inter = width // 2
    if tuple(out.shape) != tuple(input.shape[:-1]) + (inter,):
        raise ValueError(f"out shape {tuple(out.shape)} != {tuple(input.shape[:-1]) + (inter,)}")
    rows, in_stride = rows_view(input, "input")
    _, out_stride = rows_view(out, "out")
    st = _lib.load().mas_silu_and_mul_bf16(out.data_ptr(), out_stride, input.data_ptr(), in_stride, rows, inter,
                                           _lib.stream_handle(device))
    _lib.check(st, "silu_and_mul")


def silu_and_mul(input: torch.Tensor, out: torch.Tensor | None = None, enable_pdl: bool | None = None) -> torch.Tensor:
    """Returns ``out`` (allocated when not given): bf16 ``[..., d]`` from bf16 ``[..., 2d]``.

    ``enable_pdl`` is accepted and ignored (no programmatic dependent launch on gfx950).
    """
    if torch.compiler.is_compiling():
        if out is None:
            return torch.ops.mas.silu_and_mul(input)
        torch.ops.mas.silu_and_mul_out(input, out)
        return out
    if out is None:
        out = torch.empty(tuple(input.shape[:-1]) + (input.shape[-1] // 2,), dtype=input.dtype, device=input.device)
    _silu_and_mul(input, out)
    return out
