"""SiluAndMul, mirroring ``flashinfer.activation.silu_and_mul`` as called at
miniagentserve/models/devstral2/devstral2.py:224.

``out[..., i] = silu(input[..., i]) * input[..., d + i]`` for ``i < d``, ``2d = input.shape[-1]``:
the gate half comes first and the up half second (the concat order at devstral2.py:364).
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import require_dtype, require_gpu, require_same_device, rows_view

__all__ = ["silu_and_mul", "silu_and_mul_quant"]

FP8 = torch.float8_e4m3fn


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


def _silu_and_mul_quant(input: torch.Tensor, out: torch.Tensor, scale: torch.Tensor | float) -> None:
    require_gpu(input, "input")
    require_gpu(out, "out")
    require_dtype(input, "input", torch.bfloat16)
    require_dtype(out, "out", FP8)
    device = require_same_device(("input", input), ("out", out))
    width = input.shape[-1]
    if width % 2 != 0:
        raise ValueError(f"input last dimension must be even, got {width}")
    inter = width // 2
    if tuple(out.shape) != tuple(input.shape[:-1]) + (inter,):
        raise ValueError(f"out shape {tuple(out.shape)} != {tuple(input.shape[:-1]) + (inter,)}")
    scale_ptr, scale_host = None, 1.0
    if isinstance(scale, torch.Tensor):
        require_gpu(scale, "scale")
        require_dtype(scale, "scale", torch.float32)
        require_same_device(("input", input), ("scale", scale))
        if scale.numel() != 1:
            raise ValueError(f"scale must hold one value, got shape {tuple(scale.shape)}")
        scale_ptr = scale.data_ptr()
    else:
        scale_host = float(scale)
    rows, in_stride = rows_view(input, "input")
    _, out_stride = rows_view(out, "out")
    st = _lib.load().mas_silu_and_mul_quant_fp8(out.data_ptr(), out_stride, input.data_ptr(), in_stride, rows, inter,
                                                scale_ptr, scale_host, _lib.stream_handle(device))
    _lib.check(st, "silu_and_mul_quant")


def silu_and_mul_quant(input: torch.Tensor, scale: torch.Tensor | float, out: torch.Tensor | None = None,
                       enable_pdl: bool | None = None) -> torch.Tensor:
    """SiluAndMul followed by the fp8 quantize the down projection applies to its input
    (devstral2.py:93-95,110-111,224), in one pass: returns ``float8_e4m3fn [..., d]`` with
    ``out = fp8(clamp(bf16(silu(gate) * up) / scale, -448, 448))``. ``scale`` is a one-element fp32
    device tensor (the layer's ``activation_scale``) or a Python float."""
    if torch.compiler.is_compiling():
        if out is None:
            out = torch.empty(tuple(input.shape[:-1]) + (input.shape[-1] // 2,), dtype=FP8, device=input.device)
        if isinstance(scale, torch.Tensor):
            torch.ops.mas.silu_and_mul_quant(input, out, scale)
        else:
            torch.ops.mas.silu_and_mul_quant_hs(input, out, float(scale))
        return out
    if out is None:
        out = torch.empty(tuple(input.shape[:-1]) + (input.shape[-1] // 2,), dtype=FP8, device=input.device)
    _silu_and_mul_quant(input, out, scale)
    return out
