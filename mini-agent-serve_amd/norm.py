"""Fused residual add + RMSNorm, mirroring the two ``flashinfer.norm`` calls of the reference.

- ``fused_add_rmsnorm(input, residual, weight, eps, enable_pdl)``: the final norm,
  miniagentserve/models/devstral2/devstral2.py:305-307.
- ``fused_add_rmsnorm_quant(out, input, residual, weight, scale, eps, enable_pdl)``: the two
  in-layer norms feeding the FP8 qkv / gate_up GEMMs, devstral2.py:241-252.

Both update ``residual`` in place to ``bf16(f32(input) + f32(residual))`` and normalise that sum
in fp32. ``enable_pdl`` is accepted and ignored: the overlap it asks for (programmatic dependent
launch) has no gfx950 counterpart, and launches on one stream already serialise correctly.
"""
from __future__ import annotations

import torch

from . import _lib
from ._tensors import require_dtype, require_gpu, require_same_device, rows_view

__all__ = ["fused_add_rmsnorm", "fused_add_rmsnorm_quant"]

FP8 = torch.float8_e4m3fn


def _check_common(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    for name, t in (("input", input), ("residual", residual), ("weight", weight)):
        require_gpu(t, name)
        require_dtype(t, name, torch.bfloat16)
    device = require_same_device(("input", input), ("residual", residual), ("weight", weight))
    hidden = input.shape[-1]
    if weight.dim() != 1 or weight.shape[0] != hidden or (hidden > 1 and weight.stride(0) != 1):
        raise ValueError(f"weight must be a contiguous [{hidden}] vector, got shape {tuple(weight.shape)}")
    if residual.shape != input.shape:
        raise ValueError(f"residual shape {tuple(residual.shape)} != input shape {tuple(input.shape)}")
    if not (eps >= 0.0):
        raise ValueError(f"eps must be non-negative, got {eps}")
    rows, in_stride = rows_view(input, "input")
    _, res_stride = rows_view(residual, "residual")
    return device, rows, hidden, in_stride, res_stride


def _fused_add_rmsnorm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float) -> None:
    device, rows, hidden, in_stride, res_stride = _check_common(input, residual, weight, eps)
    lib = _lib.load()
    st = lib.mas_fused_add_rmsnorm_bf16(input.data_ptr(), in_stride, residual.data_ptr(), res_stride,
                                        weight.data_ptr(), rows, hidden, float(eps), _lib.stream_handle(device))
    _lib.check(st, "fused_add_rmsnorm")


def _fused_add_rmsnorm_quant(out: torch.Tensor, input: torch.Tensor, residual: torch.Tensor,
                             weight: torch.Tensor, scale: torch.Tensor | float, eps: float) -> None:
    device, rows, hidden, in_stride, res_stride = _check_common(input, residual, weight, eps)
    require_gpu(out, "out")
    require_dtype(out, "out", FP8)
    require_same_device(("input", input), ("out", out))
    if out.shape != input.shape:
        raise ValueError(f"out shape {tuple(out.shape)} != input shape {tuple(input.shape)}")
    _, out_stride = rows_view(out, "out")
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
    lib = _lib.load()
    st = lib.mas_fused_add_rmsnorm_quant_fp8(out.data_ptr(), out_stride, input.data_ptr(), in_stride,
                                             residual.data_ptr(), res_stride, weight.data_ptr(), scale_ptr,
                                             scale_host, rows, hidden, float(eps), _lib.stream_handle(device))
    _lib.check(st, "fused_add_rmsnorm_quant")


def fused_add_rmsnorm(input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                      enable_pdl: bool | None = None) -> None:
    """``residual <- input + residual``; ``input <- rmsnorm(residual) * weight``, both in place.

    input, residual: bf16 ``[..., hidden]`` with a contiguous last dimension; weight: bf16 ``[hidden]``.
    """
    if torch.compiler.is_compiling():
        torch.ops.mas.fused_add_rmsnorm(input, residual, weight, float(eps))
        return
    _fused_add_rmsnorm(input, residual, weight, eps)


def fused_add_rmsnorm_quant(out: torch.Tensor, input: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                            scale: torch.Tensor | float, eps: float = 1e-6, enable_pdl: bool | None = None) -> None:
    """``residual <- input + residual``; ``out <- fp8(clamp(rmsnorm(residual) * weight / scale, +-448))``.

    out: ``float8_e4m3fn`` with input's shape; ``input`` is only read. ``scale`` is a one-element
    fp32 device tensor (read by the kernel, no host synchronisation) or a Python float.
    """
    if torch.compiler.is_compiling():
        if isinstance(scale, torch.Tensor):
            torch.ops.mas.fused_add_rmsnorm_quant(out, input, residual, weight, scale, float(eps))
        else:
            torch.ops.mas.fused_add_rmsnorm_quant_hs(out, input, residual, weight, float(scale), float(eps))
        return
    _fused_add_rmsnorm_quant(out, input, residual, weight, scale, eps)
