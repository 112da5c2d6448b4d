"""Argument checks shared by the op wrappers: device, dtype, and strided row views.

The kernels take raw pointers plus element strides with a contiguous innermost dimension, so
each wrapper reduces its tensors to (rows, row_stride) here and rejects anything else with a
ValueError / TypeError before any work is enqueued.
"""
from __future__ import annotations

import torch


def require_gpu(t: torch.Tensor, name: str) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on a GPU device, got {t.device}")


def require_dtype(t: torch.Tensor, name: str, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        expected = " or ".join(str(d) for d in dtypes)
        raise TypeError(f"{name} must be {expected}, got {t.dtype}")


def require_same_device(*named: tuple[str, torch.Tensor]) -> torch.device:
    device = named[0][1].device
    for name, t in named[1:]:
        if t.device != device:
            raise ValueError(f"{name} is on {t.device}, expected {device} (like {named[0][0]})")
    return device


def rows_view(t: torch.Tensor, name: str, width: int | None = None) -> tuple[int, int]:
    """(rows, row_stride) of `t` read as a [rows, t.shape[-1]] matrix.

    The last dimension must be contiguous and the leading dimensions must collapse into one
    strided row index (true for contiguous tensors and for column slices such as the q/k/v
    views of a fused qkv output).
    """
    if t.dim() == 0:
        raise ValueError(f"{name} must have at least one dimension")
    if width is not None and t.shape[-1] != width:
        raise ValueError(f"{name} last dimension is {t.shape[-1]}, expected {width}")
    if t.shape[-1] > 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension (stride {t.stride(-1)})")
    rows = 1
    for s in t.shape[:-1]:
        rows *= s
    # Size-1 dimensions carry no stride information; the others must nest: collapsing
    # [..., a, b, w] into rows needs stride(a) == stride(b) * size(b).
    lead = [(t.shape[i], t.stride(i)) for i in range(t.dim() - 1) if t.shape[i] > 1]
    if not lead:
        return rows, max(t.shape[-1], 1)
    for (_, outer), (size, inner) in zip(lead, lead[1:]):
        if outer != inner * size:
            raise ValueError(f"{name}: leading dimensions with shape {tuple(t.shape)} and strides "
                             f"{t.stride()} cannot be read as one row index")
    return rows, lead[-1][1]


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def error_word(flags: torch.Tensor | None, device: torch.device) -> int | None:
    """Device address of a caller-provided 32-bit error word, or None."""
    if flags is None:
        return None
    require_gpu(flags, "error_flags")
    require_dtype(flags, "error_flags", torch.int32, torch.uint32)
    if flags.device != device:
        raise ValueError(f"error_flags is on {flags.device}, expected {device}")
    if flags.numel() < 1:
        raise ValueError("error_flags needs at least one element")
    return flags.data_ptr()
