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
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU device, got {t.device}")


def require_dtype(t: torch.Tensor, name: str, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        expected = " or ".join(str(d) for d in dtypes)
        raise TypeError(f"{name} must be {expected}, got {t.dtype}")


def require_same_device(*named: tuple[str, torch.Tensor]) -> torch.device:
    """The device of the first tensor; raises if another (GPU) tensor is on a different one."""
    first = named[0][1]
    index = first.get_device()
    for name, t in named[1:]:
        if t.get_device() != index or t.is_cuda != first.is_cuda:
            raise ValueError(f"{name} is on {t.device}, expected {first.device} (like {named[0][0]})")
    return first.device


def rows_view(t: torch.Tensor, name: str, width: int | None = None) -> tuple[int, int]:
    """(rows, row_stride) of `t` read as a [rows, t.shape[-1]] matrix.

    The last dimension must be contiguous and the leading dimensions must collapse into one
    strided row index (true for contiguous tensors and for column slices such as the q/k/v
    views of a fused qkv output).
    """
    shape = t.shape
    nd = len(shape)
    if nd == 0:
        raise ValueError(f"{name} must have at least one dimension")
    w = shape[-1]
    if width is not None and w != width:
        raise ValueError(f"{name} last dimension is {w}, expected {width}")
    strides = t.stride()
    if w > 1 and strides[-1] != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension (stride {strides[-1]})")
    if nd == 1:
        return 1, max(w, 1)
    if nd == 2:  # the common case: [rows, w] with any row stride
        return shape[0], (strides[0] if shape[0] > 1 else max(w, 1))
    rows = 1
    for s in shape[:-1]:
        rows *= s
    # Size-1 dimensions carry no stride information; the others must nest: collapsing
    # [..., a, b, w] into rows needs stride(a) == stride(b) * size(b).
    lead = [(shape[i], strides[i]) for i in range(nd - 1) if shape[i] > 1]
    if not lead:
        return rows, max(w, 1)
    for (_, outer), (size, inner) in zip(lead, lead[1:]):
        if outer != inner * size:
            raise ValueError(f"{name}: leading dimensions with shape {tuple(shape)} and strides "
                             f"{strides} cannot be read as one row index")
    return rows, lead[-1][1]


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def error_word(flags: torch.Tensor | None, device: torch.device) -> int | None:
    """Device address of a caller-provided 32-bit error word, or None."""
    if flags is None:
        return None
    require_gpu(flags, "error_flags")
    require_dtype(flags, "error_flags", torch.int32, torch.uint32)
    if flags.get_device() != device.index:
        raise ValueError(f"error_flags is on {flags.device}, expected {device}")
    if flags.numel() < 1:
        raise ValueError("error_flags needs at least one element")
    return flags.data_ptr()
