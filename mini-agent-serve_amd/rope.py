"""Rotary embedding from a cos/sin table, mirroring
``flashinfer.rope.apply_rope_with_cos_sin_cache_inplace`` as called at
miniagentserve/models/devstral2/devstral2.py:163-166.

The table has one fp32 row per position, ``[cos(p * f_0..f_{R/2-1}), sin(p * f_0..f_{R/2-1})]``
(times any attention scaling folded in by the builder), as produced by ``cos_sin_cache`` below
and by the reference's ``_yarn_cos_sin_cache`` (devstral2.py:44-90). ``rotary_dim`` R is the
table width; the first R elements of each head are rotated and the rest left untouched.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from ._tensors import error_word, require_dtype, require_gpu, require_same_device

__all__ = ["apply_rope_with_cos_sin_cache_inplace", "cos_sin_cache", "yarn_cos_sin_cache", "rope_inv_freq",
           "yarn_inv_freq"]

SUPPORTED_ROTARY_DIMS = (32, 64, 128, 256, 512)


def _head_view(t: torch.Tensor, name: str, head_size: int) -> tuple[int, int, int, int]:
    """(rows, row_stride, head_stride, num_heads) of a [nnz, H*D] or [nnz, H, D] tensor."""
    if t.dim() == 2:
        if t.shape[1] % head_size != 0:
            raise ValueError(f"{name} width {t.shape[1]} is not a multiple of head_size {head_size}")
        if t.shape[1] > 1 and t.stride(1) != 1:
            raise ValueError(f"{name} must be contiguous in its last dimension")
        return t.shape[0], t.stride(0), head_size, t.shape[1] // head_size
    if t.dim() == 3:
        if t.shape[2] != head_size:
            raise ValueError(f"{name} head dimension {t.shape[2]} != head_size {head_size}")
        if head_size > 1 and t.stride(2) != 1:
            raise ValueError(f"{name} must be contiguous in its last dimension")
        return t.shape[0], t.stride(0), t.stride(1), t.shape[1]
    raise ValueError(f"{name} must be [nnz, heads * head_size] or [nnz, heads, head_size], got {tuple(t.shape)}")


def _apply_rope(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor, head_size: int,
                cos_sin_cache: torch.Tensor, is_neox: bool, error_flags: torch.Tensor | None = None) -> None:
    for name, t in (("positions", positions), ("query", query), ("key", key), ("cos_sin_cache", cos_sin_cache)):
        require_gpu(t, name)
    require_dtype(query, "query", torch.bfloat16)
    require_dtype(key, "key", torch.bfloat16)
    require_dtype(cos_sin_cache, "cos_sin_cache", torch.float32)
    require_dtype(positions, "positions", torch.int32, torch.int64)
    device = require_same_device(("query", query), ("key", key), ("positions", positions),
                                 ("cos_sin_cache", cos_sin_cache))
    if positions.dim() != 1 or (positions.numel() > 1 and positions.stride(0) != 1):
        raise ValueError("positions must be a contiguous 1-D tensor")
    if cos_sin_cache.dim() != 2 or (cos_sin_cache.shape[1] > 1 and cos_sin_cache.stride(1) != 1):
        raise ValueError("cos_sin_cache must be [max_position, rotary_dim] with a contiguous last dimension")
    rotary_dim = cos_sin_cache.shape[1]
    if rotary_dim not in SUPPORTED_ROTARY_DIMS:
        raise ValueError(f"rotary_dim (cos_sin_cache width) must be one of {SUPPORTED_ROTARY_DIMS}, got {rotary_dim}")
    if rotary_dim > head_size:
        raise ValueError(f"rotary_dim {rotary_dim} exceeds head_size {head_size}")
    q_rows, q_stride, q_hstride, hq = _head_view(query, "query", head_size)
    k_rows, k_stride, k_hstride, hk = _head_view(key, "key", head_size)
    if not (q_rows == k_rows == positions.shape[0]):
        raise ValueError(f"query rows {q_rows}, key rows {k_rows} and positions {positions.shape[0]} differ")
    st = _lib.load().mas_rope_cos_sin_cache_bf16(
        query.data_ptr(), q_stride, q_hstride, hq, key.data_ptr(), k_stride, k_hstride, hk, positions.data_ptr(),
        int(positions.dtype == torch.int64), cos_sin_cache.data_ptr(), cos_sin_cache.stride(0),
        cos_sin_cache.shape[0], q_rows, head_size, rotary_dim, int(bool(is_neox)), error_word(error_flags, device),
        _lib.stream_handle(device))
    _lib.check(st, "apply_rope_with_cos_sin_cache_inplace")


def apply_rope_with_cos_sin_cache_inplace(positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor,
                                          head_size: int, cos_sin_cache: torch.Tensor, is_neox: bool = True,
                                          *, error_flags: torch.Tensor | None = None) -> None:
    """Rotates every q and k head of each token by its position, in place.

    positions: int32/int64 ``[nnz]``; query/key: bf16 ``[nnz, heads * head_size]`` or
    ``[nnz, heads, head_size]``, any row stride (column slices of a fused qkv output are fine);
    cos_sin_cache: fp32 ``[max_position, rotary_dim]``. ``is_neox`` selects rotate-half pairs
    (i, i + R/2); otherwise interleaved pairs (2i, 2i + 1). A position outside the table leaves
    that token untouched and, when ``error_flags`` (a 1-element int32 device tensor) is given,
    sets bit 2 in it.
    """
    if torch.compiler.is_compiling():
        torch.ops.mas.apply_rope_with_cos_sin_cache_inplace(positions, query, key, int(head_size), cos_sin_cache,
                                                            bool(is_neox), error_flags)
        return
    _apply_rope(positions, query, key, head_size, cos_sin_cache, is_neox, error_flags)


def rope_inv_freq(rotary_dim: int, theta: float) -> torch.Tensor:
    """Plain RoPE inverse frequencies ``theta ** (-2i / rotary_dim)`` in fp32 (CPU)."""
    return 1.0 / (theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))


def yarn_inv_freq(rotary_dim: int, theta: float, factor: float, original_max_position: int,
                  beta_fast: float = 32.0, beta_slow: float = 1.0, mscale: float = 0.0, mscale_all_dim: float = 0.0,
                  truncate: bool = True) -> tuple[torch.Tensor, float]:
    """YaRN inverse frequencies (fp32, CPU) and attention scaling with the reference's parameters
    (devstral2.py:44-85; the config fields come from configs.py:33-43): frequencies blended between
    extrapolation and interpolation by a linear ramp over the correction range."""

    def get_mscale(scale: float, m: float = 1.0) -> float:
        return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0

    def correction_dim(num_rotations: float) -> float:
        return (rotary_dim * math.log(original_max_position / (num_rotations * 2 * math.pi))) / (2 * math.log(theta))

    low, high = correction_dim(beta_fast), correction_dim(beta_slow)
    if truncate:
        low, high = math.floor(low), math.ceil(high)
    low, high = max(low, 0), min(high, rotary_dim - 1)
    if low == high:
        high += 0.001
    pos_freqs = theta ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim)
    extrapolation = 1.0 / pos_freqs
    interpolation = 1.0 / (factor * pos_freqs)
    ramp = torch.clamp((torch.arange(rotary_dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
    keep = 1 - ramp
    inv_freq = interpolation * (1 - keep) + extrapolation * keep
    if mscale and mscale_all_dim:
        scaling = get_mscale(factor, mscale) / get_mscale(factor, mscale_all_dim)
    else:
        scaling = get_mscale(factor)
    return inv_freq, scaling


def cos_sin_cache(max_position: int, rotary_dim: int, theta: float = 1e6, scaling: float = 1.0,
                  inv_freq: torch.Tensor | None = None) -> torch.Tensor:
    """RoPE table on the CPU, fp32 ``[max_position, rotary_dim]``: row p is
    ``cat(cos(p f), sin(p f)) * scaling``, with ``f = rope_inv_freq(rotary_dim, theta)`` unless
    ``inv_freq`` is given. Angles are formed in fp32, like devstral2.py:87-90."""
    if inv_freq is None:
        inv_freq = rope_inv_freq(rotary_dim, theta)
    positions = torch.arange(max_position, dtype=torch.float32)
    freqs = positions[:, None] * inv_freq.float()
    table = torch.cat((freqs.cos(), freqs.sin()), dim=-1)
    return table * scaling if scaling != 1.0 else table


def yarn_cos_sin_cache(max_position: int, rotary_dim: int, theta: float, factor: float,
                       original_max_position: int, beta_fast: float = 32.0, beta_slow: float = 1.0,
                       mscale: float = 0.0, mscale_all_dim: float = 0.0, truncate: bool = True) -> torch.Tensor:
    """The reference's YaRN table (``_yarn_cos_sin_cache``, devstral2.py:44-90)."""
    inv_freq, scaling = yarn_inv_freq(rotary_dim, theta, factor, original_max_position, beta_fast, beta_slow, mscale,
                                      mscale_all_dim, truncate)
    positions = torch.arange(max_position, dtype=torch.float32)
    freqs = positions[:, None] * inv_freq
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1) * scaling
