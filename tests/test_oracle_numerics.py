"""Pins the oracle's bf16 and fp8-e4m3fn codecs bit for bit against torch's dtype conversions."""
from __future__ import annotations

import numpy as np
import torch

from oracle import numerics as on


def _torch_bf16_bits(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _torch_fp8_codes(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_bf16_decode_exhaustive():
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = torch.from_numpy(codes.view(np.int16)).view(torch.bfloat16).float().numpy()
    got = on.bf16_to_f32(codes)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_bf16_encode_matches_torch_on_random_and_special_values():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32),
        rng.uniform(-1e38, 1e38, 20_000).astype(np.float32),
        # every fp32 bit pattern with a random upper half: covers ties (low half 0x8000) and both parities
        (rng.integers(0, 1 << 16, 50_000, dtype=np.uint32) << 16 | rng.integers(0, 1 << 16, 50_000,
                                                                              dtype=np.uint32)).view(np.float32),
        (rng.integers(0, 1 << 16, 20_000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, np.inf, -np.inf, 3.3895314e38, -3.3895314e38, 1e-45, -1e-45, 1.17549435e-38],
                 dtype=np.float32),
    ])
    finite = ~np.isnan(x)
    assert np.array_equal(on.f32_to_bf16(x[finite]), _torch_bf16_bits(x[finite]))
    nan_bits = on.f32_to_bf16(np.array([np.nan, -np.nan], dtype=np.float32))
    assert np.all(np.isnan(on.bf16_to_f32(nan_bits)))


def test_fp8_decode_exhaustive():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = on.fp8_to_f32(codes)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok], want[ok])
    assert on.FP8_VALUES[0x7E] == 448.0 and on.FP8_VALUES[0x01] == 2.0 ** -9


def test_fp8_encode_matches_torch_after_clamp():
    """The reference quantizes as (x / scale).clamp(-448, 448).to(float8_e4m3fn) (devstral2.py:93-95)."""
    rng = np.random.default_rng(1)
    vals = on.FP8_VALUES[np.isfinite(on.FP8_VALUES)].astype(np.float64)
    pos = np.unique(np.abs(vals))
    mids = (pos[1:] + pos[:-1]) / 2                        # exact ties between neighbours
    x = np.concatenate([
        rng.standard_normal(100_000) * 50,
        rng.uniform(-600, 600, 50_000),
        rng.uniform(-2 ** -5, 2 ** -5, 50_000),               # subnormal region
        vals, mids, -mids, np.nextafter(mids, 0), np.nextafter(mids, 1000),
        [0.0, -0.0, 448.0, -448.0, 449.0, 464.0, 1e30, -1e30, np.inf, -np.inf],
    ]).astype(np.float32)
    want = _torch_fp8_codes(np.clip(x, -448.0, 448.0))
    got = on.f32_to_fp8_saturate(x)
    assert np.array_equal(got, want)


def test_fp8_encode_nan_keeps_sign():
    got = on.f32_to_fp8_saturate(np.array([np.nan, -np.nan], dtype=np.float32))
    want = _torch_fp8_codes(np.clip(np.array([np.nan, -np.nan], dtype=np.float32), -448, 448))
    assert np.all(np.isnan(on.fp8_to_f32(got)))
    assert got[0] == 0x7F and got[1] == 0xFF
    assert np.all(np.isnan(on.fp8_to_f32(want)))


def test_fp8_encode_dense_sweep_of_bf16_inputs():
    """Every bf16 value (the precision the norm's fp32 result is formed from) in [-512, 512]."""
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    x = on.bf16_to_f32(codes)
    x = x[np.isfinite(x) & (np.abs(x) <= 512)]
    assert np.array_equal(on.f32_to_fp8_saturate(x), _torch_fp8_codes(np.clip(x, -448, 448)))
