"""Oracle restatement of the hot-path ops - test infrastructure (see oracle/__init__.py).

Every function takes and returns numpy arrays; bf16 tensors are uint16 bit patterns and fp8 tensors
uint8 codes (oracle.numerics). "fp32 math" means: widen each bf16 to fp32, compute in fp32 in the
order written, round once to the output format.
"""
from __future__ import annotations

import math

import numpy as np

from .numerics import bf16_to_f32, f32_to_bf16, f32_to_fp8_saturate

F32 = np.float32


def _rms_normalise(x_bits: np.ndarray, r_bits: np.ndarray, w_bits: np.ndarray, eps: float):
    x = bf16_to_f32(x_bits)
    r = bf16_to_f32(r_bits)
    w = bf16_to_f32(w_bits)
    s = x + r                                                   # fp32 sum of two bf16, exact order-free
    hidden = s.shape[-1]
    mean_sq = np.sum(s * s, axis=-1, dtype=F32, keepdims=True) / F32(hidden)
    rstd = F32(1.0) / np.sqrt(mean_sq + F32(eps), dtype=F32)
    y = (s * rstd) * w
    return s, y


def fused_add_rmsnorm(x_bits, r_bits, w_bits, eps: float):
    """Final norm, devstral2.py:305-307 (flashinfer.norm.fused_add_rmsnorm, in place):
    s = f32(x) + f32(r); r' = bf16(s); x' = bf16((s * rsqrt(mean(s^2) + eps)) * f32(w)).
    Returns (x', r') as bf16 bit patterns."""
    s, y = _rms_normalise(x_bits, r_bits, w_bits, eps)
    return f32_to_bf16(y), f32_to_bf16(s)


def fused_add_rmsnorm_quant(x_bits, r_bits, w_bits, scale: float, eps: float):
    """In-layer norms, devstral2.py:241-252 (flashinfer.norm.fused_add_rmsnorm_quant): the same s
    and r', and out = e4m3fn(clamp(y / scale, -448, 448)) with y as above; the division by the
    activation scale follows the reference's own quantize at devstral2.py:93-95.
    Returns (out codes, r')."""
    s, y = _rms_normalise(x_bits, r_bits, w_bits, eps)
    q = y / F32(scale)
    return f32_to_fp8_saturate(q), f32_to_bf16(s)


def silu_and_mul(x_bits):
    """devstral2.py:224 (flashinfer.activation.silu_and_mul): gate = first half of the last
    dimension, up = second half (concat order devstral2.py:364);
    out = bf16((g / (1 + exp(-g))) * u)."""
    d = x_bits.shape[-1] // 2
    g = bf16_to_f32(x_bits[..., :d])
    u = bf16_to_f32(x_bits[..., d:])
    with np.errstate(over="ignore"):
        e = np.exp(-g, dtype=F32)
    y = (g / (F32(1.0) + e)) * u
    return f32_to_bf16(y)


def quantize_activation(y_bits, scale: float):
    """The quantize FP8Linear.forward applies to a bf16 input (devstral2.py:93-95,110-111):
    e4m3fn(clamp(f32(y) / scale, -448, 448)). Returns fp8 codes."""
    with np.errstate(invalid="ignore"):
        return f32_to_fp8_saturate(bf16_to_f32(y_bits) / F32(scale))


def silu_and_mul_quant(x_bits, scale: float):
    """SiluAndMul (devstral2.py:224) followed by the quantize down_proj applies to its bf16 result
    (devstral2.py:93-95,110-111). Returns fp8 codes."""
    return quantize_activation(silu_and_mul(x_bits), scale)


def rope(q_bits, k_bits, positions, table, is_neox: bool = True):
    """devstral2.py:163-166 (flashinfer.rope.apply_rope_with_cos_sin_cache_inplace).

    q_bits [N, Hq, D], k_bits [N, Hk, D] (bf16 bits); table fp32 [P, R] = [cos | sin].
    NeoX pairs (i, i + R/2), GPT-J pairs (2i, 2i + 1), each with c = T[p, i], s = T[p, R/2 + i]:
    a' = bf16(a*c - b*s), b' = bf16(b*c + a*s). Head elements past R are copied unchanged.
    Returns the rotated (q, k)."""
    table = np.asarray(table, dtype=F32)
    rot = table.shape[1]
    half = rot // 2
    pos = np.asarray(positions, dtype=np.int64)
    c = table[pos, :half][:, None, :]
    s = table[pos, half:rot][:, None, :]

    def apply(bits):
        out = np.array(bits, dtype=np.uint16, copy=True)
        x = bf16_to_f32(bits[..., :rot])
        if is_neox:
            a, b = x[..., :half], x[..., half:]
        else:
            a, b = x[..., 0::2], x[..., 1::2]
        ya = a * c - b * s
        yb = b * c + a * s
        if is_neox:
            out[..., :half] = f32_to_bf16(ya)
            out[..., half:rot] = f32_to_bf16(yb)
        else:
            out[..., 0:rot:2] = f32_to_bf16(ya)
            out[..., 1:rot:2] = f32_to_bf16(yb)
        return out

    return apply(q_bits), apply(k_bits)


def llama_4_q_scale_table(beta: float, original_max_position: int, rows: int) -> np.ndarray:
    """devstral2.py:176-178 on k = floor(pos / original_max) (an integer, so floor(pos.float() /
    original_max) = pos // original_max for pos < 2^24): bf16(1 + f32(beta) * f32(log1p(k))), with
    log1p evaluated in fp64 and rounded to fp32. Returns bf16 bits [rows]."""
    k = np.arange(rows, dtype=np.float64)
    lg = np.log1p(k).astype(F32)
    return f32_to_bf16(F32(1.0) + F32(beta) * lg)


def llama_4_scale_q(q_bits, positions, scale_table, original_max_position: int):
    """devstral2.py:179: q * bf16(scale)[:, None, None] in bf16 arithmetic:
    bf16(f32(q) * f32(S[pos // original_max])). q_bits [N, Hq, D]; returns bf16 bits."""
    pos = np.asarray(positions, dtype=np.int64)
    s = bf16_to_f32(np.asarray(scale_table, dtype=np.uint16)[pos // original_max_position])
    return f32_to_bf16(bf16_to_f32(q_bits) * s[:, None, None])


def paged_destinations(batch_indices, positions, kv_indices, kv_indptr, page_size: int):
    """(page, entry) per token for the block-table form, devstral2.py:170-173 with kv_indptr from
    :289: page = kv_indices[kv_indptr[b] + p // page_size], entry = p % page_size."""
    b = np.asarray(batch_indices, dtype=np.int64)
    p = np.asarray(positions, dtype=np.int64)
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    page = np.asarray(kv_indices, dtype=np.int64)[indptr[b] + p // page_size]
    return page, p % page_size


def append_paged_kv_cache(k_cache, v_cache, key, value, batch_indices, positions, kv_indices, kv_indptr):
    """NHD caches [pages, page_size, heads, dim]; key/value [N, heads, dim]. Returns updated copies.
    With duplicate destinations the later token wins here (the GPU allows any writer to win)."""
    page_size = k_cache.shape[1]
    page, entry = paged_destinations(batch_indices, positions, kv_indices, kv_indptr, page_size)
    k_out, v_out = k_cache.copy(), v_cache.copy()
    k_out[page, entry] = key
    v_out[page, entry] = value
    return k_out, v_out


def store_kv_slots(k_cache, v_cache, key, value, slot_mapping):
    """Slot form: page = slot // page_size, entry = slot % page_size; negative slots skipped."""
    page_size = k_cache.shape[1]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = slots >= 0
    k_out, v_out = k_cache.copy(), v_cache.copy()
    k_out[slots[keep] // page_size, slots[keep] % page_size] = key[keep]
    v_out[slots[keep] // page_size, slots[keep] % page_size] = value[keep]
    return k_out, v_out


def paged_decode_attention(q_bits, k_cache_bits, v_cache_bits, block_tables, seq_lens, bmm1_scale: float,
                           bmm2_scale: float = 1.0):
    """trtllm_batch_decode_with_kv_cache (devstral2.py:184-196) on NHD caches [pages, page_size, Hk, D]:
    for row b, query head h (kv head h // (Hq // Hk)) and positions p < seq_lens[b] at page
    block_tables[b, p // page_size], entry p % page_size:
    out = bf16(bmm2_scale * sum_p softmax_p(bmm1_scale * q . k_p) v_p), fp32 math. Rows with no
    position give zeros. q_bits [B, Hq, D]; returns bf16 bits [B, Hq, D]."""
    q = bf16_to_f32(np.asarray(q_bits))
    batch, hq, dim = q.shape
    page_size, hk = k_cache_bits.shape[1], k_cache_bits.shape[2]
    group = hq // hk
    tables = np.asarray(block_tables, dtype=np.int64)
    out = np.zeros((batch, hq, dim), dtype=np.uint16)
    for b in range(batch):
        length = int(seq_lens[b])
        if length <= 0:
            continue
        pos = np.arange(length)
        pages = tables[b, pos // page_size]
        k = bf16_to_f32(k_cache_bits[pages, pos % page_size])          # [L, Hk, D]
        v = bf16_to_f32(v_cache_bits[pages, pos % page_size])
        for h in range(hq):
            kvh = h // group
            s = (k[:, kvh, :] @ q[b, h]).astype(F32) * F32(bmm1_scale)
            e = np.exp(s - s.max(), dtype=F32)
            o = (e @ v[:, kvh, :]).astype(F32) / np.sum(e, dtype=F32) * F32(bmm2_scale)
            out[b, h] = f32_to_bf16(o.astype(F32))
    return out


def paged_context_attention(q_bits, k_cache_bits, v_cache_bits, block_tables, seq_lens, cu_seqlens_q,
                            bmm1_scale: float, bmm2_scale: float = 1.0):
    """trtllm_batch_context_with_kv_cache (devstral2.py:198-213): row j owns query tokens
    cu[j]:cu[j+1] (q_len) and kv_len = seq_lens[j] positions; token i sits at kv_len - q_len + i and
    attends to positions 0..that (causal, aligned to the end). fp32 math, output rounded to bf16;
    tokens left before position 0 give zeros. q_bits [tokens, Hq, D]; returns bf16 bits."""
    q = bf16_to_f32(np.asarray(q_bits))
    tokens, hq, dim = q.shape
    page_size, hk = k_cache_bits.shape[1], k_cache_bits.shape[2]
    group = hq // hk
    tables = np.asarray(block_tables, dtype=np.int64)
    cu = np.asarray(cu_seqlens_q, dtype=np.int64)
    out = np.zeros((tokens, hq, dim), dtype=np.uint16)
    for j in range(len(cu) - 1):
        q0, q_len, kv_len = int(cu[j]), int(cu[j + 1] - cu[j]), int(seq_lens[j])
        if q_len <= 0 or kv_len <= 0:
            continue
        pos = np.arange(kv_len)
        pages = tables[j, pos // page_size]
        k = bf16_to_f32(k_cache_bits[pages, pos % page_size])
        v = bf16_to_f32(v_cache_bits[pages, pos % page_size])
        for i in range(q_len):
            qpos = kv_len - q_len + i
            if qpos < 0:
                continue
            for h in range(hq):
                kvh = h // group
                s = (k[: qpos + 1, kvh, :] @ q[q0 + i, h]).astype(F32) * F32(bmm1_scale)
                e = np.exp(s - s.max(), dtype=F32)
                o = (e @ v[: qpos + 1, kvh, :]).astype(F32) / np.sum(e, dtype=F32) * F32(bmm2_scale)
                out[q0 + i, h] = f32_to_bf16(o.astype(F32))
    return out


def embedding(weight_bits, ids):
    """nn.Embedding at devstral2.py:260,282: rows of the table selected by the ids."""
    return np.asarray(weight_bits)[np.asarray(ids, dtype=np.int64)]


def fill_placeholders(ids, last_tokens):
    """ModelRunner.fill_placeholders (model_runner.py:149-154): every id -1 - r becomes
    last_tokens[r]; other ids stay. Returns the new int64 ids."""
    ids = np.asarray(ids, dtype=np.int64)
    last = np.asarray(last_tokens, dtype=np.int64)
    rows = np.clip(-1 - ids, 0, None)
    return np.where(ids < 0, last[rows], ids)


def rope_inv_freq(rotary_dim: int, theta: float) -> np.ndarray:
    """Plain RoPE inverse frequencies theta^(-2i/R), computed in fp64 and rounded to fp32."""
    i = np.arange(0, rotary_dim, 2, dtype=np.float64)
    return (1.0 / theta ** (i / rotary_dim)).astype(F32)


def yarn_inv_freq_and_scaling(rotary_dim: int, theta: float, factor: float, original_max_position: int,
                              beta_fast: float, beta_slow: float, mscale: float, mscale_all_dim: float,
                              truncate: bool) -> tuple[np.ndarray, float]:
    """YaRN inverse frequencies and attention scaling as devstral2.py:44-85 defines them
    (fp64 here; the reference's torch code works in fp32)."""

    def mscale_of(scale: float, m: float = 1.0) -> float:
        return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0

    def dim_for(rotations: float) -> float:
        return rotary_dim * math.log(original_max_position / (rotations * 2 * math.pi)) / (2 * math.log(theta))

    lo, hi = dim_for(beta_fast), dim_for(beta_slow)
    if truncate:
        lo, hi = math.floor(lo), math.ceil(hi)
    lo, hi = max(lo, 0), min(hi, rotary_dim - 1)
    if lo == hi:
        hi += 0.001
    base = theta ** (np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim)
    ramp = np.clip((np.arange(rotary_dim // 2, dtype=np.float64) - lo) / (hi - lo), 0.0, 1.0)
    inv = (1.0 / (factor * base)) * ramp + (1.0 / base) * (1.0 - ramp)
    if mscale and mscale_all_dim:
        scaling = mscale_of(factor, mscale) / mscale_of(factor, mscale_all_dim)
    else:
        scaling = mscale_of(factor)
    return inv, scaling


def cos_sin_table(max_position: int, inv_freq: np.ndarray, scaling: float = 1.0) -> np.ndarray:
    """[max_position, R] fp32: row p = [cos(p f), sin(p f)] * scaling, angles formed in fp32 like
    devstral2.py:88-90 and evaluated in fp64 before rounding."""
    p = np.arange(max_position, dtype=F32)[:, None]
    ang = (p * np.asarray(inv_freq, dtype=F32)[None, :]).astype(np.float64)
    table = np.concatenate([np.cos(ang), np.sin(ang)], axis=1) * scaling
    return table.astype(F32)
