"""Pins each oracle op against an independent computation: a library routine (torch, transformers),
a closed form, an invariant, or brute force on tiny inputs. A dropped term, a swapped half, a
wrong sign or a wrong index in the oracle fails at least one of these.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import ATOL, RTOL, bits, from_bits
from oracle import numerics as on
from oracle import ops

BF16_ULP_REL = 2.0 ** -7   # one bf16 ulp relative to the value, an upper bound for rounding differences


def _randn_bf16(gen, *shape, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(*shape, generator=gen)).bfloat16()


# ---- RMSNorm ------------------------------------------------------------------------------------

@pytest.mark.parametrize("rows,hidden", [(1, 8), (7, 64), (33, 5120), (4, 12288)])
def test_rmsnorm_matches_torch_rms_norm(rows, hidden):
    g = torch.Generator().manual_seed(rows * 1000 + hidden)
    x, r = _randn_bf16(g, rows, hidden), _randn_bf16(g, rows, hidden)
    w = _randn_bf16(g, hidden, scale=0.1, shift=1.0)
    got_x, got_r = ops.fused_add_rmsnorm(bits(x), bits(r), bits(w), 1e-5)

    s = x.float() + r.float()
    # residual: torch's bf16 add widens, adds in fp32 and rounds once - bit-exact
    assert np.array_equal(got_r, bits(x + r))
    want = F.rms_norm(s, (hidden,), eps=1e-5) * w.float()
    got = on.bf16_to_f32(got_x)
    np.testing.assert_allclose(got, want.numpy(), rtol=2 * BF16_ULP_REL, atol=1e-6)


def test_rmsnorm_matches_hf_ministral3_rmsnorm():
    from transformers.models.ministral3.modeling_ministral3 import Ministral3RMSNorm
    g = torch.Generator().manual_seed(5)
    x, r = _randn_bf16(g, 16, 5120), _randn_bf16(g, 16, 5120)
    w = _randn_bf16(g, 5120, scale=0.1, shift=1.0)
    norm = Ministral3RMSNorm(5120, eps=1e-5)
    with torch.no_grad():
        norm.weight.copy_(w.float())
        want = norm(x.float() + r.float())        # fp32 input: HF computes in fp32 throughout
    got = on.bf16_to_f32(ops.fused_add_rmsnorm(bits(x), bits(r), bits(w), 1e-5)[0])
    np.testing.assert_allclose(got, want.numpy(), rtol=2 * BF16_ULP_REL, atol=1e-6)


def test_rmsnorm_closed_forms():
    hidden = 256
    w_one = from_bits(on.f32_to_bf16(np.ones(hidden, np.float32)))
    # constant row c (as s = c + 0): output c / sqrt(c^2 + eps) exactly up to bf16 rounding
    for c in (0.5, -3.0, 40.0):
        x = torch.full((1, hidden), c).bfloat16()
        r = torch.zeros(1, hidden).bfloat16()
        got = on.bf16_to_f32(ops.fused_add_rmsnorm(bits(x), bits(r), bits(w_one), 1e-5)[0])
        want = c / np.sqrt(c * c + 1e-5)
        np.testing.assert_allclose(got, want, rtol=BF16_ULP_REL)
    # zero row: 0 * rsqrt(eps) = 0
    z = torch.zeros(2, hidden).bfloat16()
    out, res = ops.fused_add_rmsnorm(bits(z), bits(z), bits(w_one), 1e-6)
    assert np.all(on.bf16_to_f32(out) == 0) and np.all(on.bf16_to_f32(res) == 0)
    # scale invariance: rmsnorm(a*s) == rmsnorm(s) for a power of two (exact in fp32 / bf16), eps -> 0
    g = torch.Generator().manual_seed(9)
    x = _randn_bf16(g, 4, hidden)
    zeros = torch.zeros(4, hidden).bfloat16()
    a = ops.fused_add_rmsnorm(bits(x), bits(zeros), bits(w_one), 0.0)[0]
    b = ops.fused_add_rmsnorm(bits((x.float() * 8).bfloat16()), bits(zeros), bits(w_one), 0.0)[0]
    assert np.array_equal(a, b)
    # weight enters linearly: doubling w doubles the output exactly
    w2 = from_bits(on.f32_to_bf16(np.full(hidden, 2.0, np.float32)))
    c = ops.fused_add_rmsnorm(bits(x), bits(zeros), bits(w2), 1e-5)[0]
    d = ops.fused_add_rmsnorm(bits(x), bits(zeros), bits(w_one), 1e-5)[0]
    assert np.array_equal(on.bf16_to_f32(c), 2 * on.bf16_to_f32(d))


def test_rmsnorm_quant_matches_reference_quantize():
    """out = (rmsnorm(s) * w / scale).clamp(-448, 448).to(fp8), the reference's quantize_fp8 applied to
    the fp32 norm output (devstral2.py:93-95)."""
    g = torch.Generator().manual_seed(11)
    x, r = _randn_bf16(g, 32, 5120, scale=3.0), _randn_bf16(g, 32, 5120)
    w = _randn_bf16(g, 5120, scale=0.1, shift=1.0)
    for scale in (0.005, 0.5, 1.0):
        codes, res = ops.fused_add_rmsnorm_quant(bits(x), bits(r), bits(w), scale, 1e-5)
        assert np.array_equal(res, bits(x + r))
        s = x.float() + r.float()
        y = F.rms_norm(s, (5120,), eps=1e-5) * w.float()
        want = (y / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        got_v, want_v = on.fp8_to_f32(codes), on.fp8_to_f32(want)
        # identical except where y itself differs by an fp32 ulp at an fp8 tie: at most 1 e4m3 ulp
        ulp = np.maximum(np.abs(want_v) * 2.0 ** -3, 2.0 ** -9)
        assert np.all(np.abs(got_v - want_v) <= ulp)
        assert np.mean(codes == want) > 0.999
        if scale == 0.005:
            assert np.any(np.abs(got_v) == 448.0)     # saturation exercised


# ---- SiluAndMul -----------------------------------------------------------------------------------

def test_silu_and_mul_matches_torch_silu():
    g = torch.Generator().manual_seed(3)
    x = _randn_bf16(g, 64, 2 * 1024, scale=4.0)
    got = on.bf16_to_f32(ops.silu_and_mul(bits(x)))
    gate, up = x[:, :1024].float(), x[:, 1024:].float()
    want = F.silu(gate) * up
    np.testing.assert_allclose(got, want.numpy(), rtol=2 * BF16_ULP_REL, atol=1e-30)


def test_silu_and_mul_gate_is_first_half():
    """Swapping the halves must change the result (gate first, up second: devstral2.py:364)."""
    g = torch.Generator().manual_seed(4)
    x = _randn_bf16(g, 4, 64)
    swapped = torch.cat([x[:, 32:], x[:, :32]], dim=1)
    assert not np.array_equal(ops.silu_and_mul(bits(x)), ops.silu_and_mul(bits(swapped)))
    up = torch.ones(4, 32).bfloat16()
    gate = x[:, :32]
    got = on.bf16_to_f32(ops.silu_and_mul(bits(torch.cat([gate, up], 1))))
    np.testing.assert_allclose(got, F.silu(gate.float()).numpy(), rtol=2 * BF16_ULP_REL, atol=1e-30)


def test_silu_and_mul_limits():
    gate = np.array([0.0, -0.0, 30.0, 80.0, -30.0, -100.0, -1e30, 1e30], np.float32)
    up = np.array([5.0, 5.0, 2.0, 0.5, 3.0, 3.0, 1.0, 1.0], np.float32)
    x = np.concatenate([on.f32_to_bf16(gate), on.f32_to_bf16(up)])[None, :]
    got = on.bf16_to_f32(ops.silu_and_mul(x))[0]
    assert got[0] == 0 and got[1] == 0                       # silu(0) = 0
    np.testing.assert_allclose(got[2:4], on.round_bf16(gate[2:4] * up[2:4]))   # g >> 0: g * u
    assert np.all(np.abs(got[4:7]) < 1e-10)                 # g << 0: 0 (exp overflow is benign)
    assert got[7] == on.round_bf16(np.array([1e30], np.float32))[0]


def test_silu_and_mul_quant_matches_reference_quantize():
    """The reference's down_proj quantize applied to the bf16 SiluAndMul output:
    (y / scale).clamp(-448, 448).to(float8_e4m3fn), y = (F.silu(g) * u).bfloat16()."""
    g = torch.Generator().manual_seed(15)
    x = _randn_bf16(g, 48, 2 * 512, scale=3.0)
    for scale in (0.004, 0.05, 1.0):
        got = ops.silu_and_mul_quant(bits(x), scale)
        y = (F.silu(x[:, :512].float()) * x[:, 512:].float()).bfloat16()
        want = (y.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        gv, wv = on.fp8_to_f32(got), on.fp8_to_f32(want)
        # y may differ by one bf16 ulp (exp rounding), which moves fp8 by at most one step
        assert np.all(np.abs(gv - wv) <= np.maximum(np.abs(wv) * 2.0 ** -3, 2.0 ** -9))
        assert np.mean(got == want) > 0.995
        if scale == 0.004:
            assert np.any(np.abs(gv) == 448.0)



def test_quantize_activation_matches_reference_quantize_exhaustively():
    """The o_proj / down_proj input quantize on every finite bf16 value: bit for bit
    (y.float() / scale).clamp(-448, 448).to(float8_e4m3fn), with saturation at both ends."""
    y = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    yt = torch.from_numpy(y.view(np.int16)).view(torch.bfloat16)
    finite = torch.isfinite(yt).numpy()
    for scale in (0.0037, 0.5, 3.0):
        got = ops.quantize_activation(y, scale)
        want = (yt.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        np.testing.assert_array_equal(got[finite], want[finite])
        assert np.all(on.fp8_to_f32(got[finite]) <= 448.0)

# ---- RoPE -----------------------------------------------------------------------------------------

def _hf_rope(q, k, positions, table):
    from transformers.models.ministral3.modeling_ministral3 import apply_rotary_pos_emb
    half = table.shape[1] // 2
    c = torch.from_numpy(table[positions, :half])
    s = torch.from_numpy(table[positions, half:])
    cos = torch.cat([c, c], dim=-1)[:, None, :]       # HF duplicates the angles: emb = cat(freqs, freqs)
    sin = torch.cat([s, s], dim=-1)[:, None, :]
    qe, ke = apply_rotary_pos_emb(q.float()[None].transpose(1, 2), k.float()[None].transpose(1, 2),
                                  cos.transpose(0, 1), sin.transpose(0, 1))
    return qe.transpose(1, 2)[0], ke.transpose(1, 2)[0]


def test_rope_neox_matches_hf_rotate_half():
    g = torch.Generator().manual_seed(6)
    n, hq, hk, d = 16, 4, 2, 128
    q, k = _randn_bf16(g, n, hq, d), _randn_bf16(g, n, hk, d)
    table = ops.cos_sin_table(32768, ops.rope_inv_freq(d, 1e6))
    pos = torch.randint(0, 32768, (n,), generator=g).numpy()
    got_q, got_k = ops.rope(bits(q), bits(k), pos, table, is_neox=True)
    want_q, want_k = _hf_rope(q, k, pos, table)
    np.testing.assert_allclose(on.bf16_to_f32(got_q), want_q.numpy(), rtol=2 * BF16_ULP_REL, atol=2e-2 * 2 ** -7)
    np.testing.assert_allclose(on.bf16_to_f32(got_k), want_k.numpy(), rtol=2 * BF16_ULP_REL, atol=2e-2 * 2 ** -7)


def test_rope_gptj_matches_complex_multiply():
    g = torch.Generator().manual_seed(7)
    n, h, d = 8, 3, 64
    x = _randn_bf16(g, n, h, d)
    table = ops.cos_sin_table(4096, ops.rope_inv_freq(d, 1e4))
    pos = torch.randint(0, 4096, (n,), generator=g).numpy()
    got, _ = ops.rope(bits(x), bits(x[:, :1]), pos, table, is_neox=False)
    xf = x.float().numpy().astype(np.float64)
    z = xf[..., 0::2] + 1j * xf[..., 1::2]
    rot = np.exp(1j * 0)  # noqa: F841  (angles come from the table, as in the kernels)
    e = table[pos, : d // 2].astype(np.float64) + 1j * table[pos, d // 2:].astype(np.float64)
    w = z * e[:, None, :]
    want = np.empty_like(xf)
    want[..., 0::2], want[..., 1::2] = w.real, w.imag
    np.testing.assert_allclose(on.bf16_to_f32(got), want, rtol=2 * BF16_ULP_REL, atol=1e-3)


def test_rope_invariants():
    g = torch.Generator().manual_seed(8)
    n, h, d = 12, 5, 128
    x = _randn_bf16(g, n, h, d)
    table = ops.cos_sin_table(8192, ops.rope_inv_freq(d, 1e6))
    # position 0 with plain RoPE: cos = 1, sin = 0 -> identity, bit for bit, both layouts
    for neox in (True, False):
        got, _ = ops.rope(bits(x), bits(x), np.zeros(n, np.int64), table, is_neox=neox)
        assert np.array_equal(got, bits(x))
    # rotation preserves each pair's norm (up to bf16 rounding)
    pos = torch.randint(0, 8192, (n,), generator=g).numpy()
    got, _ = ops.rope(bits(x), bits(x), pos, table, is_neox=True)
    xf, yf = bits_f = on.bf16_to_f32(bits(x)), on.bf16_to_f32(got)  # noqa: F841
    n_in = xf[..., :64] ** 2 + xf[..., 64:] ** 2
    n_out = yf[..., :64] ** 2 + yf[..., 64:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=4 * BF16_ULP_REL, atol=1e-4)
    # partial rotary: elements past the table width are untouched
    small = ops.cos_sin_table(64, ops.rope_inv_freq(32, 1e4))
    got, _ = ops.rope(bits(x), bits(x), np.arange(n) % 64, small, is_neox=True)
    assert np.array_equal(got[..., 32:], bits(x)[..., 32:])
    assert not np.array_equal(got[..., :32], bits(x)[..., :32])


def test_rope_table_matches_hf_default_and_yarn():
    from transformers import modeling_rope_utils as ru
    from transformers.models.ministral3.configuration_ministral3 import Ministral3Config
    from transformers.models.ministral3.modeling_ministral3 import Ministral3RotaryEmbedding

    cfg = Ministral3Config(head_dim=128, hidden_size=5120, num_attention_heads=32, max_position_embeddings=32768,
                           rope_parameters={"rope_type": "default", "rope_theta": 1e6})
    hf_inv, _ = Ministral3RotaryEmbedding.compute_default_rope_parameters(cfg)
    np.testing.assert_allclose(ops.rope_inv_freq(128, 1e6), hf_inv.numpy(), rtol=1e-6)

    for factor, orig, mscale, mscale_all in ((16.0, 16384, 1.0, 1.0), (4.0, 8192, 0.0, 0.0), (40.0, 4096, 0.707, 1.0)):
        params = {"rope_type": "yarn", "rope_theta": 1e6, "factor": factor, "original_max_position_embeddings": orig,
                  "beta_fast": 32.0, "beta_slow": 1.0, "mscale": mscale, "mscale_all_dim": mscale_all}
        cfg = Ministral3Config(head_dim=128, hidden_size=5120, num_attention_heads=32,
                               max_position_embeddings=orig * int(factor), rope_parameters=params)
        hf_inv, hf_scale = ru._compute_yarn_parameters(cfg)
        inv, scale = ops.yarn_inv_freq_and_scaling(128, 1e6, factor, orig, 32.0, 1.0, mscale, mscale_all, True)
        np.testing.assert_allclose(inv, hf_inv.numpy(), rtol=1e-6)
        assert scale == pytest.approx(hf_scale, rel=1e-12)
        # the whole table against transformers' rotary embedding (fp32 angles, cos/sin times the factor)
        rope = Ministral3RotaryEmbedding(cfg)
        positions = torch.arange(4096)[None]
        hf_cos, hf_sin = rope(torch.zeros(1, dtype=torch.float32), positions)
        # same fp32 inverse frequencies on both sides (an ulp in f grows to 4096 ulps of angle at p = 4096)
        table = ops.cos_sin_table(4096, hf_inv.numpy(), scale)
        np.testing.assert_allclose(table[:, :64], hf_cos[0, :, :64].numpy(), atol=3e-6)
        np.testing.assert_allclose(table[:, 64:], hf_sin[0, :, :64].numpy(), atol=3e-6)
        np.testing.assert_allclose(hf_cos[0, :, 64:].numpy(), hf_cos[0, :, :64].numpy())   # HF duplicates halves


def test_package_table_builders_match_oracle(mas):
    """The library's host-side table builders (they feed the RoPE kernel) against the oracle's:
    inverse frequencies within a few fp32 ulps, then the tables from identical frequencies."""
    inv = ops.rope_inv_freq(128, 1e6)
    np.testing.assert_allclose(mas.rope.rope_inv_freq(128, 1e6).numpy(), inv, rtol=1e-6)
    plain = mas.rope.cos_sin_cache(32768, 128, inv_freq=torch.from_numpy(inv)).numpy()
    np.testing.assert_allclose(plain, ops.cos_sin_table(32768, inv), atol=4e-6)

    args = (128, 1e8, 16.0, 16384, 32.0, 1.0, 1.0, 1.0, True)
    pkg_inv, pkg_scale = mas.rope.yarn_inv_freq(*args)
    inv, scale = ops.yarn_inv_freq_and_scaling(*args)
    np.testing.assert_allclose(pkg_inv.numpy(), inv, rtol=1e-6)
    assert pkg_scale == pytest.approx(scale, rel=1e-12)
    yarn = mas.rope.yarn_cos_sin_cache(4096, *args).numpy()
    np.testing.assert_allclose(yarn, ops.cos_sin_table(4096, pkg_inv.numpy(), scale), atol=4e-6)


# ---- KV store and embedding -------------------------------------------------------------------------

def _brute_force_append(k_cache, key, batch_indices, positions, kv_indices, kv_indptr):
    out = k_cache.copy()
    page_size = k_cache.shape[1]
    for t in range(len(positions)):
        b, p = int(batch_indices[t]), int(positions[t])
        page = int(kv_indices[int(kv_indptr[b]) + p // page_size])
        out[page, p % page_size] = key[t]
    return out


def test_paged_append_matches_brute_force_and_slot_form():
    rng = np.random.default_rng(12)
    pages, page_size, heads, dim, batch, width = 9, 4, 2, 8, 3, 3
    k_cache = rng.integers(0, 1 << 16, (pages, page_size, heads, dim), dtype=np.uint16)
    v_cache = rng.integers(0, 1 << 16, (pages, page_size, heads, dim), dtype=np.uint16)
    tables = rng.permutation(pages)[: batch * width].reshape(batch, width).astype(np.int32)
    indptr = (np.arange(batch + 1) * width).astype(np.int32)
    lens = [5, 12, 1]
    bidx = np.concatenate([np.full(n, b) for b, n in enumerate(lens)]).astype(np.int32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.int32)
    key = rng.integers(0, 1 << 16, (len(pos), heads, dim), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, (len(pos), heads, dim), dtype=np.uint16)
    k_out, v_out = ops.append_paged_kv_cache(k_cache, v_cache, key, val, bidx, pos, tables.flatten(), indptr)
    assert np.array_equal(k_out, _brute_force_append(k_cache, key, bidx, pos, tables.flatten(), indptr))
    assert np.array_equal(v_out, _brute_force_append(v_cache, val, bidx, pos, tables.flatten(), indptr))
    # untouched slots keep their contents
    touched = np.zeros((pages, page_size), bool)
    page, entry = ops.paged_destinations(bidx, pos, tables.flatten(), indptr, page_size)
    touched[page, entry] = True
    assert np.array_equal(k_out[~touched], k_cache[~touched])
    # slot form with slot = table[b, p // page_size] * page_size + p % page_size gives the same caches
    slots = tables[bidx, pos // page_size].astype(np.int64) * page_size + pos % page_size
    k2, v2 = ops.store_kv_slots(k_cache, v_cache, key, val, slots)
    assert np.array_equal(k2, k_out) and np.array_equal(v2, v_out)
    # negative slots are skipped
    slots[0] = -1
    k3, _ = ops.store_kv_slots(k_cache, v_cache, key, val, slots)
    assert np.array_equal(k3[page[0], entry[0]], k_cache[page[0], entry[0]])


def test_package_slot_helper_matches_oracle(mas):
    rng = np.random.default_rng(13)
    tables = torch.from_numpy(rng.permutation(64)[:24].reshape(4, 6).astype(np.int32))
    bidx = torch.tensor([0, 0, 1, 2, 3, 3], dtype=torch.int32)
    pos = torch.tensor([0, 17, 5, 40, 3, 95], dtype=torch.int32)
    got = mas.page.slot_mapping_from_block_tables(tables, bidx, pos, 16).numpy()
    page, entry = ops.paged_destinations(bidx.numpy(), pos.numpy(), tables.flatten().numpy(),
                                         (np.arange(5) * 6).astype(np.int32), 16)
    assert np.array_equal(got, page * 16 + entry)


def test_embedding_matches_torch():
    g = torch.Generator().manual_seed(14)
    table = _randn_bf16(g, 50, 24)
    ids = torch.tensor([0, 49, 7, 7, 0, 31])
    assert np.array_equal(ops.embedding(bits(table), ids.numpy()), bits(F.embedding(ids, table)))


@pytest.mark.parametrize("beta,interval", [(0.1, 8192), (0.5, 16), (1.0, 1)])
def test_llama_4_q_scale_matches_hf(beta, interval):
    """The oracle's llama-4 query scale (devstral2.py:175-179) against transformers' Ministral3
    get_llama_4_attn_scale (1 + beta * log(1 + floor(pos / M)), fp32) at every position of 48
    intervals, both rounded to bf16 as the reference does before the multiply; k = 0 gives 1."""
    from transformers.models.ministral3.modeling_ministral3 import get_llama_4_attn_scale

    rows = 48
    table = ops.llama_4_q_scale_table(beta, interval, rows)
    assert table[0] == 0x3F80
    step = max(interval // 64, 1)
    pos = torch.arange(0, rows * interval, step)
    hf = get_llama_4_attn_scale(pos[None], beta, interval)[0, 0, :, 0].to(torch.bfloat16)
    assert np.array_equal(table[pos.numpy() // interval], bits(hf))
    # the multiply: bf16(f32(q) * f32(scale)) is torch's bf16 product
    g = torch.Generator().manual_seed(interval)
    q = torch.randn(pos.shape[0], 4, 32, generator=g).bfloat16()
    want = q * from_bits(table[pos.numpy() // interval])[:, None, None]
    assert np.array_equal(ops.llama_4_scale_q(bits(q), pos.numpy(), table, interval), bits(want))


def test_fill_placeholders_closed_form():
    """model_runner.py:149-154: -1 - r is row r of the previous samples; other ids pass through."""
    last = np.array([10, 20, 30], dtype=np.int32)
    assert ops.fill_placeholders([5, -1, -3, 0, -2], last).tolist() == [5, 10, 30, 0, 20]
    assert ops.fill_placeholders(np.zeros(0, dtype=np.int64), last).shape == (0,)


def _attention_case(seed, batch, hq, hk, dim, page_size, lens, pages):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    width = max(1, max(-(-n // page_size) for n in lens))
    tables = torch.randperm(pages, generator=g)[: batch * width].reshape(batch, width).to(torch.int32)
    return q, kc, vc, tables, torch.tensor(lens, dtype=torch.int32)


@pytest.mark.parametrize("batch,hq,hk,dim,page_size,lens", [(3, 8, 2, 64, 16, [1, 37, 100]),
                                                             (2, 12, 1, 128, 8, [50, 9]),
                                                             (2, 4, 4, 32, 4, [13, 3])])
def test_paged_decode_attention_matches_sdpa(batch, hq, hk, dim, page_size, lens):
    """The oracle's decode attention against torch's scaled_dot_product_attention (fp32, grouped
    query heads) on the gathered rows of each sequence."""
    pages = batch * max(-(-n // page_size) for n in lens) + 3
    q, kc, vc, tables, seq = _attention_case(batch + dim, batch, hq, hk, dim, page_size, lens, pages)
    scale = dim ** -0.5
    got = on.bf16_to_f32(ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), scale))
    for b, n in enumerate(lens):
        pos = torch.arange(n)
        pg = tables[b, pos // page_size].long()
        k = kc[pg, pos % page_size].float().permute(1, 0, 2)[None]        # [1, Hk, L, D]
        v = vc[pg, pos % page_size].float().permute(1, 0, 2)[None]
        ref = F.scaled_dot_product_attention(q[b].float()[None, :, None, :], k, v, scale=scale, enable_gqa=True)
        want = on.bf16_to_f32(bits(ref[0, :, 0, :].bfloat16()))
        np.testing.assert_allclose(got[b], want, rtol=2 ** -7, atol=1e-3)


def test_paged_decode_attention_closed_forms():
    q, kc, vc, tables, _ = _attention_case(3, 2, 4, 2, 32, 4, [8, 8], 8)
    # one position: softmax is 1, the output is that value row exactly
    out = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), np.array([1, 1]), 0.3)
    for b in range(2):
        page = int(tables[b, 0])
        for h in range(4):
            assert np.array_equal(out[b, h], bits(vc)[page, 0, h // 2])
    # scale 0 (or identical keys): the plain mean of the value rows
    out = on.bf16_to_f32(ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), np.array([8, 5]), 0.0))
    for b, n in enumerate([8, 5]):
        pos = np.arange(n)
        v = vc[tables[b, pos // 4].long(), pos % 4].float().numpy()
        np.testing.assert_allclose(out[b], np.repeat(v.mean(axis=0), 2, axis=0), rtol=2 ** -7, atol=1e-6)
    # an empty row gives zeros; bmm2_scale multiplies the output
    out = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), np.array([0, 3]), 0.5, 2.0)
    half = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), np.array([0, 3]), 0.5, 1.0)
    assert not out[0].any()
    np.testing.assert_allclose(on.bf16_to_f32(out[1]), 2 * on.bf16_to_f32(half[1]), rtol=2 ** -7)


@pytest.mark.parametrize("q_lens,kv_lens,hq,hk,dim,page_size", [([5, 12], [5, 30], 8, 2, 32, 4),
                                                                 ([3, 1], [3, 9], 4, 4, 64, 8)])
def test_paged_context_attention_matches_sdpa(q_lens, kv_lens, hq, hk, dim, page_size):
    """The oracle's causal context attention against torch's scaled_dot_product_attention with an
    explicit mask aligned to the end of each row's positions (query token i at kv_len - q_len + i)."""
    g = torch.Generator().manual_seed(sum(kv_lens))
    tokens = sum(q_lens)
    width = max(-(-n // page_size) for n in kv_lens)
    pages = len(kv_lens) * width + 2
    q = torch.randn(tokens, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    tables = torch.randperm(pages, generator=g)[: len(kv_lens) * width].reshape(len(kv_lens), width).to(torch.int32)
    cu = np.concatenate([[0], np.cumsum(q_lens)])
    scale = dim ** -0.5
    got = on.bf16_to_f32(ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), np.array(kv_lens),
                                                     cu, scale))
    for j, (ql, kl) in enumerate(zip(q_lens, kv_lens)):
        pos = torch.arange(kl)
        pg = tables[j, pos // page_size].long()
        k = kc[pg, pos % page_size].float().permute(1, 0, 2)[None]
        v = vc[pg, pos % page_size].float().permute(1, 0, 2)[None]
        qq = q[cu[j]:cu[j + 1]].float().permute(1, 0, 2)[None]              # [1, Hq, q_len, D]
        mask = (torch.arange(kl)[None, :] <= (kl - ql + torch.arange(ql))[:, None])
        ref = F.scaled_dot_product_attention(qq, k, v, attn_mask=mask, scale=scale, enable_gqa=True)
        want = on.bf16_to_f32(bits(ref[0].permute(1, 0, 2).bfloat16()))
        np.testing.assert_allclose(got[cu[j]:cu[j + 1]], want, rtol=2 ** -7, atol=1e-3)
