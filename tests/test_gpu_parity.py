"""GPU parity: every HIP kernel against the oracle on identical seeded inputs, through the C ABI.

Bit-exact where the op is a copy or a single rounding (residual, KV store, embedding); bf16
outputs of the floating-point ops within rtol 1.6e-2 / atol 1e-2 (and, informatively, the
fraction of bit-identical elements); fp8 outputs within one e4m3 step.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL, bits, fp8_codes
from oracle import numerics as on
from oracle import ops

pytestmark = pytest.mark.gpu


def _randn_bf16(gen, *shape, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(*shape, generator=gen)).bfloat16()


def _close_bf16(got_bits, want_bits, min_exact=0.99):
    got, want = on.bf16_to_f32(got_bits), on.bf16_to_f32(want_bits)
    np.testing.assert_allclose(got, want, rtol=RTOL, atol=ATOL)
    if got.size:
        assert np.mean(got_bits == want_bits) >= min_exact


# ---- fused_add_rmsnorm ------------------------------------------------------------------------------

NORM_SHAPES = [(1, 8), (3, 100), (7, 5120), (64, 5120), (256, 5120), (33, 12288), (2, 4096), (5, 65544),
               (300, 1000),
               (9, 8192),   # 1024 lanes: sixteen wavefront sums, no slot left zero
               (4, 7680)]   # 960 lanes: fifteen


@pytest.mark.parametrize("rows,hidden", NORM_SHAPES)
def test_fused_add_rmsnorm_bf16(mas, dev, rows, hidden):
    g = torch.Generator().manual_seed(rows + hidden)
    x, r = _randn_bf16(g, rows, hidden), _randn_bf16(g, rows, hidden)
    w = _randn_bf16(g, hidden, scale=0.1, shift=1.0)
    want_x, want_r = ops.fused_add_rmsnorm(bits(x), bits(r), bits(w), 1e-5)
    xd, rd = x.to(dev), r.to(dev)
    mas.fused_add_rmsnorm(xd, rd, w.to(dev), 1e-5)
    assert np.array_equal(bits(rd), want_r)
    _close_bf16(bits(xd), want_x)


def test_fused_add_rmsnorm_strided_rows_and_3d(mas, dev):
    g = torch.Generator().manual_seed(21)
    base_x = _randn_bf16(g, 24, 5120 + 64)
    base_r = _randn_bf16(g, 24, 5120 + 128)
    w = _randn_bf16(g, 5120, scale=0.1, shift=1.0)
    x, r = base_x[:, :5120], base_r[:, 64:5184]
    want_x, want_r = ops.fused_add_rmsnorm(bits(x), bits(r), bits(w), 1e-6)
    bxd, brd = base_x.to(dev), base_r.to(dev)
    mas.fused_add_rmsnorm(bxd[:, :5120], brd[:, 64:5184], w.to(dev), 1e-6)
    assert np.array_equal(bits(brd[:, 64:5184]), want_r)
    _close_bf16(bits(bxd[:, :5120]), want_x)
    # untouched columns stay untouched
    assert np.array_equal(bits(bxd[:, 5120:]), bits(base_x[:, 5120:]))
    assert np.array_equal(bits(brd[:, :64]), bits(base_r[:, :64]))
    # a 3-D [batch, seq, hidden] input
    x3, r3 = _randn_bf16(g, 2, 5, 256), _randn_bf16(g, 2, 5, 256)
    w3 = _randn_bf16(g, 256, scale=0.1, shift=1.0)
    want_x, want_r = ops.fused_add_rmsnorm(bits(x3), bits(r3), bits(w3), 1e-5)
    x3d, r3d = x3.to(dev), r3.to(dev)
    mas.fused_add_rmsnorm(x3d, r3d, w3.to(dev), 1e-5)
    assert np.array_equal(bits(r3d), want_r)
    _close_bf16(bits(x3d), want_x)


@pytest.mark.parametrize("rows,hidden", [(1, 8), (3, 100), (64, 5120), (128, 12288), (17, 4104), (5, 8192)])
@pytest.mark.parametrize("scale_kind", ["tensor", "float"])
def test_fused_add_rmsnorm_quant_fp8(mas, dev, rows, hidden, scale_kind):
    g = torch.Generator().manual_seed(rows * 3 + hidden)
    x, r = _randn_bf16(g, rows, hidden, scale=2.0), _randn_bf16(g, rows, hidden)
    w = _randn_bf16(g, hidden, scale=0.1, shift=1.0)
    scale = 0.0071
    want_q, want_r = ops.fused_add_rmsnorm_quant(bits(x), bits(r), bits(w), scale, 1e-5)
    xd, rd = x.to(dev), r.to(dev)
    out = torch.empty(rows, hidden, dtype=torch.float8_e4m3fn, device=dev)
    s = torch.tensor(scale, dtype=torch.float32, device=dev) if scale_kind == "tensor" else scale
    mas.fused_add_rmsnorm_quant(out, xd, rd, w.to(dev), s, 1e-5)
    assert np.array_equal(bits(rd), want_r)
    assert np.array_equal(bits(xd), bits(x)), "input must not be written"
    got_q = fp8_codes(out)
    gv, wv = on.fp8_to_f32(got_q), on.fp8_to_f32(want_q)
    assert np.all(np.abs(gv - wv) <= np.maximum(np.abs(wv) * 2.0 ** -3, 2.0 ** -9))
    assert np.mean(got_q == want_q) >= 0.995
    if rows * hidden >= 4096:
        assert np.any(np.abs(gv) == 448.0)   # saturation reached at this scale


def test_fused_add_rmsnorm_quant_nan_and_zero_rows(mas, dev):
    x = torch.zeros(3, 64, dtype=torch.bfloat16)
    x[1, 5] = float("nan")
    r = torch.zeros(3, 64, dtype=torch.bfloat16)
    r[2] = 1.0
    w = torch.ones(64, dtype=torch.bfloat16)
    out = torch.empty(3, 64, dtype=torch.float8_e4m3fn, device=dev)
    rd = r.to(dev)
    mas.fused_add_rmsnorm_quant(out, x.to(dev), rd, w.to(dev), 1.0, 1e-6)
    q = on.fp8_to_f32(fp8_codes(out))
    assert np.all(q[0] == 0)                     # zero row -> 0
    assert np.all(np.isnan(q[1]))                # a NaN poisons its row's norm
    np.testing.assert_allclose(q[2], 1.0 / np.sqrt(1.0 + 1e-6), rtol=2 ** -3)


# ---- silu_and_mul -----------------------------------------------------------------------------------

@pytest.mark.parametrize("rows,inter", [(1, 8), (3, 100), (2, 1000), (64, 32768), (129, 2048), (1000, 64)])
def test_silu_and_mul(mas, dev, rows, inter):
    g = torch.Generator().manual_seed(rows * 7 + inter)
    x = _randn_bf16(g, rows, 2 * inter, scale=3.0)
    out = mas.silu_and_mul(x.to(dev))
    _close_bf16(bits(out), ops.silu_and_mul(bits(x)), min_exact=0.98)


def test_silu_and_mul_strided_input_and_out(mas, dev):
    g = torch.Generator().manual_seed(31)
    base = _randn_bf16(g, 40, 2 * 512 + 64)
    x = base[:, 32:32 + 1024]
    out_base = torch.full((40, 600), 7.0, dtype=torch.bfloat16, device=dev)
    out = out_base[:, 8:520]
    mas.silu_and_mul(base.to(dev)[:, 32:32 + 1024], out=out)
    _close_bf16(bits(out), ops.silu_and_mul(bits(x)), min_exact=0.98)
    assert torch.all(out_base[:, :8] == 7.0) and torch.all(out_base[:, 520:] == 7.0)
    # leading batch dimensions
    x3 = _randn_bf16(g, 2, 3, 256)
    out3 = mas.silu_and_mul(x3.to(dev))
    assert out3.shape == (2, 3, 128)
    _close_bf16(bits(out3), ops.silu_and_mul(bits(x3)), min_exact=0.98)


@pytest.mark.parametrize("rows,inter", [(1, 8), (3, 100), (64, 32768), (129, 2048), (7, 1000)])
@pytest.mark.parametrize("scale_kind", ["tensor", "float"])
def test_silu_and_mul_quant(mas, dev, rows, inter, scale_kind):
    g = torch.Generator().manual_seed(rows * 11 + inter)
    x = _randn_bf16(g, rows, 2 * inter, scale=3.0)
    scale = 0.004
    s = torch.tensor(scale, dtype=torch.float32, device=dev) if scale_kind == "tensor" else scale
    out = mas.silu_and_mul_quant(x.to(dev), s)
    got = fp8_codes(out)
    want = ops.silu_and_mul_quant(bits(x), scale)
    gv, wv = on.fp8_to_f32(got), on.fp8_to_f32(want)
    assert np.all(np.abs(gv - wv) <= np.maximum(np.abs(wv) * 2.0 ** -3, 2.0 ** -9))
    assert np.mean(got == want) >= 0.99
    # the fused op equals silu_and_mul followed by the reference's quantize of its bf16 output
    y = mas.silu_and_mul(x.to(dev))
    ref = (y.float() / scale).clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(out.view(torch.uint8), ref.view(torch.uint8))


@pytest.mark.parametrize("scale_kind", ["tensor", "float"])
def test_silu_and_mul_quant_every_bf16_value(mas, dev, scale_kind):
    """The fp8 epilogue on every bf16 input. With gate = 32, e^-32 vanishes next to 1 in fp32, so
    silu(32) = 32 exactly, y = 32 * u is exact in bf16 (or overflows to inf, which saturates just
    as u does) and y / 32 = u. So the output must be the saturating e4m3fn encode of u for all 2^16
    patterns: both zeros, subnormals, every rounding midpoint, values past 448 and infinities. A NaN
    u must give a NaN code; its sign is not checked, since the sign of a NaN produced by
    arithmetic (32 * u, then rounding to bf16) is unspecified."""
    u_bits = np.arange(65536, dtype=np.uint16).reshape(64, 1024)
    x_bits = np.concatenate([np.full_like(u_bits, 0x4200), u_bits], axis=1)   # 0x4200 = bf16 32.0
    x = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16)
    s = torch.tensor(32.0, dtype=torch.float32, device=dev) if scale_kind == "tensor" else 32.0
    got = fp8_codes(mas.silu_and_mul_quant(x.to(dev), s))
    want = on.f32_to_fp8_saturate(on.bf16_to_f32(u_bits))
    nan = np.isnan(on.bf16_to_f32(u_bits))
    with np.errstate(over="ignore", invalid="ignore"):
        oracle = ops.silu_and_mul_quant(x_bits, 32.0)
    assert np.array_equal(oracle[~nan], want[~nan]) and np.all(oracle[nan] & 0x7F == 0x7F)
    assert np.all(got[nan] & 0x7F == 0x7F)
    bad = np.flatnonzero((got != want) & ~nan)
    assert bad.size == 0, [(hex(int(u_bits.flat[i])), hex(int(got.flat[i])), hex(int(want.flat[i]))) for i in bad[:8]]


# ---- rope -----------------------------------------------------------------------------------------

def _rope_case(mas, dev, n, hq, hk, head_dim, rotary_dim, neox, pos_dtype, seed, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    qkv = _randn_bf16(g, n, (hq + 2 * hk) * head_dim)
    table = mas.rope.cos_sin_cache(max_pos, rotary_dim, 1e6)
    pos = torch.randint(0, max_pos, (n,), generator=g).to(pos_dtype)
    q = qkv[:, : hq * head_dim].reshape(n, hq, head_dim)
    k = qkv[:, hq * head_dim: (hq + hk) * head_dim].reshape(n, hk, head_dim)
    want_q, want_k = ops.rope(bits(q), bits(k), pos.numpy(), table.numpy(), is_neox=neox)
    qkv_d = qkv.to(dev)
    qd, kd, _ = qkv_d.split([hq * head_dim, hk * head_dim, hk * head_dim], dim=-1)
    mas.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), qd, kd, head_dim, table.to(dev), neox)
    # with the kernels' fp32 order (products rounded, then one add) the result is bit-identical
    assert np.array_equal(bits(qd).reshape(n, hq, head_dim), want_q)
    assert np.array_equal(bits(kd).reshape(n, hk, head_dim), want_k)
    assert np.array_equal(bits(qkv_d[:, (hq + hk) * head_dim:]), bits(qkv[:, (hq + hk) * head_dim:])), "v changed"


@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("n,hq,hk", [(1, 1, 1), (5, 32, 8), (64, 32, 8), (300, 32, 8), (3, 96, 8), (40, 0, 8)])
def test_rope_head_128(mas, dev, neox, n, hq, hk):
    _rope_case(mas, dev, n, hq, hk, 128, 128, neox, torch.int32, n * 10 + hq)


@pytest.mark.parametrize("head_dim,rotary_dim", [(64, 64), (256, 256), (128, 64), (256, 128), (512, 512), (96, 32)])
def test_rope_other_dims(mas, dev, head_dim, rotary_dim):
    _rope_case(mas, dev, 17, 6, 2, head_dim, rotary_dim, True, torch.int64, head_dim + rotary_dim)


def test_rope_3d_views_and_position_errors(mas, dev):
    g = torch.Generator().manual_seed(41)
    n, hq, hk, d = 9, 4, 2, 128
    q = _randn_bf16(g, n, hq, d)
    k = _randn_bf16(g, n, hk, d)
    table = mas.rope.cos_sin_cache(100, d, 1e4)
    pos = torch.tensor([0, 5, 99, 100, -1, 50, 7, 1000, 3], dtype=torch.int32)
    qd, kd = q.to(dev), k.to(dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.rope.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), qd, kd, d, table.to(dev), True, error_flags=flags)
    assert int(flags.item()) == 2
    ok = np.array([p >= 0 and p < 100 for p in pos.tolist()])
    want_q, want_k = ops.rope(bits(q)[ok], bits(k)[ok], pos.numpy()[ok], table.numpy())
    assert np.array_equal(bits(qd)[ok], want_q) and np.array_equal(bits(kd)[ok], want_k)
    assert np.array_equal(bits(qd)[~ok], bits(q)[~ok]) and np.array_equal(bits(kd)[~ok], bits(k)[~ok])
    # position 0 of a plain table is the identity
    assert np.array_equal(bits(qd)[0], bits(q)[0])


def test_rope_yarn_table(mas, dev):
    g = torch.Generator().manual_seed(43)
    n, hq, hk, d = 32, 32, 8, 128
    table = mas.rope.yarn_cos_sin_cache(32768, d, 1e8, 16.0, 16384, 32.0, 1.0, 1.0, 1.0, True)
    qkv = _randn_bf16(g, n, (hq + 2 * hk) * d)
    pos = torch.randint(0, 32768, (n,), generator=g, dtype=torch.int32)
    want_q, want_k = ops.rope(bits(qkv[:, :hq * d]).reshape(n, hq, d), bits(qkv[:, hq * d:(hq + hk) * d]).reshape(
        n, hk, d), pos.numpy(), table.numpy())
    qd = qkv.to(dev)
    q, k, _ = qd.split([hq * d, hk * d, hk * d], -1)
    mas.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), q, k, d, table.to(dev))
    assert np.array_equal(bits(q).reshape(n, hq, d), want_q)
    assert np.array_equal(bits(k).reshape(n, hk, d), want_k)


# ---- paged KV store -----------------------------------------------------------------------------------

def _kv_case(gen, pages, page_size, heads, dim, lens, width):
    batch = len(lens)
    tables = torch.randperm(pages, generator=gen)[: batch * width].reshape(batch, width).to(torch.int32)
    indptr = (torch.arange(batch + 1) * width).to(torch.int32)
    bidx = torch.cat([torch.full((n,), b) for b, n in enumerate(lens)]).to(torch.int32)
    pos = torch.cat([torch.arange(n) for n in lens]).to(torch.int32)
    return tables, indptr, bidx, pos


@pytest.mark.parametrize("page_size,heads,dim,lens", [(16, 8, 128, [5, 40, 1, 16]), (256, 8, 128, [300, 2]),
                                                      (4, 2, 64, [9]), (8, 1, 8, [3, 3])])
def test_append_paged_kv_cache(mas, dev, page_size, heads, dim, lens):
    g = torch.Generator().manual_seed(page_size + heads + dim)
    width = -(-max(lens) // page_size)
    pages = len(lens) * width + 3
    tables, indptr, bidx, pos = _kv_case(g, pages, page_size, heads, dim, lens, width)
    n = len(pos)
    hq = 2
    qkv = _randn_bf16(g, n, (hq + 2 * heads) * dim)
    key = qkv[:, hq * dim:(hq + heads) * dim].reshape(n, heads, dim)
    val = qkv[:, (hq + heads) * dim:].reshape(n, heads, dim)
    k0 = torch.randn(pages, page_size, heads, dim, generator=g).bfloat16()
    v0 = torch.randn(pages, page_size, heads, dim, generator=g).bfloat16()
    want_k, want_v = ops.append_paged_kv_cache(bits(k0), bits(v0), bits(key), bits(val), bidx.numpy(), pos.numpy(),
                                               tables.flatten().numpy(), indptr.numpy())
    qkv_d = qkv.to(dev)
    kd = qkv_d[:, hq * dim:(hq + heads) * dim].view(n, heads, dim)
    vd = qkv_d[:, (hq + heads) * dim:].view(n, heads, dim)
    kc, vc = k0.to(dev), v0.to(dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.append_paged_kv_cache(kd, vd, bidx.to(dev), pos.to(dev), (kc, vc), tables.flatten().to(dev), indptr.to(dev),
                              None, "NHD", error_flags=flags)
    assert int(flags.item()) == 0
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)
    # slot-mapping form reaches the same caches
    slots = mas.page.slot_mapping_from_block_tables(tables, bidx, pos, page_size)
    kc2, vc2 = k0.to(dev), v0.to(dev)
    mas.store_kv_slots(kd, vd, kc2, vc2, slots.to(dev))
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc)


def test_kv_layouts_and_single_tensor_cache(mas, dev):
    g = torch.Generator().manual_seed(51)
    pages, ps, heads, dim = 6, 8, 4, 64
    lens = [10, 7]
    tables, indptr, bidx, pos = _kv_case(g, pages, ps, heads, dim, lens, 2)
    n = len(pos)
    key, val = _randn_bf16(g, n, heads, dim), _randn_bf16(g, n, heads, dim)
    want_k, want_v = ops.append_paged_kv_cache(np.zeros((pages, ps, heads, dim), np.uint16),
                                               np.zeros((pages, ps, heads, dim), np.uint16), bits(key), bits(val),
                                               bidx.numpy(), pos.numpy(), tables.flatten().numpy(), indptr.numpy())
    args = (bidx.to(dev), pos.to(dev))
    # HND: [pages, heads, page_size, dim]
    kh = torch.zeros(pages, heads, ps, dim, dtype=torch.bfloat16, device=dev)
    vh = torch.zeros_like(kh)
    mas.append_paged_kv_cache(key.to(dev), val.to(dev), *args, (kh, vh), tables.flatten().to(dev), indptr.to(dev),
                              None, "HND")
    assert np.array_equal(bits(kh.transpose(1, 2)), want_k) and np.array_equal(bits(vh.transpose(1, 2)), want_v)
    # one [pages, 2, page_size, heads, dim] tensor, NHD; 2-D [nnz, heads * dim] sources
    kv = torch.zeros(pages, 2, ps, heads, dim, dtype=torch.bfloat16, device=dev)
    mas.append_paged_kv_cache(key.to(dev).reshape(n, -1), val.to(dev).reshape(n, -1), *args, kv,
                              tables.flatten().to(dev), indptr.to(dev))
    assert np.array_equal(bits(kv[:, 0]), want_k) and np.array_equal(bits(kv[:, 1]), want_v)


def test_kv_duplicates_and_index_errors(mas, dev):
    g = torch.Generator().manual_seed(61)
    pages, ps, heads, dim = 5, 4, 2, 16
    # padding-style duplicates: several tokens aimed at page 4 (the sink), entry 0
    tables = torch.tensor([[0, 1], [4, 4], [4, 4], [2, 3]], dtype=torch.int32)
    indptr = torch.tensor([0, 2, 4, 6, 8], dtype=torch.int32)
    bidx = torch.tensor([0, 1, 2, 3, 0, 3, 5, 0, 1], dtype=torch.int32)
    pos = torch.tensor([0, 0, 0, 5, 7, -1, 0, 8, 0], dtype=torch.int32)
    # token 5: negative position; token 6: batch 5 >= 4; token 7: page slot 2 past this sequence's 2
    n = len(pos)
    key, val = _randn_bf16(g, n, heads, dim), _randn_bf16(g, n, heads, dim)
    kc = torch.zeros(pages, ps, heads, dim, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.append_paged_kv_cache(key.to(dev), val.to(dev), bidx.to(dev), pos.to(dev), (kc, vc),
                              tables.flatten().to(dev), indptr.to(dev), None, "NHD", error_flags=flags)
    assert int(flags.item()) == 2 | 4 | 8
    kb = bits(kc)
    assert np.array_equal(kb[0, 0], bits(key)[0]) and np.array_equal(kb[3, 1], bits(key)[3])
    assert np.array_equal(kb[1, 3], bits(key)[4])
    sink = kb[4, 0]
    assert any(np.array_equal(sink, bits(key)[t]) for t in (1, 2, 8)), "sink holds one of its writers"
    written = {(0, 0), (3, 1), (1, 3), (4, 0)}
    for p in range(pages):
        for e in range(ps):
            if (p, e) not in written:
                assert not kb[p, e].any()
    # slot form: negative slots skipped, slots past the cache flagged
    slots = torch.tensor([3, -1, 19, 20, 1000], dtype=torch.int64)
    kc.zero_()
    vc.zero_()
    flags.zero_()
    mas.store_kv_slots(key[:5].to(dev), val[:5].to(dev), kc, vc, slots.to(dev), error_flags=flags)
    assert int(flags.item()) == 16
    kb = bits(kc)
    assert np.array_equal(kb[0, 3], bits(key)[0]) and np.array_equal(kb[4, 3], bits(key)[2])
    assert int((kc != 0).sum()) == 2 * heads * dim - int((bits(key)[[0, 2]] == 0).sum())



def test_kv_store_prefill_sized_skips_and_flags_bad_tokens(mas, dev):
    """A prefill-sized step with bad tokens scattered through it: each bad token is skipped and
    flagged, and every other row lands where the oracle puts it (block-table and slot forms)."""
    g = torch.Generator().manual_seed(71)
    ps, heads, dim, lens = 64, 8, 128, [1500, 700, 3]
    width = -(-max(lens) // ps)
    pages = len(lens) * width + 5
    tables, indptr, bidx, pos = _kv_case(g, pages, ps, heads, dim, lens, width)
    n = len(pos)
    key, val = _randn_bf16(g, n, heads, dim), _randn_bf16(g, n, heads, dim)
    k0 = torch.randn(pages, ps, heads, dim, generator=g).bfloat16()
    v0 = torch.randn(pages, ps, heads, dim, generator=g).bfloat16()
    keep = np.ones(n, dtype=bool)
    bad_pos, bad_b, bad_idx = pos.clone(), bidx.clone(), tables.clone()
    bad_pos[10] = -3                                   # negative position: bit 4
    bad_b[700] = 3                                     # batch 3 of 3: bit 2
    bad_pos[n - 1] = ps * width + 5                    # past its row's pages: bit 8
    bad_idx[1, 2] = pages + 7                          # a page past the cache for 64 tokens of row 1: bit 8
    keep[[10, 700, n - 1]] = False
    keep[1500 + 2 * ps:1500 + 3 * ps] = False
    want_k, want_v = ops.append_paged_kv_cache(bits(k0), bits(v0), bits(key)[keep], bits(val)[keep],
                                               bidx.numpy()[keep], pos.numpy()[keep], tables.flatten().numpy(),
                                               indptr.numpy())
    kc, vc = k0.to(dev), v0.to(dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.append_paged_kv_cache(key.to(dev), val.to(dev), bad_b.to(dev), bad_pos.to(dev), (kc, vc),
                              bad_idx.flatten().to(dev), indptr.to(dev), None, "NHD", error_flags=flags)
    assert int(flags.item()) == 2 | 4 | 8
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)
    # slot form: negative slots skipped silently, slots past the cache flagged
    slots = mas.page.slot_mapping_from_block_tables(tables, bidx, pos, ps)
    slots[[5, 2100]] = -1
    slots[[6, 2199]] = pages * ps + 1
    skeep = (slots >= 0) & (slots < pages * ps)
    want_k, want_v = ops.store_kv_slots(bits(k0), bits(v0), bits(key), bits(val),
                                        np.where(skeep.numpy(), slots.numpy(), -1))
    kc, vc = k0.to(dev), v0.to(dev)
    flags.zero_()
    mas.store_kv_slots(key.to(dev), val.to(dev), kc, vc, slots.to(dev), error_flags=flags)
    assert int(flags.item()) == 16
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)

# ---- embedding ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("rows,vocab,hidden", [(1, 10, 8), (7, 100, 5120), (256, 4096, 5120), (5, 30, 100),
                                               (64, 1000, 12288)])
def test_embedding(mas, dev, rows, vocab, hidden):
    g = torch.Generator().manual_seed(rows + vocab)
    table = _randn_bf16(g, vocab, hidden)
    ids = torch.randint(0, vocab, (rows,), generator=g)
    ids[0] = vocab - 1
    out = mas.embedding.embedding(ids.to(dev), table.to(dev))
    assert np.array_equal(bits(out), ops.embedding(bits(table), ids.numpy()))


def test_embedding_out_of_range_ids_and_module(mas, dev):
    g = torch.Generator().manual_seed(71)
    table = _randn_bf16(g, 50, 256)
    ids = torch.tensor([3, 50, -2, 49, 0])
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = mas.embedding.embedding(ids.to(dev), table.to(dev), error_flags=flags)
    assert int(flags.item()) == 1
    ob = bits(out)
    assert np.array_equal(ob[[0, 3, 4]], bits(table)[[3, 49, 0]])
    assert not ob[[1, 2]].any()
    emb = mas.Embedding(50, 256, device=dev)
    with torch.no_grad():
        emb.weight.copy_(table.to(dev))
    ids2 = torch.tensor([[1, 2], [3, 4]], device=dev)
    assert torch.equal(emb(ids2), table.to(dev)[ids2])


@pytest.mark.parametrize("rows,vocab,hidden", [(64, 131072, 5120), (256, 4096, 5120), (9, 50, 100)])
def test_embedding_with_placeholders(mas, dev, rows, vocab, hidden):
    """The step-input path (model_runner.py:149-154 then devstral2.py:282) in one launch: the ids
    after the call equal fill_placeholders' result and the rows those ids select."""
    g = torch.Generator().manual_seed(rows + hidden)
    table = _randn_bf16(g, vocab, hidden)
    last = torch.randint(0, vocab, (rows + 3,), generator=g).to(torch.int32)
    ids = torch.randint(0, vocab, (rows,), generator=g)
    holders = torch.rand(rows, generator=g) < 0.5
    ids[holders] = -1 - torch.randint(0, rows + 3, (int(holders.sum()),), generator=g)
    ids[0] = -1                                              # row 0 of the samples
    want_ids = ops.fill_placeholders(ids.numpy(), last.numpy())
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    ids_d = ids.to(dev)
    out = mas.embedding.embedding(ids_d, table.to(dev), last_tokens=last.to(dev), error_flags=flags)
    assert np.array_equal(ids_d.cpu().numpy(), want_ids)
    assert np.array_equal(bits(out), ops.embedding(bits(table), want_ids))
    assert int(flags.item()) == 0
    # fill_placeholders alone
    ids_d = ids.to(dev)
    mas.embedding.fill_placeholders(ids_d, last.to(dev))
    assert np.array_equal(ids_d.cpu().numpy(), want_ids)


def test_embedding_placeholder_errors(mas, dev):
    g = torch.Generator().manual_seed(5)
    table = _randn_bf16(g, 50, 256)
    last = torch.tensor([7, 60, 2], dtype=torch.int32)       # 60 is past the vocab
    ids = torch.tensor([-1, -4, -2, 3, -3])                   # -4: row 3 is past the samples
    for hidden in (256, 100):                                 # vector and scalar kernels
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        ids_d = ids.to(dev)
        tab = table[:, :hidden].contiguous()
        out = mas.embedding.embedding(ids_d, tab.to(dev), last_tokens=last.to(dev), error_flags=flags)
        assert ids_d.tolist() == [7, -4, 60, 3, 2]
        assert int(flags.item()) == 1 | 32
        ob = bits(out)
        assert np.array_equal(ob[[0, 3, 4]], bits(tab)[[7, 3, 2]])
        assert not ob[[1, 2]].any()
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    ids_d = ids.to(dev)
    mas.embedding.fill_placeholders(ids_d, last.to(dev), error_flags=flags)
    assert ids_d.tolist() == [7, -4, 60, 3, 2] and int(flags.item()) == 32


# ---- empty inputs -------------------------------------------------------------------------------------

def test_empty_inputs_are_no_ops(mas, dev):
    e = torch.empty(0, 5120, dtype=torch.bfloat16, device=dev)
    mas.fused_add_rmsnorm(e, e.clone(), torch.ones(5120, dtype=torch.bfloat16, device=dev))
    mas.fused_add_rmsnorm_quant(torch.empty(0, 5120, dtype=torch.float8_e4m3fn, device=dev), e, e.clone(),
                                torch.ones(5120, dtype=torch.bfloat16, device=dev), 1.0)
    assert mas.silu_and_mul(torch.empty(0, 64, dtype=torch.bfloat16, device=dev)).shape == (0, 32)
    table = mas.rope.cos_sin_cache(16, 128).to(dev)
    mas.apply_rope_with_cos_sin_cache_inplace(torch.empty(0, dtype=torch.int32, device=dev),
                                              torch.empty(0, 4 * 128, dtype=torch.bfloat16, device=dev),
                                              torch.empty(0, 128, dtype=torch.bfloat16, device=dev), 128, table)
    kc = torch.zeros(2, 4, 1, 128, dtype=torch.bfloat16, device=dev)
    z32 = torch.empty(0, dtype=torch.int32, device=dev)
    mas.append_paged_kv_cache(torch.empty(0, 1, 128, dtype=torch.bfloat16, device=dev),
                              torch.empty(0, 1, 128, dtype=torch.bfloat16, device=dev), z32, z32, (kc, kc.clone()),
                              torch.zeros(1, dtype=torch.int32, device=dev),
                              torch.zeros(2, dtype=torch.int32, device=dev))
    out = mas.embedding.embedding(torch.empty(0, dtype=torch.int64, device=dev),
                                  torch.zeros(4, 64, dtype=torch.bfloat16, device=dev))
    assert out.shape == (0, 64)
    torch.cuda.synchronize()


# ---- committed golden fixtures ------------------------------------------------------------------------

def test_kernels_reproduce_golden_fixtures(mas, dev):
    from conftest import GOLDEN_DIR, from_bits
    gd = np.load(GOLDEN_DIR / "layer_ops.npz")

    def dev_bf16(key):
        return from_bits(gd[key]).to(dev)

    x, r = dev_bf16("norm_x"), dev_bf16("norm_r")
    mas.fused_add_rmsnorm(x, r, dev_bf16("norm_w"), float(gd["norm_eps"]))
    assert np.array_equal(bits(r), gd["norm_res"])
    _close_bf16(bits(x), gd["norm_out"], min_exact=0.98)

    x, r = dev_bf16("norm_x"), dev_bf16("norm_r")
    out = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=dev)
    mas.fused_add_rmsnorm_quant(out, x, r, dev_bf16("norm_w"), float(gd["quant_scale"]), float(gd["norm_eps"]))
    assert np.array_equal(bits(r), gd["quant_res"])
    gv, wv = on.fp8_to_f32(fp8_codes(out)), on.fp8_to_f32(gd["quant_out"])
    assert np.all(np.abs(gv - wv) <= np.maximum(np.abs(wv) * 2.0 ** -3, 2.0 ** -9))

    _close_bf16(bits(mas.silu_and_mul(dev_bf16("silu_in"))), gd["silu_out"], min_exact=0.95)

    table = torch.from_numpy(gd["rope_table"]).to(dev)
    pos = torch.from_numpy(gd["rope_pos"]).to(dev)
    for layout, neox in (("neox", True), ("gptj", False)):
        q, k = dev_bf16("rope_q"), dev_bf16("rope_k")
        mas.apply_rope_with_cos_sin_cache_inplace(pos, q, k, 128, table, neox)
        assert np.array_equal(bits(q), gd[f"rope_{layout}_q"]) and np.array_equal(bits(k), gd[f"rope_{layout}_k"])

    kc, vc = dev_bf16("kv_kc0"), dev_bf16("kv_vc0")
    i32 = {key: torch.from_numpy(gd[key]).to(dev) for key in ("kv_tables", "kv_indptr", "kv_bidx", "kv_pos")}
    mas.append_paged_kv_cache(dev_bf16("kv_k"), dev_bf16("kv_v"), i32["kv_bidx"], i32["kv_pos"], (kc, vc),
                              i32["kv_tables"].flatten(), i32["kv_indptr"])
    assert np.array_equal(bits(kc), gd["kv_kc"]) and np.array_equal(bits(vc), gd["kv_vc"])

    out = mas.embedding.embedding(torch.from_numpy(gd["emb_ids"]).to(dev), dev_bf16("emb_table"))
    assert np.array_equal(bits(out), gd["emb_out"])


# ---- fused RoPE + paged KV append ------------------------------------------------------------------

@pytest.mark.parametrize("neox", [True, False])
@pytest.mark.parametrize("n,hq,hk,d,page_size", [(1, 32, 8, 128, 256), (64, 32, 8, 128, 256), (300, 32, 8, 128, 16),
                                                  (37, 96, 8, 128, 256), (9, 4, 2, 64, 4), (5, 2, 1, 256, 8),
                                                  (3, 0, 2, 128, 16)])
def test_rope_append_fused_matches_separate_calls(mas, dev, neox, n, hq, hk, d, page_size):
    g = torch.Generator().manual_seed(n * 31 + hq + d)
    lens = [n // 2, n - n // 2] if n > 1 else [1]
    lens = [x for x in lens if x > 0]
    width = -(-max(lens) // page_size) + 1
    pages = len(lens) * width + 2
    tables, indptr, bidx, pos = _kv_case(g, pages, page_size, hk, d, lens, width)
    pos = pos + 3                                          # not starting at 0
    table = mas.rope.cos_sin_cache(max(pos.tolist()) + 5, d, 1e6)
    qkv = _randn_bf16(g, n, (hq + 2 * hk) * d)
    k0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    v0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    args = (pos.to(dev), bidx.to(dev), tables.flatten().to(dev), indptr.to(dev), table.to(dev))

    def run(fused: bool):
        buf = qkv.to(dev)
        q, k, v = buf.split([hq * d, hk * d, hk * d], dim=-1)
        kc, vc = k0.to(dev), v0.to(dev)
        p, b, ind, ptr_, tab = args
        if fused:
            mas.apply_rope_and_append_paged_kv_cache(p, q, k, v.view(n, hk, d), d, tab, neox, b, (kc, vc), ind, ptr_)
        else:
            mas.apply_rope_with_cos_sin_cache_inplace(p, q, k, d, tab, neox)
            mas.append_paged_kv_cache(k.view(n, hk, d), v.view(n, hk, d), b, p, (kc, vc), ind, ptr_)
        return buf, kc, vc

    fb, fk, fv = run(True)
    sb, sk, sv = run(False)
    assert torch.equal(fb, sb) and torch.equal(fk, sk) and torch.equal(fv, sv)
    # and against the oracle
    q_bits = bits(qkv[:, : hq * d]).reshape(n, hq, d)
    k_bits = bits(qkv[:, hq * d:(hq + hk) * d]).reshape(n, hk, d)
    want_q, want_k = ops.rope(q_bits, k_bits, pos.numpy(), table.numpy(), is_neox=neox)
    want_kc, want_vc = ops.append_paged_kv_cache(bits(k0), bits(v0), want_k,
                                                 bits(qkv[:, (hq + hk) * d:]).reshape(n, hk, d), bidx.numpy(),
                                                 pos.numpy(), tables.flatten().numpy(), indptr.numpy())
    assert np.array_equal(bits(fb[:, : hq * d]).reshape(n, hq, d), want_q)
    assert np.array_equal(bits(fk), want_kc) and np.array_equal(bits(fv), want_vc)


@pytest.mark.parametrize("beta,interval", [(0.1, 16), (0.5, 7), (1.0, 1)])
def test_rope_append_fused_llama_4_q_scale(mas, dev, beta, interval):
    """RoPE + KV append + llama-4 query scale in one kernel against the reference's three steps
    (devstral2.py:163-179: rope in place, append, then q * bf16(1 + beta * log1p(floor(pos / M))))
    run with the separate ops and the reference's own torch expression: bit-identical q, k and caches.
    Then against the oracle, with the wrapper's scale table checked against the closed form."""
    g = torch.Generator().manual_seed(int(beta * 100) + interval)
    n, hq, hk, d, page_size = 48, 8, 2, 128, 16
    lens = [20, 28]
    bidx = torch.cat([torch.full((m,), b) for b, m in enumerate(lens)]).to(torch.int32)
    pos = (torch.cat([torch.arange(m) for m in lens]) * 3 + 1).to(torch.int32)   # spans several scale intervals
    table = mas.rope.cos_sin_cache(int(pos.max()) + 5, d, 1e6)
    width = -(-(int(pos.max()) + 1) // page_size) + 1
    pages = len(lens) * width + 2
    tables = torch.randperm(pages, generator=g)[: len(lens) * width].to(torch.int32).reshape(len(lens), width)
    indptr = torch.arange(len(lens) + 1, dtype=torch.int32) * width
    qkv = _randn_bf16(g, n, (hq + 2 * hk) * d)
    k0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    v0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    pd, bd, ind, ptr_, tab = pos.to(dev), bidx.to(dev), tables.flatten().to(dev), indptr.to(dev), table.to(dev)

    buf = qkv.to(dev)
    q, k, v = buf.split([hq * d, hk * d, hk * d], dim=-1)
    kc, vc = k0.to(dev), v0.to(dev)
    mas.apply_rope_and_append_paged_kv_cache(pd, q, k, v.view(n, hk, d), d, tab, True, bd, (kc, vc), ind, ptr_,
                                             llama_4_scaling_beta=beta, original_max_position_embeddings=interval)

    sbuf = qkv.to(dev)
    sq, sk, sv = sbuf.split([hq * d, hk * d, hk * d], dim=-1)
    skc, svc = k0.to(dev), v0.to(dev)
    mas.apply_rope_with_cos_sin_cache_inplace(pd, sq, sk, d, tab, True)
    mas.append_paged_kv_cache(sk.view(n, hk, d), sv.view(n, hk, d), bd, pd, (skc, svc), ind, ptr_)
    attn_scale = 1 + beta * torch.log1p(torch.floor(pd.float() / interval))
    ref_q = sq.view(n, hq, d) * attn_scale[:, None, None].to(torch.bfloat16)
    assert torch.equal(q.view(n, hq, d), ref_q)
    assert torch.equal(k, sk) and torch.equal(kc, skc) and torch.equal(vc, svc)

    rows = -(-table.shape[0] // interval)
    scale_table = bits(mas.fused.llama_4_q_scale_table(beta, interval, rows, dev))
    closed = ops.llama_4_q_scale_table(beta, interval, rows)
    assert scale_table[0] == 0x3F80                         # 1.0
    assert np.all(np.abs(scale_table.astype(np.int32) - closed.astype(np.int32)) <= 1)
    q_rot, _ = ops.rope(bits(qkv[:, : hq * d]).reshape(n, hq, d), bits(qkv[:, hq * d:(hq + hk) * d]).reshape(n, hk, d),
                        pos.numpy(), table.numpy())
    want_q = ops.llama_4_scale_q(q_rot, pos.numpy(), scale_table, interval)
    assert np.array_equal(bits(q).reshape(n, hq, d), want_q)


def test_rope_append_fused_error_paths(mas, dev):
    g = torch.Generator().manual_seed(97)
    n, hq, hk, d, ps = 6, 4, 2, 64, 4
    tables = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    indptr = torch.tensor([0, 2, 4], dtype=torch.int32)
    bidx = torch.tensor([0, 0, 1, 1, 7, 1], dtype=torch.int32)
    pos = torch.tensor([1, 5, 30, 2, 0, 3], dtype=torch.int32)      # 30: past the table and the pages
    table = mas.rope.cos_sin_cache(16, d, 1e4)
    qkv = _randn_bf16(g, n, (hq + 2 * hk) * d)
    buf = qkv.to(dev)
    q, k, v = buf.split([hq * d, hk * d, hk * d], dim=-1)
    kc = torch.zeros(4, ps, hk, d, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.apply_rope_and_append_paged_kv_cache(pos.to(dev), q, k, v.view(n, hk, d), d, table.to(dev), True,
                                             bidx.to(dev), (kc, vc), tables.flatten().to(dev), indptr.to(dev),
                                             error_flags=flags)
    assert int(flags.item()) == 2 | 4 | 8
    ok_rope = (pos < 16).numpy()
    want_q, want_k = ops.rope(bits(qkv[:, :hq * d]).reshape(n, hq, d)[ok_rope],
                              bits(qkv[:, hq * d:(hq + hk) * d]).reshape(n, hk, d)[ok_rope], pos.numpy()[ok_rope],
                              table.numpy())
    assert np.array_equal(bits(q).reshape(n, hq, d)[ok_rope], want_q)
    assert np.array_equal(bits(q).reshape(n, hq, d)[~ok_rope], bits(qkv[:, :hq * d]).reshape(n, hq, d)[~ok_rope])
    # tokens 0, 1, 3, 5 land in the cache; token 2 (page slot past its sequence) and 4 (batch 7) do not
    kb = bits(kc)
    k_rot = bits(k).reshape(n, hk, d)
    for t, (page, entry) in {0: (0, 1), 1: (1, 1), 3: (2, 2), 5: (2, 3)}.items():
        assert np.array_equal(kb[page, entry], k_rot[t])
    assert int((kc != 0).any(dim=-1).any(dim=-1).sum()) == 4
