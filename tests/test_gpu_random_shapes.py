"""Seeded random shapes for the layer ops against the oracle, through the C ABI: row counts,
widths (ragged ones included, which take the generic paths), head counts, head dims, rotary dims,
page sizes and position ranges drawn per seed. The same bars as the fixed-shape parity tests:
residual, RoPE, KV store, fused RoPE + KV and embedding bit-exact; bf16 arithmetic within
rtol 1.6e-2 / atol 1e-2."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL, bits
from oracle import numerics as on
from oracle import ops

pytestmark = pytest.mark.gpu

SEEDS = range(16)


def _bf16(gen, *shape, scale=1.0, shift=0.0):
    return (shift + scale * torch.randn(*shape, generator=gen)).bfloat16()


def _close(got_bits, want_bits, min_exact):
    np.testing.assert_allclose(on.bf16_to_f32(got_bits), on.bf16_to_f32(want_bits), rtol=RTOL, atol=ATOL)
    if got_bits.size:
        assert np.mean(got_bits == want_bits) >= min_exact


@pytest.mark.parametrize("seed", SEEDS)
def test_fused_add_rmsnorm_random(mas, dev, seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 300))
    hidden = int(rng.choice([int(rng.integers(1, 4000)), 8 * int(rng.integers(1, 2048))]))
    g = torch.Generator().manual_seed(seed)
    x, r = _bf16(g, rows, hidden), _bf16(g, rows, hidden)
    w = _bf16(g, hidden, scale=0.1, shift=1.0)
    want_x, want_r = ops.fused_add_rmsnorm(bits(x), bits(r), bits(w), 1e-5)
    xd, rd = x.to(dev), r.to(dev)
    mas.fused_add_rmsnorm(xd, rd, w.to(dev), 1e-5)
    assert np.array_equal(bits(rd), want_r)
    _close(bits(xd), want_x, 0.98)


@pytest.mark.parametrize("seed", SEEDS)
def test_silu_and_mul_random(mas, dev, seed):
    rng = np.random.default_rng(100 + seed)
    rows = int(rng.integers(1, 400))
    inter = int(rng.choice([int(rng.integers(1, 3000)), 8 * int(rng.integers(1, 2000))]))
    g = torch.Generator().manual_seed(100 + seed)
    x = _bf16(g, rows, 2 * inter, scale=3.0)
    out = mas.silu_and_mul(x.to(dev))
    _close(bits(out), ops.silu_and_mul(bits(x)), 0.97)


@pytest.mark.parametrize("seed", SEEDS)
def test_rope_random(mas, dev, seed):
    rng = np.random.default_rng(200 + seed)
    n = int(rng.integers(1, 400))
    hk = int(rng.choice([1, 2, 8]))
    hq = hk * int(rng.choice([1, 2, 4, 12]))
    head_dim = int(rng.choice([64, 128, 256]))
    rotary_dim = int(rng.choice([d for d in (32, 64, 128, 256) if d <= head_dim]))
    neox = bool(rng.integers(0, 2))
    max_pos = int(rng.choice([64, 4096, 40000]))
    g = torch.Generator().manual_seed(200 + seed)
    qkv = _bf16(g, n, (hq + 2 * hk) * head_dim)
    table = mas.rope.cos_sin_cache(max_pos, rotary_dim, 1e6)
    pos = torch.randint(0, max_pos, (n,), generator=g)
    q = qkv[:, : hq * head_dim].reshape(n, hq, head_dim)
    k = qkv[:, hq * head_dim: (hq + hk) * head_dim].reshape(n, hk, head_dim)
    want_q, want_k = ops.rope(bits(q), bits(k), pos.numpy(), table.numpy(), is_neox=neox)
    qkv_d = qkv.to(dev)
    qd, kd, _ = qkv_d.split([hq * head_dim, hk * head_dim, hk * head_dim], dim=-1)
    mas.apply_rope_with_cos_sin_cache_inplace(pos.to(dev), qd, kd, head_dim, table.to(dev), neox)
    assert np.array_equal(bits(qd).reshape(n, hq, head_dim), want_q)
    assert np.array_equal(bits(kd).reshape(n, hk, head_dim), want_k)
    assert torch.equal(qkv_d[:, (hq + hk) * head_dim:].cpu(), qkv[:, (hq + hk) * head_dim:])


def _paged_rows(rng, g, page_size):
    """1-6 rows of 1-300 new tokens each after 0-500 earlier positions; distinct pages per row."""
    rows = int(rng.integers(1, 7))
    starts = [int(rng.integers(0, 501)) for _ in range(rows)]
    lens = [int(rng.integers(1, 301)) for _ in range(rows)]
    width = max(-(-(s + n) // page_size) for s, n in zip(starts, lens))
    pages = rows * width + 2
    tables = torch.randperm(pages, generator=g)[: rows * width].reshape(rows, width).to(torch.int32)
    indptr = (torch.arange(rows + 1) * width).to(torch.int32)
    bidx = torch.cat([torch.full((n,), b) for b, n in enumerate(lens)]).to(torch.int32)
    pos = torch.cat([torch.arange(s, s + n) for s, n in zip(starts, lens)]).to(torch.int32)
    return pages, tables, indptr, bidx, pos


@pytest.mark.parametrize("seed", SEEDS)
def test_append_paged_kv_cache_random(mas, dev, seed):
    rng = np.random.default_rng(300 + seed)
    g = torch.Generator().manual_seed(300 + seed)
    page_size = int(rng.choice([4, 16, 64, 256]))
    heads = int(rng.choice([1, 2, 8]))
    dim = int(rng.choice([64, 128, 256]))
    pages, tables, indptr, bidx, pos = _paged_rows(rng, g, page_size)
    n = len(pos)
    qkv = _bf16(g, n, (2 + 2 * heads) * dim)
    key = qkv[:, 2 * dim:(2 + heads) * dim].reshape(n, heads, dim)
    val = qkv[:, (2 + heads) * dim:].reshape(n, heads, dim)
    k0 = torch.randn(pages, page_size, heads, dim, generator=g).bfloat16()
    v0 = torch.randn(pages, page_size, heads, dim, generator=g).bfloat16()
    want_k, want_v = ops.append_paged_kv_cache(bits(k0), bits(v0), bits(key), bits(val), bidx.numpy(), pos.numpy(),
                                               tables.flatten().numpy(), indptr.numpy())
    qkv_d = qkv.to(dev)
    kc, vc = k0.to(dev), v0.to(dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.append_paged_kv_cache(qkv_d[:, 2 * dim:(2 + heads) * dim].view(n, heads, dim),
                              qkv_d[:, (2 + heads) * dim:].view(n, heads, dim), bidx.to(dev), pos.to(dev), (kc, vc),
                              tables.flatten().to(dev), indptr.to(dev), None, "NHD", error_flags=flags)
    assert int(flags.item()) == 0
    assert np.array_equal(bits(kc), want_k) and np.array_equal(bits(vc), want_v)


@pytest.mark.parametrize("seed", SEEDS)
def test_rope_append_fused_random(mas, dev, seed):
    rng = np.random.default_rng(400 + seed)
    g = torch.Generator().manual_seed(400 + seed)
    page_size = int(rng.choice([8, 16, 256]))
    hk = int(rng.choice([1, 2, 8]))
    hq = hk * int(rng.choice([0, 1, 4, 12]))
    d = int(rng.choice([64, 128, 256]))
    neox = bool(rng.integers(0, 2))
    pages, tables, indptr, bidx, pos = _paged_rows(rng, g, page_size)
    n = len(pos)
    table = mas.rope.cos_sin_cache(int(pos.max()) + 1 + int(rng.integers(0, 100)), d, 1e6)
    qkv = _bf16(g, n, (hq + 2 * hk) * d)
    k0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    v0 = torch.randn(pages, page_size, hk, d, generator=g).bfloat16()
    buf = qkv.to(dev)
    q, k, v = buf.split([hq * d, hk * d, hk * d], dim=-1)
    kc, vc = k0.to(dev), v0.to(dev)
    mas.apply_rope_and_append_paged_kv_cache(pos.to(dev), q, k, v.view(n, hk, d), d, table.to(dev), neox,
                                             bidx.to(dev), (kc, vc), tables.flatten().to(dev), indptr.to(dev))
    q_bits = bits(qkv[:, : hq * d]).reshape(n, hq, d)
    k_bits = bits(qkv[:, hq * d:(hq + hk) * d]).reshape(n, hk, d)
    want_q, want_k = ops.rope(q_bits, k_bits, pos.numpy(), table.numpy(), is_neox=neox)
    want_kc, want_vc = ops.append_paged_kv_cache(bits(k0), bits(v0), want_k,
                                                 bits(qkv[:, (hq + hk) * d:]).reshape(n, hk, d), bidx.numpy(),
                                                 pos.numpy(), tables.flatten().numpy(), indptr.numpy())
    assert np.array_equal(bits(buf[:, : hq * d]).reshape(n, hq, d), want_q)
    assert np.array_equal(bits(kc), want_kc) and np.array_equal(bits(vc), want_vc)


@pytest.mark.parametrize("seed", SEEDS)
def test_embedding_random(mas, dev, seed):
    rng = np.random.default_rng(500 + seed)
    rows = int(rng.integers(1, 600))
    vocab = int(rng.integers(1, 5000))
    hidden = int(rng.choice([int(rng.integers(1, 3000)), 8 * int(rng.integers(1, 1024))]))
    g = torch.Generator().manual_seed(500 + seed)
    table = _bf16(g, vocab, hidden)
    ids = torch.randint(0, vocab, (rows,), generator=g)
    out = mas.embedding.embedding(ids.to(dev), table.to(dev))
    assert np.array_equal(bits(out), ops.embedding(bits(table), ids.numpy()))
