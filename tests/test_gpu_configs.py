"""The five layer-kernel workloads at their full sizes on the GPU.

At these sizes the numpy oracle is too slow, so each kernel is checked through properties that do
not depend on size: bit copies (KV store, embedding) and the residual update (one bf16 rounding of
an fp32 sum) must equal torch's own indexing / bf16 add on the GPU bit for bit; the normalised,
gated and rotated outputs must match a float32 torch reference of the same formula within
rtol 1.6e-2 / atol 1e-2 (the float32 formula is itself checked against the oracle on small inputs
in tests/test_oracle_ops.py); untouched KV slots must stay untouched; RoPE must preserve pair norms.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from conftest import ATOL, RTOL

pytestmark = pytest.mark.gpu

LAYER_SHAPES = ["rmsnorm_256x5120", "decode64_24b", "prefill8192_24b", "prefill16384_123b"]


def _assert_close_bf16(got: torch.Tensor, want_f32: torch.Tensor, chunk: int = 1 << 26):
    g, w = got.reshape(-1), want_f32.reshape(-1)
    for i in range(0, g.numel(), chunk):
        torch.testing.assert_close(g[i:i + chunk].float(), w[i:i + chunk].to(torch.bfloat16).float(), rtol=RTOL,
                                   atol=ATOL)


def _norm_ref(x, r, w, eps):
    s = x.float() + r.float()
    y = s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps) * w.float()
    return s, y


@pytest.mark.parametrize("name", LAYER_SHAPES)
def test_norm_full_size(mas, dev, name):
    shape = mas.workloads.SHAPES[name]
    li = mas.workloads.make_layer_inputs(shape, dev, seed=2, fill_on_device=True, with_cache=False)
    x0, r0 = li.hidden.clone(), li.residual.clone()
    mas.fused_add_rmsnorm(li.hidden, li.residual, li.norm_weight, shape.eps)
    assert torch.equal(li.residual, x0 + r0)           # bf16 add: widen, add in fp32, round once
    rows = 2048
    for i in range(0, shape.tokens, rows):
        _, y = _norm_ref(x0[i:i + rows], r0[i:i + rows], li.norm_weight, shape.eps)
        _assert_close_bf16(li.hidden[i:i + rows], y)
    # fp8 epilogue on the same inputs
    out = torch.empty_like(x0, dtype=torch.float8_e4m3fn)
    res = r0.clone()
    scale = torch.tensor(0.02, device=dev)
    mas.fused_add_rmsnorm_quant(out, x0, res, li.norm_weight, scale, shape.eps)
    assert torch.equal(res, x0 + r0)
    for i in range(0, shape.tokens, rows):
        _, y = _norm_ref(x0[i:i + rows], r0[i:i + rows], li.norm_weight, shape.eps)
        want = (y / 0.02).clamp(-448, 448)
        got = out[i:i + rows].float()
        step = torch.clamp(want.abs() * 2.0 ** -3, min=2.0 ** -9)     # one e4m3 step
        assert bool(((got - want.to(torch.float8_e4m3fn).float()).abs() <= step).all())


@pytest.mark.parametrize("name", LAYER_SHAPES[1:])
def test_silu_and_mul_full_size(mas, dev, name):
    shape = mas.workloads.SHAPES[name]
    li = mas.workloads.make_layer_inputs(shape, dev, seed=3, fill_on_device=True, with_cache=False)
    out = mas.silu_and_mul(li.gate_up)
    rows = 1024
    for i in range(0, shape.tokens, rows):
        g, u = li.gate_up[i:i + rows, : shape.inter].float(), li.gate_up[i:i + rows, shape.inter:].float()
        _assert_close_bf16(out[i:i + rows], F.silu(g) * u)


@pytest.mark.parametrize("name", LAYER_SHAPES[1:])
def test_rope_full_size(mas, dev, name):
    shape = mas.workloads.SHAPES[name]
    li = mas.workloads.make_layer_inputs(shape, dev, seed=4, fill_on_device=True, with_cache=False)
    hq, hk, d = shape.q_heads, shape.kv_heads, shape.head_dim
    q0 = li.q.clone().view(shape.tokens, hq, d)
    k0 = li.k.clone().view(shape.tokens, hk, d)
    v0 = li.v.clone()
    mas.apply_rope_with_cos_sin_cache_inplace(li.positions, li.q, li.k, d, li.table, True)
    assert torch.equal(li.v, v0)
    rows = 1024
    for i in range(0, shape.tokens, rows):
        t = li.table[li.positions[i:i + rows].long()]
        c, s = t[:, None, : d // 2], t[:, None, d // 2:]
        for x0, got in ((q0[i:i + rows], li.q[i:i + rows].view(-1, hq, d)),
                        (k0[i:i + rows], li.k[i:i + rows].view(-1, hk, d))):
            a, b = x0[..., : d // 2].float(), x0[..., d // 2:].float()
            want = torch.cat([a * c - b * s, b * c + a * s], dim=-1)
            _assert_close_bf16(got, want)
            n_in = a.pow(2) + b.pow(2)
            n_out = got[..., : d // 2].float().pow(2) + got[..., d // 2:].float().pow(2)
            torch.testing.assert_close(n_out, n_in, rtol=4 * 2 ** -7, atol=1e-3)


@pytest.mark.parametrize("name", LAYER_SHAPES[1:])
@pytest.mark.parametrize("form", ["block_table", "slots"])
def test_kv_store_full_size(mas, dev, name, form):
    shape = mas.workloads.SHAPES[name]
    li = mas.workloads.make_layer_inputs(shape, dev, seed=5, fill_on_device=True)
    hk, d = shape.kv_heads, shape.head_dim
    k = li.k.view(shape.tokens, hk, d)
    v = li.v.view(shape.tokens, hk, d)
    sentinel = torch.tensor(-7.0, dtype=torch.bfloat16)
    li.k_cache.fill_(sentinel)
    li.v_cache.fill_(sentinel)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    if form == "block_table":
        mas.append_paged_kv_cache(k, v, li.batch_indices, li.positions, (li.k_cache, li.v_cache),
                                  li.block_tables.flatten(), li.kv_indptr, None, "NHD", error_flags=flags)
    else:
        mas.store_kv_slots(k, v, li.k_cache, li.v_cache, li.slot_mapping, error_flags=flags)
    assert int(flags.item()) == 0
    flat_k = li.k_cache.view(-1, hk, d)
    flat_v = li.v_cache.view(-1, hk, d)
    assert torch.equal(flat_k[li.slot_mapping], k) and torch.equal(flat_v[li.slot_mapping], v)
    touched = torch.zeros(flat_k.shape[0], dtype=torch.bool, device=dev)
    touched[li.slot_mapping] = True
    assert bool((flat_k[~touched] == sentinel).all()) and bool((flat_v[~touched] == sentinel).all())


def test_decode_pass_full_size(mas, dev):
    """The 40-layer, 256-sequence decode pass: every layer's kernels checked against float32 torch."""
    shape = mas.workloads.SHAPES["decode_pass_256x40"]
    p = mas.layer_pass.DecodePass(shape, dev, seed=6)
    hq, hk, d = shape.q_heads, shape.kv_heads, shape.head_dim
    before = [(b.inputs.hidden.clone(), b.inputs.attn_out.clone(), b.inputs.qkv.clone()) for b in p.layers]
    p.run()
    torch.cuda.synchronize()
    emb = p.embed_table[p.ids]
    residual = torch.zeros(shape.tokens, shape.hidden, dtype=torch.bfloat16, device=dev)
    for i, b in enumerate(p.layers):
        li = b.inputs
        h0, a0, qkv0 = before[i]
        if i == 0:
            h0 = emb                       # layer 0's first norm reads the embedding output
        s1, y1 = _norm_ref(h0, residual, li.norm_weight, shape.eps)
        residual = (h0 + residual)
        _assert_close_bf16(li.hidden, y1)
        s2, y2 = _norm_ref(a0, residual, li.post_norm_weight, shape.eps)
        residual = (a0 + residual)
        _assert_close_bf16(li.attn_out, y2)
        g, u = li.gate_up[:, : shape.inter].float(), li.gate_up[:, shape.inter:].float()
        _assert_close_bf16(b.silu_out, F.silu(g) * u)
        t = li.table[li.positions.long()]
        c, s = t[:, None, : d // 2], t[:, None, d // 2:]
        k0 = qkv0[:, hq * d:(hq + hk) * d].view(-1, hk, d).float()
        want_k = torch.cat([k0[..., : d // 2] * c - k0[..., d // 2:] * s,
                            k0[..., d // 2:] * c + k0[..., : d // 2] * s], -1)
        _assert_close_bf16(li.k.view(-1, hk, d), want_k)
        assert torch.equal(li.k_cache.view(-1, hk, d)[li.slot_mapping], li.k.view(-1, hk, d))
        assert torch.equal(li.v_cache.view(-1, hk, d)[li.slot_mapping], li.v.view(-1, hk, d))
    # the shared residual stream ends where the chain of bf16 adds does
    assert torch.equal(p.layers[0].inputs.residual, residual)


def test_embedding_full_size(mas, dev):
    shape = mas.workloads.SHAPES["decode_pass_256x40"]
    gen = torch.Generator(device=dev).manual_seed(8)
    table = torch.randn(shape.vocab, shape.hidden, generator=gen, device=dev).to(torch.bfloat16)
    ids = torch.randint(0, shape.vocab, (shape.tokens,), device=dev)
    ids[0], ids[1] = 0, shape.vocab - 1
    assert torch.equal(mas.embedding.embedding(ids, table), F.embedding(ids, table))
