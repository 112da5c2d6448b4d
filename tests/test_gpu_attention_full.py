"""Decode and context attention at the benchmark's full sizes (64 decode rows up to 8192 positions;
4 prompts of 2048 and of 4096 tokens), for both head groups (4 and 12 query heads per kv head).

At these sizes the numpy oracle is too slow, so the kernels are checked against a float32 torch
restatement of the same formula on the GPU, within rtol 1.6e-2 / atol 1e-2 after one bf16 rounding
of the reference. That restatement is itself checked against the oracle on small inputs on the CPU
(the two tests without the gpu marker), where a dropped scale, a transposed operand or a missing
causal mask would fail it."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL, bits
from oracle import ops


def _gather(cache: torch.Tensor, table_row: torch.Tensor, length: int) -> torch.Tensor:
    """Positions 0..length-1 of one row's pages: [length, Hk, D] float32."""
    page_size = cache.shape[1]
    pages = table_row[: -(-length // page_size)].long()
    return cache[pages].reshape(-1, cache.shape[2], cache.shape[3])[:length].float()


def decode_reference_f32(q, k_cache, v_cache, tables, seq_lens, scale1, scale2=1.0) -> torch.Tensor:
    """out[b, h] = scale2 * softmax(scale1 * q[b, h] . K_b^T) V_b over the row's positions, float32."""
    batch, hq, dim = q.shape
    hk = k_cache.shape[2]
    group = hq // hk
    out = torch.zeros(batch, hq, dim, dtype=torch.float32, device=q.device)
    for b in range(batch):
        n = int(seq_lens[b])
        if n == 0:
            continue
        k = _gather(k_cache, tables[b], n).permute(1, 2, 0).contiguous()   # [Hk, D, n]
        v = _gather(v_cache, tables[b], n).permute(1, 0, 2).contiguous()   # [Hk, n, D]
        qg = q[b].float().reshape(hk, group, dim)
        p = torch.softmax(torch.bmm(qg, k) * scale1, dim=-1)
        out[b] = (torch.bmm(p, v) * scale2).reshape(hq, dim)
    return out


def context_reference_f32(q, k_cache, v_cache, tables, seq_lens, cu, scale1, scale2=1.0) -> torch.Tensor:
    """Causal attention aligned to the end of each row's cached positions, float32."""
    tokens, hq, dim = q.shape
    hk = k_cache.shape[2]
    group = hq // hk
    out = torch.zeros(tokens, hq, dim, dtype=torch.float32, device=q.device)
    for j in range(len(cu) - 1):
        t0, t1 = int(cu[j]), int(cu[j + 1])
        n, ql = int(seq_lens[j]), t1 - t0
        if ql == 0:
            continue
        k = _gather(k_cache, tables[j], n).permute(1, 2, 0).contiguous()   # [Hk, D, n]
        v = _gather(v_cache, tables[j], n).permute(1, 0, 2).contiguous()   # [Hk, n, D]
        pos = torch.arange(n - ql, n, device=q.device)[:, None]             # each token's own position
        allowed = torch.arange(n, device=q.device)[None, :] <= pos          # [ql, n]
        for kv in range(hk):                                                # one kv head at a time: [G, ql, n]
            qh = q[t0:t1, kv * group:(kv + 1) * group].float().permute(1, 0, 2).contiguous()
            s = torch.matmul(qh, k[kv]) * scale1
            s = s.masked_fill(~allowed, float("-inf"))
            o = torch.matmul(torch.softmax(s, dim=-1), v[kv]) * scale2      # [G, ql, D]
            out[t0:t1, kv * group:(kv + 1) * group] = o.permute(1, 0, 2)
    return out


def _assert_close(got: torch.Tensor, want_f32: torch.Tensor):
    torch.testing.assert_close(got.float(), want_f32.to(torch.bfloat16).float(), rtol=RTOL, atol=ATOL)


def _small_paged(seed, tokens, hq, hk, dim, page_size, lens):
    g = torch.Generator().manual_seed(seed)
    width = max(1, max(-(-n // page_size) for n in lens))
    pages = len(lens) * width + 2
    q = torch.randn(tokens, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    tables = torch.randperm(pages, generator=g)[: len(lens) * width].reshape(len(lens), width).to(torch.int32)
    return q, kc, vc, tables, torch.tensor(lens, dtype=torch.int32)


def test_decode_reference_matches_the_oracle():
    q, kc, vc, tables, seq = _small_paged(3, 3, 24, 2, 64, 16, [40, 1, 0])
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 0.11, 0.7)
    got = decode_reference_f32(q, kc, vc, tables, seq, 0.11, 0.7).bfloat16()
    np.testing.assert_array_equal(bits(got) != 0, want != 0)
    _assert_close(got, torch.from_numpy(want.astype(np.int32) << 16).view(torch.float32))


def test_context_reference_matches_the_oracle():
    q_lens, kv_lens = [9, 0, 5], [30, 4, 5]            # chunked prefill, an empty row, a plain prompt
    q, kc, vc, tables, seq = _small_paged(4, sum(q_lens), 24, 2, 64, 8, kv_lens)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(),
                                       0.13, 0.8)
    got = context_reference_f32(q, kc, vc, tables, seq, cu, 0.13, 0.8)
    _assert_close(got.bfloat16(), torch.from_numpy(want.astype(np.int32) << 16).view(torch.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["decode_attn_64x8192_24b", "decode_attn_64x8192_123b"])
def test_decode_attention_full_size(mas, dev, name):
    inp = mas.workloads.make_attention_inputs(name, dev, seed=5)
    scale = inp.shape.head_dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = mas.attention.trtllm_batch_decode_with_kv_cache(
        inp.q, (inp.k_cache, inp.v_cache), inp.workspace, inp.block_tables, inp.seq_lens, 0, scale, 1.0,
        kv_layout="NHD", error_flags=flags)
    want = decode_reference_f32(inp.q, inp.k_cache, inp.v_cache, inp.block_tables.cpu(), inp.seq_lens.cpu(), scale)
    _assert_close(out, want)
    assert int(flags.item()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["context_attn_4x2048_24b", "context_attn_4x4096_123b"])
def test_context_attention_full_size(mas, dev, name):
    inp = mas.workloads.make_context_inputs(name, dev, seed=6)
    s = inp.shape
    scale = s.head_dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    out = mas.attention.trtllm_batch_context_with_kv_cache(
        inp.q, (inp.k_cache, inp.v_cache), ws, inp.block_tables, inp.seq_lens, s.q_len, s.cached + s.q_len,
        scale, 1.0, s.rows, inp.cu_seqlens_q, None, kv_layout="NHD", error_flags=flags)
    want = context_reference_f32(inp.q, inp.k_cache, inp.v_cache, inp.block_tables.cpu(), inp.seq_lens.cpu(),
                                 inp.cu_seqlens_q.cpu(), scale)
    _assert_close(out, want)
    assert int(flags.item()) == 0


def _grid_order_tile_major(cus: int, rows: int, q_len: int, kv_hint: int, hq: int, hk: int) -> bool:
    """The launch's choice between rows in turn and tile-major order for a grid launch: fewer than 8
    rows, and the longest tile's time against the launch's time per resident workgroup."""
    group = hq // hk
    waves, tokens = (8, 64) if group >= 8 else (4, 32)
    gx, gy = hk * -(-group // 4), -(-q_len // tokens)
    mean = max(kv_hint - q_len // 2 + tokens // 2, tokens)
    return rows < 8 and 10 * kv_hint * cus * (8 // waves) >= 3 * rows * gx * gy * mean


@pytest.mark.gpu
def test_context_attention_grid_orders_agree(mas, dev):
    """4 prompts of 2048 tokens under a block table 32768 positions wide: the max_kv_len hint moves
    the launch between its two grid orders (rows in turn, or every row's longest tiles first).
    Workgroups compute the same tiles either way, so the outputs are bit-identical, and both match
    the float32 restatement."""
    rows, q_len, hq, hk, dim, ps, width = 4, 2048, 32, 8, 128, 256, 128
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    if _grid_order_tile_major(cus, rows, q_len, q_len, hq, hk) == _grid_order_tile_major(cus, rows, q_len,
                                                                                          width * ps, hq, hk):
        pytest.skip(f"on {cus} CUs both hints pick the same order")
    g = torch.Generator().manual_seed(11)
    pages = rows * (q_len // ps) + 1
    q = torch.randn(rows * q_len, hq, dim, generator=g).bfloat16().to(dev)
    kc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16().to(dev)
    vc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16().to(dev)
    tables = torch.zeros(rows, width, dtype=torch.int32)
    per_row = q_len // ps
    tables[:, :per_row] = (torch.randperm(pages - 1, generator=g)[: rows * per_row].reshape(rows, per_row)
                           .to(torch.int32) + 1)
    tables = tables.to(dev)
    seq = torch.full((rows,), q_len, dtype=torch.int32, device=dev)
    cu = torch.arange(0, rows * q_len + 1, q_len, dtype=torch.int32, device=dev)
    scale = dim ** -0.5
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    outs = []
    for hint in (q_len, width * ps):
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        outs.append(mas.attention.trtllm_batch_context_with_kv_cache(
            q, (kc, vc), ws, tables, seq, q_len, hint, scale, 1.0, rows, cu, None, kv_layout="NHD",
            error_flags=flags))
        assert int(flags.item()) == 0
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    want = context_reference_f32(q, kc, vc, tables.cpu(), seq.cpu(), cu.cpu(), scale)
    _assert_close(outs[0], want)
