"""Paged decode attention (trtllm_batch_decode_with_kv_cache, devstral2.py:184-196) on the GPU
against the oracle, through the C ABI. bf16 outputs within rtol 1.6e-2 / atol 1e-2, most of them
bit-identical (the fp32 sums run in a different order than numpy's)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL, bits
from oracle import numerics as on
from oracle import ops

pytestmark = pytest.mark.gpu


def _case(seed, batch, hq, hk, dim, page_size, lens, extra_pages=3):
    g = torch.Generator().manual_seed(seed)
    width = max(1, max(-(-n // page_size) for n in lens))
    pages = batch * width + extra_pages
    q = torch.randn(batch, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    tables = torch.randperm(pages, generator=g)[: batch * width].reshape(batch, width).to(torch.int32)
    return q, kc, vc, tables, torch.tensor(lens, dtype=torch.int32)


def _check(got, want, min_exact=0.9):
    gv, wv = on.bf16_to_f32(got), on.bf16_to_f32(want)
    np.testing.assert_allclose(gv, wv, rtol=RTOL, atol=ATOL)
    assert np.mean(got == want) >= min_exact


def _run(mas, dev, q, kc, vc, tables, seq, scale, workspace_bytes=None, out=None, flags=None, scale2=1.0):
    if workspace_bytes is None:
        workspace_bytes = 128 << 20
    ws = torch.zeros(workspace_bytes, dtype=torch.uint8, device=dev)
    return mas.attention.trtllm_batch_decode_with_kv_cache(
        q.to(dev) if q.device.type == "cpu" else q, (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev),
        0, scale, scale2, out=out, kv_layout="NHD", error_flags=flags)


CASES = [
    (4, 32, 8, 128, 256, [1, 255, 256, 5000]),      # Devstral-Small-2 heads, chunk edges, a long row
    (3, 96, 8, 128, 256, [700, 3, 1300]),          # the 123B head group (12 per kv head)
    (5, 8, 8, 128, 16, [17, 1, 64, 300, 0]),       # one head per kv head, small pages, an empty row
    (2, 16, 2, 64, 32, [100, 1000]),               # head_dim 64, 8 per kv head
    (2, 16, 1, 256, 64, [513, 77]),                # head_dim 256, 16 per kv head
    (3, 6, 2, 128, 4, [9, 40, 2]),                 # 3 per kv head (padded), pages of 4
    (2, 16, 4, 128, 512, [700, 1500]),             # pages of two chunks
    (2, 8, 2, 128, 256, [9000, 100]),              # 36 splits: the combine's path past 32 splits
    (2, 16, 2, 64, 256, [600, 257]),               # head_dim 64 on pages of a chunk (scalar page ids)
    (2, 16, 1, 256, 512, [1100, 300]),             # head_dim 256 on pages of two chunks
]


@pytest.mark.parametrize("batch,hq,hk,dim,page_size,lens", CASES)
def test_decode_attention_matches_oracle(mas, dev, batch, hq, hk, dim, page_size, lens):
    q, kc, vc, tables, seq = _case(batch * 7 + dim + hq, batch, hq, hk, dim, page_size, lens)
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, scale, flags=flags)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), scale)
    _check(bits(out), want)
    assert int(flags.item()) == 0
    if 0 in lens:
        assert not out[lens.index(0)].any()


@pytest.mark.parametrize("page_size", [16, 256])
def test_decode_attention_hnd_layout(mas, dev, page_size):
    """kv_layout="HND" ([pages, kv_heads, page_size, head_dim]): the same results as NHD."""
    batch, hq, hk, dim, lens = 3, 32, 8, 128, [300, 1, 777]
    q, kc, vc, tables, seq = _case(21 + page_size, batch, hq, hk, dim, page_size, lens)
    ws = torch.zeros(128 << 20, dtype=torch.uint8, device=dev)
    kh, vh = kc.transpose(1, 2).contiguous().to(dev), vc.transpose(1, 2).contiguous().to(dev)
    out = mas.attention.trtllm_batch_decode_with_kv_cache(q.to(dev), (kh, vh), ws, tables.to(dev), seq.to(dev), 0,
                                                          dim ** -0.5, 1.0, kv_layout="HND")
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), dim ** -0.5)
    _check(bits(out), want)


def test_decode_attention_single_and_multi_split_rows(mas, dev):
    """Rows that fit one split are written by the split kernel and skipped by the combine kernel;
    longer rows go through the partials. A batch mixing both (and empty rows), on a workspace whose
    previous contents are garbage (0xff), matches the oracle."""
    ws = torch.full((8 << 20,), 255, dtype=torch.uint8, device=dev)
    for seed, (batch, hq, hk, lens) in enumerate([(4, 32, 8, [3000, 1, 0, 700]), (2, 96, 8, [9000, 5]),
                                                  (3, 16, 2, [256, 257, 5000])]):
        q, kc, vc, tables, seq = _case(40 + seed, batch, hq, hk, 128, 256, lens)
        out = mas.attention.trtllm_batch_decode_with_kv_cache(q.to(dev), (kc.to(dev), vc.to(dev)), ws,
                                                              tables.to(dev), seq.to(dev), 0, 0.088, 1.0)
        torch.cuda.synchronize()
        want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 0.088)
        _check(bits(out), want)


@pytest.mark.parametrize("batch,hq,hk,page_size,lens", [
    (1, 32, 8, 256, [4096]),              # one row: 64 splits of 64 positions (big pages)
    (2, 96, 8, 16, [2000, 129]),          # 123B heads, small pages: block-table entries from mid-chunk starts
    (3, 16, 2, 64, [63, 64, 65]),         # rows at the edge of one short split
])
def test_decode_attention_small_grids_take_short_splits(mas, dev, batch, hq, hk, page_size, lens):
    """Grids of fewer (row, kv head, split) items than the GPU has SIMDs split rows into 128- or
    64-position pieces (more wavefronts, fewer dependent steps each); results as the oracle's."""
    q, kc, vc, tables, seq = _case(50 + batch, batch, hq, hk, 128, page_size, lens)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, 0.088, flags=flags)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 0.088)
    _check(bits(out), want)
    assert int(flags.item()) == 0


def test_decode_attention_long_splits_and_bmm2_scale(mas, dev):
    """A workspace too small for one split per 256 positions makes each wavefront walk several
    chunks, merging them with the running max: same results as the oracle."""
    batch, hq, hk, dim, ps, lens = 3, 32, 8, 128, 256, [3000, 1, 2049]
    q, kc, vc, tables, seq = _case(11, batch, hq, hk, dim, ps, lens)
    full = mas.attention.decode_workspace_bytes(batch, hq, dim, tables.shape[1], ps, 1)
    four = mas.attention.decode_workspace_bytes(batch, hq, dim, tables.shape[1], ps, 4)
    assert four < full
    out = _run(mas, dev, q, kc, vc, tables, seq, 0.09, workspace_bytes=four, scale2=0.5)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 0.09, 0.5)
    _check(bits(out), want)
    with pytest.raises(mas._lib.KernelError):
        _run(mas, dev, q, kc, vc, tables, seq, 0.09, workspace_bytes=16)


@pytest.mark.parametrize("batch,hq,hk,width,max_len", [
    (32, 16, 8, 2048, 1500),    # 32 x 8 x 128 splits of one chunk > 16384: two chunks per split
    (4500, 2, 2, 64, 400),      # 4500 x 2 x 2 splits of two chunks > 16384: one split of 4 chunks per row
    (2, 4, 2, 2048, 1500),      # a small grid, but 128 chunks per row > 64 splits: two chunks per split
])
def test_decode_attention_large_grids_take_longer_splits(mas, dev, batch, hq, hk, width, max_len):
    """Past 16384 (row, kv head, split) work items or 64 splits per row the kernel walks several
    chunks per split even with a full workspace; results as the oracle's. The block tables are wide (16-slot pages) and
    the rows short, so the oracle stays cheap while the grid is large."""
    dim, ps = 128, 16
    g = torch.Generator().manual_seed(batch)
    lens = torch.randint(1, max_len + 1, (batch,), generator=g).to(torch.int32)
    pages = int(((lens + ps - 1) // ps).sum()) + 1
    tables = torch.randint(0, pages, (batch, width), generator=g, dtype=torch.int32)
    q = torch.randn(batch, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16()
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, lens, 0.09, flags=flags)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), lens.numpy(), 0.09)
    _check(bits(out), want)
    assert int(flags.item()) == 0


def test_decode_attention_strided_query_and_out(mas, dev):
    """q as the column view of the qkv rows (row stride (Hq + 2 Hk) * D), out as a strided view."""
    batch, hq, hk, dim, ps, lens = 4, 32, 8, 128, 16, [33, 70, 5, 16]
    _, kc, vc, tables, seq = _case(5, batch, hq, hk, dim, ps, lens)
    g = torch.Generator().manual_seed(6)
    qkv = torch.randn(batch, (hq + 2 * hk) * dim, generator=g).bfloat16().to(dev)
    q = qkv[:, : hq * dim].view(batch, hq, dim)
    out_base = torch.full((batch, hq + 1, dim), 3.0, dtype=torch.bfloat16, device=dev)
    out = out_base[:, 1:]
    _run(mas, dev, q, kc, vc, tables, seq, 0.1, out=out)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 0.1)
    _check(bits(out), want)
    assert torch.all(out_base[:, 0] == 3.0)


def test_decode_attention_error_paths(mas, dev):
    batch, hq, hk, dim, ps = 3, 8, 2, 128, 16
    q, kc, vc, tables, _ = _case(9, batch, hq, hk, dim, ps, [40, 40, 40])
    pages = kc.shape[0]
    bad = tables.clone()
    bad[0, 1] = pages + 5                               # positions 16..31 of row 0 point past the cache
    seq = torch.tensor([40, 10_000, 20], dtype=torch.int32)   # row 1 past the table's reach (3 pages = 48)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, bad, seq, 0.1, flags=flags)
    assert int(flags.item()) == 2 | 8
    # row 0 without positions 16..31: the oracle on the remaining rows
    keep = [p for p in range(40) if not 16 <= p < 32]
    kc2 = torch.cat([kc, torch.zeros(1, ps, hk, dim, dtype=torch.bfloat16)])
    vc2 = torch.cat([vc, torch.zeros(1, ps, hk, dim, dtype=torch.bfloat16)])
    # rebuild row 0's keys as a contiguous sequence in fresh pages
    k_rows = kc[tables[0, torch.tensor(keep) // ps].long(), torch.tensor(keep) % ps]
    v_rows = vc[tables[0, torch.tensor(keep) // ps].long(), torch.tensor(keep) % ps]
    n = len(keep)
    kc3 = torch.zeros(2, ps, hk, dim, dtype=torch.bfloat16)
    vc3 = torch.zeros_like(kc3)
    kc3.view(-1, hk, dim)[:n] = k_rows
    vc3.view(-1, hk, dim)[:n] = v_rows
    want0 = ops.paged_decode_attention(bits(q[:1]), bits(kc3), bits(vc3), np.array([[0, 1]]), np.array([n]), 0.1)
    _check(bits(out[:1]), want0)
    # row 1 clamped to 48 positions, row 2 untouched
    want = ops.paged_decode_attention(bits(q), bits(kc2), bits(vc2), tables.numpy(), np.array([40, 48, 20]), 0.1)
    _check(bits(out[1:]), want[1:])


def test_decode_attention_in_graph_replays(mas, dev):
    batch, hq, hk, dim, ps, lens = 4, 32, 8, 128, 256, [300, 1, 2000, 17]
    q, kc, vc, tables, seq = _case(21, batch, hq, hk, dim, ps, lens)
    qd, kd, vd, td, sd = q.to(dev), kc.to(dev), vc.to(dev), tables.to(dev), seq.to(dev)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=dev)
    out = torch.empty(batch, hq, dim, dtype=torch.bfloat16, device=dev)

    def call():
        mas.attention.trtllm_batch_decode_with_kv_cache(qd, (kd, vd), ws, td, sd, 0, 0.088, 1.0, out=out)

    call()
    torch.cuda.synchronize()
    want = out.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)


@pytest.mark.parametrize("dim,hq,hk,scale_kind", [(128, 32, 8, "tensor"), (64, 16, 2, "float"),
                                                 (256, 16, 1, "tensor")])
def test_decode_attention_fp8_output_is_the_o_proj_quantize(mas, dev, dim, hq, hk, scale_kind):
    """With out_quant_scale the kernel writes fp8(clamp(bf16(O) / scale, -448, 448)): bit for bit the
    o_proj input quantize (devstral2.py:93-95,110-111) of its own bf16 output. The small scale
    saturates part of the outputs."""
    batch, ps, lens = 3, 32, [300, 1, 77]
    q, kc, vc, tables, seq = _case(dim + hq, batch, hq, hk, dim, ps, lens)
    ref = _run(mas, dev, q, kc, vc, tables, seq, 0.3, scale2=4.0)
    for s in (0.004, 0.37):
        scale = torch.tensor([s], dtype=torch.float32, device=dev) if scale_kind == "tensor" else s
        ws = torch.zeros(128 << 20, dtype=torch.uint8, device=dev)
        out = mas.attention.trtllm_batch_decode_with_kv_cache(
            q.to(dev), (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev), 0, 0.3, 4.0,
            kv_layout="NHD", out_quant_scale=scale)
        assert out.dtype == torch.float8_e4m3fn and tuple(out.shape) == (batch, hq, dim)
        codes = out.view(torch.uint8).cpu().numpy()
        np.testing.assert_array_equal(codes, ops.quantize_activation(bits(ref), s))
        torch_q = (ref.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        assert torch.equal(out.view(torch.uint8), torch_q.view(torch.uint8))
    assert np.mean(np.abs(on.bf16_to_f32(bits(ref))) / 0.004 > 448.0) > 0.01


def test_decode_attention_fp8_output_argument_checks(mas, dev):
    batch, hq, hk, dim, ps, lens = 2, 8, 2, 128, 16, [20, 5]
    q, kc, vc, tables, seq = _case(2, batch, hq, hk, dim, ps, lens)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    args = (q.to(dev), (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev), 0, 0.1, 1.0)
    with pytest.raises(ValueError):       # fp8 output without a scale
        mas.attention.trtllm_batch_decode_with_kv_cache(*args, out_dtype=torch.float8_e4m3fn)
    with pytest.raises(TypeError):        # a scale with a bf16 output
        mas.attention.trtllm_batch_decode_with_kv_cache(*args, out=torch.empty(batch, hq, dim, dtype=torch.bfloat16,
                                                                               device=dev), out_quant_scale=0.5)
    with pytest.raises(ValueError):
        mas.attention.trtllm_batch_decode_with_kv_cache(*args, out_quant_scale=0.0)
    with pytest.raises(ValueError):
        mas.attention.trtllm_batch_decode_with_kv_cache(*args, out_quant_scale=torch.ones(2, device=dev))


def _random_config(seed):
    """A seeded mix: 1-40 rows of 0-3000 positions, group sizes 1-16, head_dim 64 / 128 / 256, pages
    of 4-512 slots, the reference's workspace or a small one (longer splits), block tables as wide
    as the rows or 4-32 times wider."""
    rng = np.random.default_rng(seed)
    batch = int(rng.choice([1, 2, 5, 16, 40]))
    lens = [int(rng.integers(0, 3001)) for _ in range(batch)]
    hk = int(rng.choice([1, 2, 8]))
    group = int(rng.choice([1, 2, 3, 4, 6, 8, 12, 16]))
    dim = int(rng.choice([64, 128, 256]))
    ps = int(rng.choice([4, 16, 64, 256, 512]))
    widen = int(rng.choice([1, 1, 4, 32]))  # a block table 4 or 32 times wider than the rows need
    return batch, hk * group, hk, dim, ps, lens, widen


@pytest.mark.parametrize("seed", range(30))
def test_decode_attention_random_configs(mas, dev, seed):
    batch, hq, hk, dim, ps, lens, widen = _random_config(seed)
    q, kc, vc, tables, seq = _case(200 + seed, batch, hq, hk, dim, ps, lens)
    if widen > 1:   # padding columns hold out-of-range page ids
        wide = torch.full((tables.shape[0], tables.shape[1] * widen), -7, dtype=torch.int32)
        wide[:, : tables.shape[1]] = tables
        tables = wide
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    full = mas.attention.decode_workspace_bytes(batch, hq, dim, tables.shape[1], ps, 1)
    ws = full if seed % 3 else max(16, full // 4)
    out = _run(mas, dev, q, kc, vc, tables, seq, dim ** -0.5, workspace_bytes=ws, flags=flags)
    assert int(flags.item()) == 0
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), dim ** -0.5)
    _check(bits(out), want)


def test_decode_attention_peaked_scores(mas, dev):
    """Scores spread over hundreds of units (q ~ N(0, 9), scale 1): nearly one-hot softmax rows whose
    running max moves often, over single- and multi-split rows."""
    q, kc, vc, tables, seq = _case(43, 4, 32, 8, 128, 16, [3000, 200, 17, 1])
    q = (q.float() * 3.0).bfloat16()
    out = _run(mas, dev, q, kc, vc, tables, seq, 1.0)
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), 1.0)
    _check(bits(out), want)


@pytest.mark.parametrize("reach,ps", [(32768, 16), (131072, 16), (32768, 256)])
def test_decode_attention_block_table_wider_than_rows(mas, dev, reach, ps):
    """A block table as wide as a graph captured for the longest context (the reference captures
    its decode graphs with max_blocks columns) over rows far shorter: each row still gets short
    splits; results match the oracle, and no padding column is read as a page."""
    lens = [1, 300, 2000, 777, 4096, 60, 1500, 9]
    q, kc, vc, tables, seq = _case(47 + ps, len(lens), 32, 8, 128, ps, lens)
    wide = torch.full((len(lens), reach // ps), -7, dtype=torch.int32)   # out-of-range page ids
    wide[:, : tables.shape[1]] = tables
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, wide, seq, 0.088, flags=flags)
    assert int(flags.item()) == 0
    want = ops.paged_decode_attention(bits(q), bits(kc), bits(vc), wide.numpy(), seq.numpy(), 0.088)
    _check(bits(out), want)
