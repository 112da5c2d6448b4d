"""Causal paged context attention (trtllm_batch_context_with_kv_cache, devstral2.py:198-213) on the
GPU against the oracle, through the C ABI: bf16 outputs within rtol 1.6e-2 / atol 1e-2 (P enters the
P.V product as bf16, as in flash-attention kernels, so fewer outputs are bit-identical than for the
other ops)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import ATOL, RTOL, bits
from oracle import numerics as on
from oracle import ops

pytestmark = pytest.mark.gpu


def _case(seed, q_lens, kv_lens, hq, hk, dim, page_size):
    g = torch.Generator().manual_seed(seed)
    tokens = sum(q_lens)
    width = max(1, max(-(-n // page_size) for n in kv_lens))
    pages = len(kv_lens) * width + 2
    q = torch.randn(tokens, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, page_size, hk, dim, generator=g).bfloat16()
    tables = torch.randperm(pages, generator=g)[: len(kv_lens) * width].reshape(len(kv_lens), width).to(torch.int32)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    return q, kc, vc, tables, torch.tensor(kv_lens, dtype=torch.int32), cu


def _workspace(dev, nbytes):
    """A workspace whose bytes are all 0xff (NaN as float32): its contents on entry must not matter."""
    return torch.full((nbytes,), 255, dtype=torch.uint8, device=dev)


SPLIT_WS = 256 << 20  # holds the partials of every split case below


def _run(mas, dev, q, kc, vc, tables, seq, cu, scale, out=None, flags=None, scale2=1.0, ws_bytes=16, max_kv=0,
         quant=None):
    ws = _workspace(dev, ws_bytes)
    max_q = int((cu[1:] - cu[:-1]).max()) if len(cu) > 1 else 0
    return mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev) if q.device.type == "cpu" else q, (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev),
        max_q, max_kv, scale, scale2, len(cu) - 1, cu.to(dev), None, out=out, kv_layout="NHD", error_flags=flags,
        out_quant_scale=quant)


def _check(got, want, min_exact=0.55):
    """Within tolerance of the oracle, and at least `min_exact` of the outputs bit-identical. The
    kernel rounds P to bf16 against a lazy running max (moved only when a row's max rises by more
    than 2^8 in p), so the largest p of a row is rounded too: 58-73% of the outputs of the cases
    checked at the default share match the exact-max oracle bit for bit (60-73% with the max moved
    on every rise)."""
    np.testing.assert_allclose(on.bf16_to_f32(got), on.bf16_to_f32(want), rtol=RTOL, atol=ATOL)
    assert np.mean(got == want) >= min_exact


CASES = [
    ([100, 37], [100, 37], 32, 8, 128, 16),        # plain prefill, Devstral-Small-2 heads
    ([64, 1, 9], [300, 77, 9], 32, 8, 128, 256),   # chunked prefill: new tokens after cached ones
    ([70, 20], [70, 150], 96, 8, 128, 64),         # the 123B head group (12 per kv head)
    ([40], [140], 8, 8, 128, 16),                  # one head per kv head
    ([33, 90], [33, 95], 16, 8, 64, 32),           # 2 per kv head, head_dim 64
    ([17, 5], [50, 5], 6, 2, 64, 4),               # 3 per kv head, pages of 4
    ([200], [200], 8, 1, 128, 128),                # 8 per kv head, a longer row
    ([130, 64], [600, 64], 16, 4, 128, 512),       # pages of eight tiles, chunked prefill
    ([20, 0, 7], [30, 10, 7], 8, 2, 128, 64),      # a row with no new tokens between two others
    ([45, 19], [80, 19], 16, 2, 64, 16),           # 8 per kv head (eight-wavefront groups), head_dim 64, small pages
    ([70, 33], [90, 33], 24, 2, 128, 32),          # 12 per kv head, pages smaller than a tile
    ([50, 23], [75, 23], 32, 8, 128, 8),           # pages of 8 slots: eight pages per tile by LDS DMA
    ([60, 31], [99, 40], 96, 8, 128, 16),          # 16-slot pages, eight wavefronts (123B group)
    ([41], [77], 8, 4, 64, 16),                    # 16-slot pages, head_dim 64
    ([90, 17], [150, 17], 16, 8, 64, 64),          # head_dim 64 on pages of one tile
    ([70], [200], 32, 8, 64, 128),                 # head_dim 64 on pages of two tiles
]


@pytest.mark.parametrize("q_lens,kv_lens,hq,hk,dim,page_size", CASES)
def test_context_attention_matches_oracle(mas, dev, q_lens, kv_lens, hq, hk, dim, page_size):
    q, kc, vc, tables, seq, cu = _case(sum(kv_lens) + hq, q_lens, kv_lens, hq, hk, dim, page_size)
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, scale, flags=flags)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), scale)
    _check(bits(out), want)
    assert int(flags.item()) == 0


@pytest.mark.parametrize("page_size,kv0,ws_bytes", [(16, 120, 16), (256, 120, 16), (16, 2000, SPLIT_WS)])
def test_context_attention_hnd_layout(mas, dev, page_size, kv0, ws_bytes):
    """kv_layout="HND" ([pages, kv_heads, page_size, head_dim]): the same results as NHD (the last
    case under split-KV)."""
    q_lens, kv_lens, hq, hk, dim = [50, 9], [kv0, 9], 32, 8, 128
    q, kc, vc, tables, seq, cu = _case(31 + page_size, q_lens, kv_lens, hq, hk, dim, page_size)
    kh, vh = kc.transpose(1, 2).contiguous().to(dev), vc.transpose(1, 2).contiguous().to(dev)
    ws = _workspace(dev, ws_bytes)
    out = mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kh, vh), ws, tables.to(dev), seq.to(dev), max(q_lens), kv0, 0.09, 1.0, len(q_lens), cu.to(dev),
        None, kv_layout="HND")
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.09)
    _check(bits(out), want)


def test_context_attention_strided_views_and_bmm2_scale(mas, dev):
    """query as the column view of the qkv rows, out as a strided view, bmm2_scale applied."""
    q_lens, kv_lens, hq, hk, dim, ps = [48, 30], [60, 30], 32, 8, 128, 16
    _, kc, vc, tables, seq, cu = _case(3, q_lens, kv_lens, hq, hk, dim, ps)
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(sum(q_lens), (hq + 2 * hk) * dim, generator=g).bfloat16().to(dev)
    q = qkv[:, : hq * dim].view(-1, hq, dim)
    out_base = torch.full((sum(q_lens), hq + 2, dim), 5.0, dtype=torch.bfloat16, device=dev)
    out = out_base[:, 1:hq + 1]
    _run(mas, dev, q, kc, vc, tables, seq, cu, 0.07, out=out, scale2=2.0)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.07, 2.0)
    _check(bits(out), want)
    assert torch.all(out_base[:, 0] == 5.0) and torch.all(out_base[:, hq + 1] == 5.0)


@pytest.mark.parametrize("ps", [8, 16, 32])   # head_dim 64, four wavefronts: each page by LDS DMA, 8, 4 or 2 per tile
def test_context_attention_error_paths(mas, dev, ps):
    q_lens, kv_lens, hq, hk, dim = [20, 10], [40, 10], 8, 2, 64
    q, kc, vc, tables, _, cu = _case(8, q_lens, kv_lens, hq, hk, dim, ps)
    seq = torch.tensor([40, 4], dtype=torch.int32)       # row 1: kv_len 4 < q_len 10
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.1, flags=flags)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    _check(bits(out), want)
    assert not out[20:26].any()                           # the tokens before position 0 get zeros
    bad = tables.clone()
    bad[0, 16 // ps] = kc.shape[0] + 3                    # the page of row 0's position 16 points past the cache
    flags.zero_()
    _run(mas, dev, q, kc, vc, bad, torch.tensor([40, 10], dtype=torch.int32), cu, 0.1, flags=flags)
    assert int(flags.item()) == 8


def test_context_attention_max_q_len_too_small_is_flagged(mas, dev):
    """max_q_len sizes the grid: a row with more query tokens than it covers gets its covered tokens
    right, leaves the rest unwritten and sets error bit 2."""
    q_lens, kv_lens, hq, hk, dim, ps = [40, 10], [40, 10], 8, 2, 128, 16
    q, kc, vc, tables, seq, cu = _case(13, q_lens, kv_lens, hq, hk, dim, ps)
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev), 20, 0, 0.1, 1.0, 2, cu.to(dev), None,
        out=out, kv_layout="NHD", error_flags=flags)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    covered = [t for t in range(50) if not 32 <= t < 40]       # 32 tokens per grid tile (4 heads per kv head)
    _check(bits(out)[covered], want[covered])
    assert torch.all(out[32:40] == 7.0)


@pytest.mark.parametrize("kv0,ws_bytes", [(256, 16), (2048, SPLIT_WS)])  # one kernel; split-KV and its merge
def test_context_attention_in_graph_replays(mas, dev, kv0, ws_bytes):
    q_lens, kv_lens, hq, hk, dim, ps = [128, 64], [kv0, 64], 32, 8, 128, 64
    q, kc, vc, tables, seq, cu = _case(12, q_lens, kv_lens, hq, hk, dim, ps)
    qd, kd, vd, td, sd, cd = q.to(dev), kc.to(dev), vc.to(dev), tables.to(dev), seq.to(dev), cu.to(dev)
    ws = _workspace(dev, ws_bytes)
    out = torch.empty_like(qd)

    def call():
        mas.attention.trtllm_batch_context_with_kv_cache(qd, (kd, vd), ws, td, sd, 128, kv0, 0.088, 1.0, 2, cd,
                                                         None, out=out)

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
    if ws_bytes > 16:
        got = bits(want)
        ref = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.088)
        _check(got, ref)


@pytest.mark.parametrize("dim,hq,hk,scale_kind", [(128, 32, 8, "tensor"), (64, 6, 2, "float")])
def test_context_attention_fp8_output_is_the_o_proj_quantize(mas, dev, dim, hq, hk, scale_kind):
    """With out_quant_scale the kernel writes fp8(clamp(bf16(O) / scale, -448, 448)): bit for bit the
    o_proj input quantize (devstral2.py:93-95,110-111) of its own bf16 output."""
    q_lens, kv_lens, ps = [70, 3], [90, 3], 16
    q, kc, vc, tables, seq, cu = _case(dim + hq, q_lens, kv_lens, hq, hk, dim, ps)
    ref = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.2, scale2=4.0)
    ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    for s in (0.004, 0.37):
        scale = torch.tensor(s, dtype=torch.float32, device=dev) if scale_kind == "tensor" else s
        out = mas.attention.trtllm_batch_context_with_kv_cache(
            q.to(dev), (kc.to(dev), vc.to(dev)), ws, tables.to(dev), seq.to(dev), max(q_lens), 0, 0.2, 4.0,
            len(q_lens), cu.to(dev), None, kv_layout="NHD", out_quant_scale=scale)
        assert out.dtype == torch.float8_e4m3fn and tuple(out.shape) == tuple(q.shape)
        codes = out.view(torch.uint8).cpu().numpy()
        np.testing.assert_array_equal(codes, ops.quantize_activation(bits(ref), s))
        torch_q = (ref.float() / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        assert torch.equal(out.view(torch.uint8), torch_q.view(torch.uint8))
    assert np.mean(np.abs(on.bf16_to_f32(bits(ref))) / 0.004 > 448.0) > 0.01


def test_context_attention_short_row_position_error_is_flagged(mas, dev):
    """A bad seq_len on a row with fewer query tokens than max_q_len (its later token tiles are
    empty) is still flagged: tile 0's workgroup reports it."""
    q_lens, kv_lens, hq, hk, dim, ps = [70, 10], [70, 10], 8, 2, 128, 16   # 3 token tiles of 32
    q, kc, vc, tables, _, cu = _case(21, q_lens, kv_lens, hq, hk, dim, ps)
    for row1 in (4, 10_000):                       # below q_len, past the block table's reach
        seq = torch.tensor([70, row1], dtype=torch.int32)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        out = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.1, flags=flags)
        assert int(flags.item()) == 2, row1
        clamped = torch.tensor([70, min(row1, tables.shape[1] * ps)], dtype=torch.int32)
        want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), clamped.numpy(), cu.numpy(),
                                           0.1)
        _check(bits(out), want)


# Split-KV (few new tokens after a long cached prefix: a grid smaller than one round of resident
# workgroups, and a workspace): each token tile's keys are split over several workgroups and
# merged by a second kernel. The split result differs from the one-kernel result in rounding
# only, so the two are not bit-identical: that inequality shows the split path ran.
SPLIT_CASES = [
    # q_lens, kv_lens, hq, hk, dim, page_size, max_kv_len
    ([128], [4224], 32, 8, 128, 16, 4224),                # 128 new tokens after 4096 cached, Devstral-Small-2 heads
    ([64, 1, 9], [3000, 777, 9], 96, 8, 128, 256, 3000),  # the 123B head group, ragged rows
    ([33], [1500], 16, 8, 64, 32, 1500),                  # head_dim 64, two heads per kv head
    ([20, 7], [2000, 7], 24, 2, 128, 8, 2000),            # per-lane pages (8 slots), eight wavefronts
    ([40], [2500], 8, 8, 128, 64, 0),                     # no max_kv_len: splits over the block table's reach
    ([40], [2500], 8, 8, 128, 64, 1024),                  # max_kv_len below the real length: the last split takes the rest
    ([96], [1200], 32, 8, 128, 128, 1200),                # pages of two tiles, three token tiles of 32
    ([50], [2600], 16, 8, 64, 128, 2600),                 # head_dim 64 on pages of two tiles
    ([32], [16400], 32, 8, 128, 16, 16400),               # 32 new tokens after 16368 cached: more than 16 splits
]


@pytest.mark.parametrize("q_lens,kv_lens,hq,hk,dim,page_size,max_kv", SPLIT_CASES)
def test_context_attention_split_kv_matches_oracle(mas, dev, q_lens, kv_lens, hq, hk, dim, page_size, max_kv):
    q, kc, vc, tables, seq, cu = _case(sum(kv_lens) + 7 * hq, q_lens, kv_lens, hq, hk, dim, page_size)
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, scale, flags=flags, ws_bytes=SPLIT_WS, max_kv=max_kv)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), scale)
    one_kernel = _run(mas, dev, q, kc, vc, tables, seq, cu, scale, max_kv=max_kv)
    assert not torch.equal(out, one_kernel)
    # Over thousands of positions the outputs are small averages and P's bf16 rounding leaves fewer
    # of them bit-identical to the oracle: the split result must match as often as the one-kernel
    # result does, less 2 points.
    exact = np.mean(bits(out) == want)
    exact_one = np.mean(bits(one_kernel) == want)
    assert exact >= min(0.6, exact_one - 0.02), (exact, exact_one)
    _check(bits(out), want, min_exact=0.0)
    _check(bits(one_kernel), want, min_exact=0.0)


def test_context_attention_split_kv_small_workspace(mas, dev):
    """A workspace too small for the grid's 10 splits' partials gets fewer (here 3): still the oracle's
    result; one too small for 2 gets the one-kernel result, bit for bit."""
    q_lens, kv_lens, hq, hk, dim, ps = [32], [3000], 8, 8, 128, 16
    q, kc, vc, tables, seq, cu = _case(5, q_lens, kv_lens, hq, hk, dim, ps)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.09)
    one_kernel = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.09, max_kv=3000)
    per_split = 128 * hq * (dim + 2) * 4   # one token tile (one head per kv head: 4 wavefronts x 32 tokens)
    three = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.09, ws_bytes=3 * per_split + 100, max_kv=3000)
    _check(bits(three), want)
    assert not torch.equal(three, one_kernel)
    full = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.09, ws_bytes=SPLIT_WS, max_kv=3000)
    assert not torch.equal(three, full)                   # 3 splits, not 16
    tiny = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.09, ws_bytes=2 * per_split - 16, max_kv=3000)
    assert torch.equal(tiny, one_kernel)
    # context_workspace_bytes: enough for the most splits any grid takes (32; this one takes 10)
    need = mas.attention.context_workspace_bytes(1, 32, hq, hk, dim)
    assert need == 32 * per_split
    exact = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.09, ws_bytes=need, max_kv=3000)
    assert torch.equal(exact, full)


@pytest.mark.parametrize("ps", [8, 64])
def test_context_attention_split_kv_error_paths(mas, dev, ps):
    """Under split-KV: a row with kv_len < q_len (flag 2, zeros before position 0) and a page id past
    the cache in a late split (flag 8, its positions skipped as the oracle skips them)."""
    q_lens, kv_lens, hq, hk, dim = [20, 10], [2000, 10], 8, 2, 64
    q, kc, vc, tables, _, cu = _case(9, q_lens, kv_lens, hq, hk, dim, ps)
    seq = torch.tensor([2000, 4], dtype=torch.int32)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.1, flags=flags, ws_bytes=SPLIT_WS, max_kv=2000)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    _check(bits(out), want)
    assert not out[20:26].any()
    bad = tables.clone()
    bad[0, 1500 // ps] = kc.shape[0] + 3                  # the page of row 0's position 1500
    flags.zero_()
    _run(mas, dev, q, kc, vc, bad, torch.tensor([2000, 10], dtype=torch.int32), cu, 0.1, flags=flags,
         ws_bytes=SPLIT_WS, max_kv=2000)
    assert int(flags.item()) == 8


def test_context_attention_split_kv_empty_row_and_short_grid(mas, dev):
    """Under split-KV: a row whose seq_len is 0 (every split empty: zeros, flag 2), and max_q_len
    below a row's query count (its tokens past the grid left unwritten, flag 2)."""
    q_lens, kv_lens, hq, hk, dim, ps = [40, 8], [2000, 8], 32, 8, 128, 16
    q, kc, vc, tables, _, cu = _case(17, q_lens, kv_lens, hq, hk, dim, ps)
    seq = torch.tensor([2000, 0], dtype=torch.int32)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.1, flags=flags, ws_bytes=SPLIT_WS, max_kv=2000)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    _check(bits(out), want, min_exact=0.5)
    assert not out[40:].any()
    # max_q_len 32 covers one 32-token tile of row 0's 40 tokens
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=dev)
    flags.zero_()
    seq = torch.tensor([2000, 8], dtype=torch.int32)
    mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kc.to(dev), vc.to(dev)), _workspace(dev, SPLIT_WS), tables.to(dev), seq.to(dev), 32, 2000, 0.1,
        1.0, 2, cu.to(dev), None, out=out, kv_layout="NHD", error_flags=flags)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    covered = [t for t in range(48) if not 32 <= t < 40]
    _check(bits(out)[covered], want[covered], min_exact=0.0)
    assert torch.all(out[32:40] == 7.0)


@pytest.mark.parametrize("dim,hq,hk", [(128, 32, 8), (64, 6, 2)])
def test_context_attention_split_kv_fp8_output(mas, dev, dim, hq, hk):
    """The merge kernel's fp8 output is the o_proj input quantize of its own bf16 output, bit for bit."""
    q_lens, kv_lens, ps = [40, 3], [1800, 3], 16
    q, kc, vc, tables, seq, cu = _case(dim + 3 * hq, q_lens, kv_lens, hq, hk, dim, ps)
    ref = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.2, scale2=4.0, ws_bytes=SPLIT_WS, max_kv=1800)
    for s in (0.004, 0.37):
        out = _run(mas, dev, q, kc, vc, tables, seq, cu, 0.2, scale2=4.0, ws_bytes=SPLIT_WS, max_kv=1800,
                   quant=torch.tensor(s, dtype=torch.float32, device=dev))
        assert out.dtype == torch.float8_e4m3fn
        np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), ops.quantize_activation(bits(ref), s))


def _random_config(seed):
    """A seeded mix: 1-3 rows of 1-96 new tokens after 0-2900 cached positions (some rows without
    new tokens), group sizes 1-12, head_dim 64 / 128, pages of 4-256 slots (every block-table read
    mode: per lane, LDS DMA by page at 8 / 16 / 32 slots, and by tile), with and without a
    split-KV workspace and max_kv_len, block tables as wide as the rows or 4-32 times wider."""
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 4))
    q_lens = [int(rng.integers(0 if r else 1, 97)) for r in range(rows)]
    kv_lens = [q + int(rng.choice([0, rng.integers(1, 2900)])) for q in q_lens]
    hk = int(rng.choice([1, 2, 8]))
    group = int(rng.choice([1, 2, 3, 4, 8, 12]))
    dim = int(rng.choice([64, 128]))
    ps = int(rng.choice([4, 8, 16, 32, 64, 256]))
    ws = int(rng.choice([16, SPLIT_WS]))
    max_kv = int(rng.choice([0, max(kv_lens)]))
    widen = int(rng.choice([1, 1, 4, 32]))  # a block table 4 or 32 times wider than the rows need
    return q_lens, kv_lens, hk * group, hk, dim, ps, ws, max_kv, widen


@pytest.mark.parametrize("seed", range(64))
def test_context_attention_random_configs(mas, dev, seed):
    q_lens, kv_lens, hq, hk, dim, ps, ws, max_kv, widen = _random_config(seed)
    q, kc, vc, tables, seq, cu = _case(100 + seed, q_lens, kv_lens, hq, hk, dim, ps)
    if widen > 1:   # padding columns hold out-of-range page ids; max_kv_len then is the table's reach
        wide = torch.full((tables.shape[0], tables.shape[1] * widen), -7, dtype=torch.int32)
        wide[:, : tables.shape[1]] = tables
        tables = wide
        max_kv = tables.shape[1] * ps if max_kv else 0
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, dim ** -0.5, flags=flags, ws_bytes=ws, max_kv=max_kv)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(),
                                       dim ** -0.5)
    _check(bits(out), want, min_exact=0.5)


def test_context_attention_medium_grid_stays_one_kernel(mas, dev):
    """Many short rows (24 rows of 32 new tokens after 512 cached: 192 workgroups on MI355X's 256
    CUs) are not split even with a workspace: the merge would cost more than the split saves, so
    the result is the one-kernel result, bit for bit."""
    rows, q_len, cached, hq, hk, dim, ps = 24, 32, 512, 32, 8, 128, 16
    q, kc, vc, tables, seq, cu = _case(23, [q_len] * rows, [q_len + cached] * rows, hq, hk, dim, ps)
    one_kernel = _run(mas, dev, q, kc, vc, tables, seq, cu, dim ** -0.5, max_kv=q_len + cached)
    with_ws = _run(mas, dev, q, kc, vc, tables, seq, cu, dim ** -0.5, ws_bytes=SPLIT_WS, max_kv=q_len + cached)
    assert torch.equal(one_kernel, with_ws)


@pytest.mark.parametrize("ws_bytes", [16, SPLIT_WS])
def test_context_attention_peaked_scores(mas, dev, ws_bytes):
    """Scores spread over hundreds of units (q ~ N(0, 9), scale 1): each row's softmax is nearly
    one-hot and its running max moves often; one kernel and split-KV both match the oracle."""
    q_lens, kv_lens, hq, hk, dim, ps = [40, 7], [1500, 7], 16, 4, 128, 16
    q, kc, vc, tables, seq, cu = _case(41, q_lens, kv_lens, hq, hk, dim, ps)
    q = (q.float() * 3.0).bfloat16()
    out = _run(mas, dev, q, kc, vc, tables, seq, cu, 1.0, ws_bytes=ws_bytes, max_kv=1500)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 1.0)
    _check(bits(out), want, min_exact=0.5)


@pytest.mark.parametrize("reach", [32768, 131072])
def test_context_attention_block_table_wider_than_rows(mas, dev, reach):
    """The reference passes max_kv_len = the block table's reach (devstral2.py:296), which in a graph
    captured for the longest context far exceeds the rows: each token tile still divides its own
    positions among the splits; results match the oracle and no padding column is read as a page."""
    q_lens, kv_lens, hq, hk, dim, ps = [128, 20], [4224, 900], 32, 8, 128, 16
    q, kc, vc, tables, seq, cu = _case(53, q_lens, kv_lens, hq, hk, dim, ps)
    wide = torch.full((len(q_lens), reach // ps), -7, dtype=torch.int32)   # out-of-range page ids
    wide[:, : tables.shape[1]] = tables
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _run(mas, dev, q, kc, vc, wide, seq, cu, dim ** -0.5, flags=flags, ws_bytes=SPLIT_WS, max_kv=reach)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), wide.numpy(), seq.numpy(), cu.numpy(),
                                       dim ** -0.5)
    _check(bits(out), want, min_exact=0.5)
