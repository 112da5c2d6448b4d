"""Context attention in the layout of the reference's captured graphs (model_runner.py:155-221):
17 prompt rows, the real prompts first, then one padding row holding the step's padding tokens
(their kv_len = their count, every block-table entry the sink page) and empty rows (no query
tokens, seq_len 1); max_q_len = the step's prompt tokens (devstral2.py:295) and max_kv_len = the
block table's reach (devstral2.py:296), the table as wide as the longest context the graphs serve.
The host sees only those bounds, so the split-KV decision is made on the device (the planned
launch): results against the oracle within rtol 1.6e-2 / atol 1e-2, and bit-identical to the
one-kernel launch where no split pays."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import bits
from oracle import ops
from test_gpu_context_attention import _check, _workspace

pytestmark = pytest.mark.gpu

PREFILL_ROWS = 17
WS = 128 << 20  # the reference's workspace (devstral2.py:35)


def _graph_case(seed, prompts, pad_tokens, hq, hk, dim, ps, reach=32768, rows=PREFILL_ROWS):
    """prompts: (new tokens, cached positions) per real row. Returns q, caches (the last page is the
    sink), tables [rows, reach / ps] (columns past a row's pages hold an out-of-range id), seq_lens,
    cu_seqlens_q and max_q_len (all prompt tokens, padding included)."""
    g = torch.Generator().manual_seed(seed)
    width = reach // ps
    need = [-(-(n + c) // ps) for n, c in prompts]
    pages = sum(need) + 1
    sink = pages - 1
    perm = torch.randperm(pages - 1, generator=g).to(torch.int32)
    tables = torch.full((rows, width), -7, dtype=torch.int32)
    lens, cu, at = [], [0], 0
    for r, ((n, c), k) in enumerate(zip(prompts, need)):
        tables[r, :k] = perm[at:at + k]
        at += k
        lens.append(n + c)
        cu.append(cu[-1] + n)
    first = len(prompts)
    if first < rows:
        lens.append(max(pad_tokens, 1))
        cu.append(cu[-1] + pad_tokens)
        tables[first] = sink
        for _ in range(first + 1, rows):
            lens.append(1)
            cu.append(cu[-1])
        tables[first + 1:, 0] = sink
    tokens = cu[-1]
    q = torch.randn(tokens, hq, dim, generator=g).bfloat16()
    kc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16()
    vc = torch.randn(pages, ps, hk, dim, generator=g).bfloat16()
    return (q, kc, vc, tables, torch.tensor(lens, dtype=torch.int32), torch.tensor(cu, dtype=torch.int32), tokens)


def _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, ws_bytes=WS, flags=None, quant=None,
          layout="NHD"):
    kd, vd = kc.to(dev), vc.to(dev)
    if layout == "HND":
        kd, vd = kd.transpose(1, 2).contiguous(), vd.transpose(1, 2).contiguous()
    return mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kd, vd), _workspace(dev, ws_bytes), tables.to(dev), seq.to(dev), max_q, reach, scale, 1.0,
        len(cu) - 1, cu.to(dev), None, out_quant_scale=quant, kv_layout=layout, error_flags=flags)


PLANNED_CASES = [
    # prompts (new, cached), padding tokens, hq, hk, head_dim, page size
    ([(100, 4000)], 28, 32, 8, 128, 16),                      # an agent turn on Devstral-Small-2 heads (t = 128)
    ([(60, 3000)], 4, 96, 8, 128, 16),                        # the 123B head group (t = 64)
    ([(50, 2000), (30, 0), (40, 700)], 8, 32, 8, 128, 16),    # three prompts of mixed lengths
    ([(200, 1500)], 56, 16, 8, 64, 16),                       # head_dim 64, two heads per kv head
    ([(32, 16368)], 32, 32, 8, 128, 16),                      # more than 16 splits
    ([(90, 5000), (7, 9000)], 31, 32, 8, 128, 256),           # pages of four tiles
    ([(70, 2500), (130, 10)], 56, 24, 2, 128, 8),             # per-lane pages (8 slots), eight wavefronts
    ([(120, 900), (3, 3000), (1, 2)], 4, 32, 8, 128, 64),     # pages of one tile; one-token prompts
]


@pytest.mark.parametrize("prompts,pad,hq,hk,dim,ps", PLANNED_CASES)
def test_planned_context_attention_matches_oracle(mas, dev, prompts, pad, hq, hk, dim, ps):
    q, kc, vc, tables, seq, cu, max_q = _graph_case(sum(n for n, _ in prompts) + hq + ps, prompts, pad, hq, hk,
                                                    dim, ps)
    reach = tables.shape[1] * ps
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, flags=flags)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), scale)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, ws_bytes=16)
    assert not torch.equal(out, one_kernel)  # the plan split the long rows
    exact = np.mean(bits(out) == want)
    exact_one = np.mean(bits(one_kernel) == want)
    assert exact >= min(0.6, exact_one - 0.02), (exact, exact_one)
    _check(bits(out), want, min_exact=0.0)


@pytest.mark.parametrize("case", [0, 2, 3, 4, 6])
def test_self_planned_launch_equals_the_planner_launch(mas, dev, case):
    """A step of up to 64 rows lays its plan out in the kernels themselves (no planner launch); with
    more rows the planner launch writes it. From the same real rows both lay out the same plan, so
    the outputs match bit for bit: 17 rows against the same prompts padded to 70 rows (cases whose
    split counts stay within both grids, so the grid size does not change the plan)."""
    prompts, pad, hq, hk, dim, ps = PLANNED_CASES[case]
    seed = sum(n for n, _ in prompts) + hq + ps
    q, kc, vc, tables, seq, cu, max_q = _graph_case(seed, prompts, pad, hq, hk, dim, ps)
    q70, kc70, vc70, tables70, seq70, cu70, max_q70 = _graph_case(seed, prompts, pad, hq, hk, dim, ps, rows=70)
    assert torch.equal(q, q70) and torch.equal(kc, kc70) and max_q == max_q70
    reach = tables.shape[1] * ps
    scale = dim ** -0.5
    flags, flags70 = (torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(2))
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, flags=flags)
    out70 = _call(mas, dev, q70, kc70, vc70, tables70, seq70, cu70, max_q70, reach, scale, flags=flags70)
    assert int(flags.item()) == 0 and int(flags70.item()) == 0
    assert torch.equal(out, out70)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, ws_bytes=16)
    assert not torch.equal(out, one_kernel)  # the plan split the long rows


@pytest.mark.parametrize("n_prompts,cached", [(40, 3000), (24, 6000)], ids=["40_unsplit", "24_split"])
def test_self_planned_64_rows_equal_the_planner_on_65(mas, dev, n_prompts, cached):
    """The largest self-planned step (64 rows, a row per lane) against the same prompts on 65 rows,
    which the planner launch lays out, bit for bit: 40 one-tile prompts (320 workgroups, unsplit)
    and 24 after longer prefixes (split), so the per-row counts fill lanes across the wavefront's
    four 16-lane rows. The first three prompts also against the oracle."""
    g = torch.Generator().manual_seed(640 + n_prompts)
    prompts = [(int(torch.randint(1, 25, (1,), generator=g)), int(torch.randint(0, cached, (1,), generator=g)))
               for _ in range(n_prompts)]
    tokens = sum(n for n, _ in prompts)
    pad = -(-tokens // 64) * 64 - tokens
    q, kc, vc, tables, seq, cu, max_q = _graph_case(640, prompts, pad, 32, 8, 128, 16, rows=64)
    q65, kc65, vc65, tables65, seq65, cu65, max_q65 = _graph_case(640, prompts, pad, 32, 8, 128, 16, rows=65)
    assert torch.equal(q, q65) and torch.equal(kc, kc65) and max_q == max_q65
    reach = tables.shape[1] * 16
    flags, flags65 = (torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(2))
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.088, flags=flags)
    out65 = _call(mas, dev, q65, kc65, vc65, tables65, seq65, cu65, max_q65, reach, 0.088, flags=flags65)
    assert int(flags.item()) == 0 and int(flags65.item()) == 0
    assert torch.equal(out, out65)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.088, ws_bytes=16)
    if n_prompts == 40:
        assert torch.equal(out, one_kernel)      # unsplit: the grid launch's work
    else:
        assert not torch.equal(out, one_kernel)  # the plan split the long rows
    t3 = int(cu[3])
    want = ops.paged_context_attention(bits(q[:t3]), bits(kc), bits(vc), tables[:3].numpy(), seq[:3].numpy(),
                                       cu[:4].numpy(), 0.088)
    exact = np.mean(bits(out[:t3]) == want)
    exact_one = np.mean(bits(one_kernel[:t3]) == want)
    assert exact >= min(0.6, exact_one - 0.02), (exact, exact_one)
    _check(bits(out[:t3]), want, min_exact=0.0)


def test_planned_context_attention_short_rows_equal_one_kernel(mas, dev):
    """A step of short prompts: the plan splits nothing and its items are the one-kernel grid's
    workgroups, so the output is the one-kernel output bit for bit."""
    prompts = [(40, 10), (64, 0), (9, 30)]
    q, kc, vc, tables, seq, cu, max_q = _graph_case(61, prompts, 15, 32, 8, 128, 16)
    reach = tables.shape[1] * 16
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09, ws_bytes=16)
    assert torch.equal(out, one_kernel)
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.09)
    _check(bits(out), want)


@pytest.mark.parametrize("layout", ["HND"])
def test_planned_context_attention_hnd_layout(mas, dev, layout):
    prompts = [(80, 2200)]
    q, kc, vc, tables, seq, cu, max_q = _graph_case(67, prompts, 48, 32, 8, 128, 16)
    reach = tables.shape[1] * 16
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09, layout=layout)
    nhd = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09)
    assert torch.equal(out, nhd)


@pytest.mark.parametrize("dim,hq,hk", [(128, 32, 8), (64, 16, 8)])
def test_planned_context_attention_fp8_output(mas, dev, dim, hq, hk):
    """The planned merge's and split-free items' fp8 output is the o_proj input quantize of the bf16
    output, bit for bit."""
    prompts = [(70, 1800), (2, 5)]
    q, kc, vc, tables, seq, cu, max_q = _graph_case(71 + dim, prompts, 56, hq, hk, dim, 16)
    reach = tables.shape[1] * 16
    ref = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.2)
    for s in (0.004, 0.37):
        out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.2,
                    quant=torch.tensor(s, dtype=torch.float32, device=dev))
        assert out.dtype == torch.float8_e4m3fn
        np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), ops.quantize_activation(bits(ref), s))


def test_planned_context_attention_error_bits(mas, dev):
    """The planner reports a row whose kv_len is below its q_len (bit 2; its first tokens get zeros),
    and a page id past the cache inside a split's key range is reported by the split's workgroup
    (bit 8), its positions skipped as the oracle skips them."""
    prompts = [(40, 2000), (10, 0)]
    q, kc, vc, tables, seq, cu, max_q = _graph_case(73, prompts, 14, 32, 8, 128, 16)
    reach = tables.shape[1] * 16
    seq_bad = seq.clone()
    seq_bad[1] = 4
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _call(mas, dev, q, kc, vc, tables, seq_bad, cu, max_q, reach, 0.1, flags=flags)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq_bad.numpy(), cu.numpy(), 0.1)
    _check(bits(out), want, min_exact=0.5)
    assert not out[40:46].any()
    bad = tables.clone()
    bad[0, 1500 // 16] = kc.shape[0] + 3
    flags.zero_()
    _call(mas, dev, q, kc, vc, bad, seq, cu, max_q, reach, 0.1, flags=flags)
    assert int(flags.item()) == 8


def test_planned_context_attention_max_q_len_too_small(mas, dev):
    """A row with more query tokens than max_q_len's token tiles cover: flagged by the planner, its
    covered tokens right, the rest unwritten."""
    prompts = [(100, 3000)]
    q, kc, vc, tables, seq, cu, _ = _graph_case(79, prompts, 28, 32, 8, 128, 16)
    reach = tables.shape[1] * 16
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kc.to(dev), vc.to(dev)), _workspace(dev, WS), tables.to(dev), seq.to(dev), 64, reach, 0.1, 1.0,
        PREFILL_ROWS, cu.to(dev), None, out=out, error_flags=flags)
    assert int(flags.item()) == 2
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.1)
    covered = list(range(64)) + list(range(100, 128))
    _check(bits(out)[covered], want[covered], min_exact=0.0)
    assert torch.all(out[64:100] == 7.0)


def test_planned_context_attention_small_workspace(mas, dev):
    """A workspace that holds the plan but few partials gets fewer splits (still the oracle's result);
    one too small for the plan gets the one-kernel launch, bit for bit."""
    prompts = [(100, 4000)]
    q, kc, vc, tables, seq, cu, max_q = _graph_case(83, prompts, 28, 32, 8, 128, 16)
    reach = tables.shape[1] * 16
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), 0.09)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09, ws_bytes=16)
    full = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09)
    small = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09, ws_bytes=6 << 20)
    _check(bits(small), want, min_exact=0.0)
    assert not torch.equal(small, one_kernel) and not torch.equal(small, full)
    tiny = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, 0.09, ws_bytes=64 << 10)
    assert torch.equal(tiny, one_kernel)


def test_planned_context_attention_graph_replays_new_lengths(mas, dev):
    """One captured graph (fixed buffers, as the reference's graph inputs) replayed over steps whose
    prompts differ in count, length and cached prefix: the plan follows each step's lengths, and each
    replay equals the eager call on the same inputs, bit for bit, and the oracle."""
    hq, hk, dim, ps, reach, t = 32, 8, 128, 16, 32768, 128
    steps = [
        [(100, 4000)],
        [(20, 9000), (60, 100), (40, 0)],
        [(128, 0)],
        [(5, 20000), (3, 7000)],
    ]
    cases = []
    for i, prompts in enumerate(steps):
        used = sum(n for n, _ in prompts)
        cases.append(_graph_case(90 + i, prompts, t - used, hq, hk, dim, ps, reach=reach))
    pages = max(c[1].shape[0] for c in cases)
    kc = torch.randn(pages, ps, hk, dim, generator=torch.Generator().manual_seed(5)).bfloat16()
    vc = torch.randn(pages, ps, hk, dim, generator=torch.Generator().manual_seed(6)).bfloat16()
    kd, vd = kc.to(dev), vc.to(dev)
    qb = torch.zeros(t, hq, dim, dtype=torch.bfloat16, device=dev)
    tb = torch.zeros(PREFILL_ROWS, reach // ps, dtype=torch.int32, device=dev)
    sb = torch.zeros(PREFILL_ROWS, dtype=torch.int32, device=dev)
    cb = torch.zeros(PREFILL_ROWS + 1, dtype=torch.int32, device=dev)
    ws = _workspace(dev, WS)
    out = torch.empty_like(qb)

    def load(case):
        q, _, _, tables, seq, cu, _ = case
        tables = tables.clone()
        tables[tables == case[1].shape[0] - 1] = pages - 1   # every case's sink is the shared last page
        qb.copy_(q)
        tb.copy_(tables)
        sb.copy_(seq)
        cb.copy_(cu)
        return tables

    def call():
        mas.attention.trtllm_batch_context_with_kv_cache(qb, (kd, vd), ws, tb, sb, t, reach, dim ** -0.5, 1.0,
                                                         PREFILL_ROWS, cb, None, out=out)

    load(cases[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call()
    for rounds in range(2):
        for case in cases:
            tables = load(case)
            call()
            torch.cuda.synchronize()
            eager = out.clone()
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            if rounds == 0:
                q, _, _, _, seq, cu, _ = case
                want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(),
                                                   cu.numpy(), dim ** -0.5)
                _check(bits(out), want, min_exact=0.0)


def test_planned_context_attention_compiled_and_captured(mas, dev):
    """The way the reference runs its graph steps (model_runner.py:98-119): the call compiled with
    torch.compile(dynamic=True, fullgraph=True), max_q_len taken from the query's shape
    (devstral2.py:295), warmed up three times on a side stream and captured in a CUDA graph; replays
    over steps of different prompts equal the eager call bit for bit, and the long-prefix step splits
    (its result differs from the one-kernel launch's)."""
    hq, hk, dim, ps, reach, t = 32, 8, 128, 16, 8192, 128
    steps = [[(100, 4000)], [(60, 2000), (40, 10)], [(128, 0)]]
    cases = [_graph_case(110 + i, p, t - sum(n for n, _ in p), hq, hk, dim, ps, reach=reach) for i, p in enumerate(steps)]
    pages = max(c[1].shape[0] for c in cases)
    kc = torch.randn(pages, ps, hk, dim, generator=torch.Generator().manual_seed(7)).bfloat16().to(dev)
    vc = torch.randn(pages, ps, hk, dim, generator=torch.Generator().manual_seed(8)).bfloat16().to(dev)
    qb = torch.zeros(t, hq, dim, dtype=torch.bfloat16, device=dev)
    tb = torch.zeros(PREFILL_ROWS, reach // ps, dtype=torch.int32, device=dev)
    sb = torch.zeros(PREFILL_ROWS, dtype=torch.int32, device=dev)
    cb = torch.zeros(PREFILL_ROWS + 1, dtype=torch.int32, device=dev)
    ws = _workspace(dev, WS)
    att = mas.attention

    def f(q, tables, seq, cu):
        return att.trtllm_batch_context_with_kv_cache(q, (kc, vc), ws, tables, seq, q.shape[0], tables.shape[1] * ps,
                                                      dim ** -0.5, 1.0, cu.shape[0] - 1, cu)

    def load(case):
        q, _, _, tables, seq, cu, _ = case
        tables = tables.clone()
        tables[tables == case[1].shape[0] - 1] = pages - 1
        qb.copy_(q)
        tb.copy_(tables)
        sb.copy_(seq)
        cb.copy_(cu)

    compiled = torch.compile(f, dynamic=True, fullgraph=True)
    load(cases[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            compiled(qb, tb, sb, cb)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = compiled(qb, tb, sb, cb)
    for i, case in enumerate(cases):
        load(case)
        want = f(qb, tb, sb, cb)
        torch.cuda.synchronize()
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"step {i}"
        if i == 0:
            one_kernel = att.trtllm_batch_context_with_kv_cache(qb, (kc, vc), _workspace(dev, 16), tb, sb, t, reach,
                                                                dim ** -0.5, 1.0, PREFILL_ROWS, cb)
            assert not torch.equal(out, one_kernel)


@pytest.mark.parametrize("rows,prompts,hq,hk,dim", [
    (300, [(40, 3000), (5, 900), (2, 0)], 32, 8, 128),   # 300 prompt rows (the planner's row loop wraps)
    (17, [(70, 2600), (9, 40)], 12, 2, 128),               # 6 query heads per kv head: a half-empty head block
    (17, [(90, 3000), (150, 10)], 16, 2, 64),              # head_dim 64, 8 query heads per kv head (8 wavefronts)
])
def test_planned_context_attention_more_shapes(mas, dev, rows, prompts, hq, hk, dim):
    """Planned launches beyond the graph-step defaults: a step of hundreds of prompt rows, a head
    group that leaves part of a workgroup's heads empty, head_dim 64 with eight wavefronts; split
    (the result differs from the one-kernel launch's) and within the oracle's tolerance."""
    t = -(-sum(n for n, _ in prompts) // 64) * 64
    q, kc, vc, tables, seq, cu, max_q = _graph_case(rows + hq + dim, prompts, t - sum(n for n, _ in prompts), hq, hk,
                                                    dim, 16, rows=rows)
    reach = tables.shape[1] * 16
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, flags=flags)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), scale)
    one_kernel = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, reach, scale, ws_bytes=16)
    assert not torch.equal(out, one_kernel)
    _check(bits(out), want, min_exact=0.5)


def test_planned_context_attention_degenerate_steps(mas, dev):
    """Planned launches of degenerate steps give what the grid launch gives: a step whose rows have
    no query tokens writes nothing and flags nothing; a row whose seq_len is 0 gets zeros and the
    position bit; a row whose cum_seq_lens_q entries decrease (a negative count) is skipped."""
    hq, hk, dim, ps, t = 32, 8, 128, 16, 128
    q, kc, vc, tables, seq, cu, _ = _graph_case(131, [(100, 4000)], 28, hq, hk, dim, ps)
    reach = tables.shape[1] * ps
    # no query tokens in any row
    empty_cu = torch.zeros_like(cu)
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    mas.attention.trtllm_batch_context_with_kv_cache(
        q.to(dev), (kc.to(dev), vc.to(dev)), _workspace(dev, WS), tables.to(dev), seq.to(dev), t, reach, 0.1, 1.0,
        PREFILL_ROWS, empty_cu.to(dev), None, out=out, error_flags=flags)
    assert int(flags.item()) == 0 and torch.all(out == 7.0)
    # seq_len 0 for the long row; a decreasing entry for the padding row
    seq_bad = seq.clone()
    seq_bad[0] = 0
    cu_bad = cu.clone()
    cu_bad[2] = 90  # row 1 (padding) now has 90 - 100 < 0 tokens; row 2 starts at 90
    results = []
    for ws_bytes in (WS, 16):
        out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device=dev)
        flags = torch.zeros(1, dtype=torch.int32, device=dev)
        mas.attention.trtllm_batch_context_with_kv_cache(
            q.to(dev), (kc.to(dev), vc.to(dev)), _workspace(dev, ws_bytes), tables.to(dev), seq_bad.to(dev), t, reach,
            0.1, 1.0, PREFILL_ROWS, cu_bad.to(dev), None, out=out, error_flags=flags)
        results.append((int(flags.item()), out))
    assert results[0][0] == results[1][0] == 2
    assert torch.equal(results[0][1], results[1][1])
    assert not results[0][1][:100].any()


def _random_graph_step(seed):
    """A seeded graph step: 1-5 prompts of 1-120 new tokens after 0-9000 cached positions (the step's
    tokens rounded up to 64, at most 512, the rest a padding row), group sizes 1-12, head_dim 64 /
    128, pages of 8-256 slots, a table reach of 16384 positions."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 6))
    prompts = [(int(rng.integers(1, 121)), int(rng.choice([0, rng.integers(1, 9001)]))) for _ in range(n)]
    hk = int(rng.choice([2, 8]))
    group = int(rng.choice([1, 2, 3, 4, 6, 8, 12]))
    dim = int(rng.choice([64, 128]))
    ps = int(rng.choice([8, 16, 64, 256]))
    return prompts, hk * group, hk, dim, ps


@pytest.mark.parametrize("seed", range(20))
def test_planned_context_attention_random_steps(mas, dev, seed):
    prompts, hq, hk, dim, ps = _random_graph_step(seed)
    used = sum(n for n, _ in prompts)
    t = -(-used // 64) * 64
    q, kc, vc, tables, seq, cu, max_q = _graph_case(1000 + seed, prompts, t - used, hq, hk, dim, ps, reach=16384)
    scale = dim ** -0.5
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, 16384, scale, flags=flags)
    assert int(flags.item()) == 0
    want = ops.paged_context_attention(bits(q), bits(kc), bits(vc), tables.numpy(), seq.numpy(), cu.numpy(), scale)
    _check(bits(out), want, min_exact=0.5)


@pytest.mark.parametrize("seed", range(12))
def test_self_planned_random_steps_equal_the_planner(mas, dev, seed):
    """Seeded graph steps of 18-64 rows (self-planned) with 1-40 prompts of 1-60 new tokens after
    0-9000 cached positions (8 kv heads, group sizes 1-12, head_dim 64 / 128, pages of 8-256 slots),
    against the same prompts on 65 rows (the planner launch): the same output and error bits, bit for
    bit; and the first prompt against the oracle. Both launches are planned only when the grid holds
    a workgroup per CU or more (smaller grids take the host's split-KV), so the row count is raised
    to make the self-planned grid that large."""
    rng = np.random.default_rng(5000 + seed)
    rows = int(rng.integers(18, 65))
    n = int(rng.integers(1, min(rows - 1, 40) + 1))
    prompts = []
    for _ in range(n):
        new = int(rng.integers(1, 61))
        if sum(p for p, _ in prompts) + new > 900:   # planned steps cover at most 1024 tokens
            break
        prompts.append((new, int(rng.choice([0, rng.integers(1, 9001)]))))
    hk = 8
    group = int(rng.choice([1, 2, 3, 4, 6, 8, 12]))
    dim = int(rng.choice([64, 128]))
    ps = int(rng.choice([8, 16, 64, 256]))
    hq = hk * group
    used = sum(p for p, _ in prompts)
    pad = -(-used // 64) * 64 - used
    # the grid of the host's launch rules: 4 heads per workgroup from groups of 4 (2 for 2, else 1),
    # 8 wavefronts from groups of 8, 32 tokens per wavefront row
    per_wg = 4 if group >= 4 else (2 if group == 2 else 1)
    tokens_per_wg = 32 * ((8 if group >= 8 else 4) // per_wg)
    blocks = hk * -(-group // per_wg) * -(-(used + pad) // tokens_per_wg)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    rows = max(rows, -(-cus // blocks), len(prompts) + 1)
    assert rows <= 64
    q, kc, vc, tables, seq, cu, max_q = _graph_case(6000 + seed, prompts, pad, hq, hk, dim, ps, reach=16384,
                                                    rows=rows)
    q65, kc65, vc65, tables65, seq65, cu65, max_q65 = _graph_case(6000 + seed, prompts, pad, hq, hk, dim, ps,
                                                                  reach=16384, rows=65)
    assert torch.equal(q, q65) and torch.equal(kc, kc65) and max_q == max_q65
    scale = dim ** -0.5
    flags, flags65 = (torch.zeros(1, dtype=torch.int32, device=dev) for _ in range(2))
    out = _call(mas, dev, q, kc, vc, tables, seq, cu, max_q, 16384, scale, flags=flags)
    out65 = _call(mas, dev, q65, kc65, vc65, tables65, seq65, cu65, max_q65, 16384, scale, flags=flags65)
    assert int(flags.item()) == int(flags65.item()) == 0
    assert torch.equal(out, out65), (rows, prompts, hq, hk, dim, ps)
    t1 = int(cu[1])
    want = ops.paged_context_attention(bits(q[:t1]), bits(kc), bits(vc), tables[:1].numpy(), seq[:1].numpy(),
                                       cu[:2].numpy(), scale)
    _check(bits(out[:t1]), want, min_exact=0.5)
