"""The ops inside HIP graphs and torch.compile, the two ways the reference's model runner executes
its forward (miniagentserve/engine/model_runner.py:98,101-119)."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer_pass(mas, li, out_silu):
    """The reference's per-layer order for the five kernels: norm, rope, kv store, norm, silu."""
    s = li.shape
    mas.fused_add_rmsnorm(li.hidden, li.residual, li.norm_weight, s.eps)
    mas.apply_rope_with_cos_sin_cache_inplace(li.positions, li.q, li.k, s.head_dim, li.table, True)
    k = li.k.view(s.tokens, s.kv_heads, s.head_dim)
    v = li.v.view(s.tokens, s.kv_heads, s.head_dim)
    mas.append_paged_kv_cache(k, v, li.batch_indices, li.positions, (li.k_cache, li.v_cache),
                              li.block_tables.flatten(), li.kv_indptr, None, "NHD")
    mas.fused_add_rmsnorm(li.hidden, li.residual, li.norm_weight, s.eps)
    mas.silu_and_mul(li.gate_up, out=out_silu)


def _snapshot(li, out):
    return [t.clone() for t in (li.hidden, li.residual, li.qkv, li.k_cache, li.v_cache, out)]


def test_graph_replays_match_eager(mas, dev):
    wl = mas.workloads
    shape = wl.SHAPES["decode64_24b"]
    base = wl.make_layer_inputs(shape, dev, seed=3)
    originals = _snapshot(base, torch.empty(0))[:3]

    def reset(li):
        li.hidden.copy_(originals[0])
        li.residual.copy_(originals[1])
        li.qkv.copy_(originals[2])
        li.k_cache.zero_()
        li.v_cache.zero_()

    out = torch.empty(shape.tokens, shape.inter, dtype=torch.bfloat16, device=dev)
    _layer_pass(mas, base, out)
    torch.cuda.synchronize()
    want = _snapshot(base, out)

    reset(base)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _layer_pass(mas, base, out)            # warm-up on a side stream, as the runner does
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    reset(base)
    with torch.cuda.graph(graph):
        _layer_pass(mas, base, out)
    for _ in range(3):
        reset(base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = _snapshot(base, out)
        for a, b in zip(got, want):
            assert torch.equal(a, b)


def test_torch_compile_matches_eager(mas, dev):
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(37, 1024, generator=g, device=dev).bfloat16()
    r = torch.randn(37, 1024, generator=g, device=dev).bfloat16()
    w = (1 + 0.1 * torch.randn(1024, generator=g, device=dev)).bfloat16()
    gu = torch.randn(37, 2 * 512, generator=g, device=dev).bfloat16()
    scale = torch.tensor(0.05, device=dev)

    def f(x, r, gu):
        mas.fused_add_rmsnorm(x, r, w, 1e-5)
        out8 = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
        mas.fused_add_rmsnorm_quant(out8, x, r, w, scale, 1e-5)
        return x + 0, r + 0, out8.view(torch.uint8) + 0, mas.silu_and_mul(gu) * 2

    want = f(x.clone(), r.clone(), gu)
    compiled = torch.compile(f, dynamic=True, fullgraph=True)
    got = compiled(x.clone(), r.clone(), gu)
    for a, b in zip(got, want):
        assert torch.equal(a, b)


@pytest.mark.parametrize("fp8", [False, True])
def test_layer_pass_fused_and_separate_agree(mas, dev, fp8):
    """One layer with RoPE + KV fused or as the reference's two calls: bit-identical results."""
    wl, lp = mas.workloads, mas.layer_pass
    outs = []
    for fuse in (True, False):
        li = wl.make_layer_inputs("decode64_24b", dev, seed=9)
        b = lp.LayerBuffers(li, fp8=fp8, fuse_rope_kv=fuse)
        lp.run_layer(b)
        torch.cuda.synchronize()
        tensors = [li.hidden, li.residual, li.attn_out, li.qkv, li.k_cache, li.v_cache, b.silu_out]
        if fp8:
            tensors.append(b.norm_out)
        outs.append([t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t for t in tensors])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    if fp8:
        # SiluAndMul's fp8 output is the quantize of its bf16 output
        li = wl.make_layer_inputs("decode64_24b", dev, seed=9, with_cache=False)
        y = mas.silu_and_mul(li.gate_up)
        ref = (y.float() / 0.05).clamp(-448, 448).to(torch.float8_e4m3fn)
        assert torch.equal(outs[0][6], ref.view(torch.uint8))


def test_torch_compile_attention_matches_eager(mas, dev):
    """Both attention ops, bf16 and fp8 outputs (device-tensor scale), through torch.compile's custom
    ops: the same bytes as eager (context attention with 40 new tokens after 1160 cached: split-KV
    in the workspace)."""
    g = torch.Generator(device=dev).manual_seed(8)
    pages, ps, hq, hk, d = 48, 64, 8, 2, 128
    kc = torch.randn(pages, ps, hk, d, generator=g, device=dev).bfloat16()
    vc = torch.randn(pages, ps, hk, d, generator=g, device=dev).bfloat16()
    tables = torch.randperm(pages, device=dev).reshape(2, 24).to(torch.int32)
    seq = torch.tensor([1200, 90], dtype=torch.int32, device=dev)
    qd = torch.randn(2, hq, d, generator=g, device=dev).bfloat16()
    cu = torch.tensor([0, 40, 70], dtype=torch.int32, device=dev)
    qc = torch.randn(70, hq, d, generator=g, device=dev).bfloat16()
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device=dev)
    scale = torch.tensor(0.02, device=dev)
    att = mas.attention

    def f(qd, qc):
        o1 = att.trtllm_batch_decode_with_kv_cache(qd, (kc, vc), ws, tables, seq, 1536, 0.09, 1.0)
        o2 = att.trtllm_batch_decode_with_kv_cache(qd, (kc, vc), ws, tables, seq, 1536, 0.09, 1.0,
                                                   out_quant_scale=scale)
        o3 = att.trtllm_batch_context_with_kv_cache(qc, (kc, vc), ws, tables, seq, 40, 1200, 0.09, 1.0, 2, cu)
        o4 = att.trtllm_batch_context_with_kv_cache(qc, (kc, vc), ws, tables, seq, 40, 1200, 0.09, 1.0, 2, cu,
                                                    out_quant_scale=0.02)
        return o1 + 0, o2.view(torch.uint8) + 0, o3 + 0, o4.view(torch.uint8) + 0

    want = f(qd, qc)
    compiled = torch.compile(f, dynamic=True, fullgraph=True)
    got = compiled(qd, qc)
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    small_ws = torch.zeros(16, dtype=torch.uint8, device=dev)
    one_kernel = att.trtllm_batch_context_with_kv_cache(qc, (kc, vc), small_ws, tables, seq, 40, 1200, 0.09, 1.0, 2, cu)
    assert not torch.equal(one_kernel, want[2])   # the split ran (its rounding differs)


def test_torch_compile_context_attention_keeps_lengths_symbolic(mas, dev):
    """max_q_len taken from a traced shape, as the reference derives it (devstral2.py:295), stays
    symbolic through the custom op: a second call with another token count runs the same compiled
    graph (no recompilation) and gives eager's bytes."""
    g = torch.Generator(device=dev).manual_seed(11)
    pages, ps, hq, hk, d = 16, 64, 8, 2, 128
    kc = torch.randn(pages, ps, hk, d, generator=g, device=dev).bfloat16()
    vc = torch.randn(pages, ps, hk, d, generator=g, device=dev).bfloat16()
    tables = torch.randperm(pages, device=dev).reshape(2, 8).to(torch.int32)
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device=dev)
    att = mas.attention

    def f(qc, cu, seq):
        return att.trtllm_batch_context_with_kv_cache(qc, (kc, vc), ws, tables, seq, qc.shape[0],
                                                      tables.shape[1] * ps, 0.09, 1.0, 2, cu) + 0

    compiled = torch.compile(f, dynamic=True, fullgraph=True)
    for n0 in (40, 57):
        qc = torch.randn(n0 + 30, hq, d, generator=g, device=dev).bfloat16()
        cu = torch.tensor([0, n0, n0 + 30], dtype=torch.int32, device=dev)
        seq = torch.tensor([n0 + 300, 30], dtype=torch.int32, device=dev)
        want = f(qc, cu, seq)
        with torch._dynamo.config.patch(error_on_recompile=n0 != 40):
            got = compiled(qc, cu, seq)
        assert torch.equal(got, want)
