#!/usr/bin/env python3
"""Benchmark of the MI355X layer kernels on the reference's layer-kernel workloads.

Default workload: one Devstral-Small-2 decoder layer at a 64-token decode step (hidden 5120,
intermediate 32768, 32 q / 8 kv heads of 128, KV pool 2048 pages x 256 slots). A step is that
layer's hot-path kernels over one 64-token batch - RMSNorm+residual, RoPE + paged KV store (one
fused kernel; the reference's two separate calls are timed alongside), RMSNorm+residual,
SiluAndMul. Inputs are resident in HBM before the timed region. The cold protocol (default)
cycles through enough distinct layer buffer sets (each with its own KV cache) that a step never
finds its data in the 256 MB Infinity Cache - what a 40-layer forward pass sees; steps are replayed
from a captured HIP graph, as the reference's model runner replays its decode graphs.

Printed on one JSON line: the metric (credited HBM bytes per step / time per step), microseconds
per layer, each kernel's average launch duration and bandwidth (HIP events around a graph of
back-to-back launches of that kernel, on the stream it runs on) beside the same for its memory
skeleton (a kernel moving the same streams of the same buffers with no arithmetic: the practical
ceiling at that size, launch ramp-up and drain included), the roofline of the dominant kernel, the
CPU baseline (the numpy oracle timed on a bounded sample of the same workload on the host, one
thread) and, for the layer workloads, the same sample as torch CPU code on all of torch's host
threads (`cpu_torch`).

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--protocol cold|hot] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

METRIC = "HBM GB/s & % of peak for layer kernels; µs/layer at 64-token decode"
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA
COLD_BYTES = 768 << 20         # working set cycled by the cold protocol (3x the Infinity Cache)
# HBM bytes per launch of a workload's dominant kernel, from two rocprofv3 counter passes
# (FETCH_SIZE, then WRITE_SIZE) over `bench.py --pmc-probe`, each calibrated by the same counter on
# a 256 MiB device copy (fetch factor 1.9997, write factor 1.0000). Re-measure when the kernel changes.
MEASURED_TRAFFIC = {("decode64_24b", "silu_and_mul"): 12_611_644,
                    ("prefill8192_24b", "silu_and_mul"): 1_610_374_077,
                    ("prefill16384_123b", "silu_and_mul"): 2_818_327_781,
                    ("decode_attn_64x8192_24b", "paged_decode_attention"): 1_114_384_294}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=None, help="timed steps (default: workload-dependent)")
    p.add_argument("--warmup", type=int, default=None)
    p.add_argument("--workload", default="decode64_24b")
    p.add_argument("--protocol", choices=("cold", "hot"), default="cold")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU time of the baseline sample")
    p.add_argument("--fp8", action="store_true",
                   help="the reference's FP8 dataflow: norms write fp8 for the qkv / gate_up GEMMs and SiluAndMul "
                        "writes the quantized down_proj input")
    p.add_argument("--pmc-probe", action="store_true",
                   help="short run for rocprofv3 --pmc: the dominant kernel 20 times on the cold layer sets, "
                        "then a 256 MiB device copy (the calibration reference for FETCH_SIZE / WRITE_SIZE)")
    p.add_argument("--separate-rope-kv", action="store_true",
                   help="run RoPE and the KV append as the reference's two calls (default: one fused kernel, "
                        "same results, one launch fewer per layer); the other form is timed alongside")
    return p.parse_args()


def footprint_bytes(shape) -> int:
    """Bytes one layer set's kernels touch (inputs + outputs + destination cache rows)."""
    n, h, i = shape.tokens, shape.hidden, shape.inter
    return 2 * (4 * n * h + 3 * n * i + n * shape.qkv_width) + 4 * n * shape.kv_heads * shape.head_dim


def step_ops(shape, fp8: bool) -> tuple[str, ...]:
    """The kernels timed one by one: norm, RoPE, KV store, SiluAndMul (the dominant kernel), and the
    fused RoPE + KV kernel; their fp8-output forms under the fp8 dataflow."""
    norm = "fused_add_rmsnorm_quant" if fp8 else "fused_add_rmsnorm"
    if shape.norm_only:
        return (norm,)
    return (norm, "rope", "append_paged_kv_cache", "silu_and_mul_quant" if fp8 else "silu_and_mul", "rope_append")


SKELETON_OPS = ("fused_add_rmsnorm", "rope", "append_paged_kv_cache", "silu_and_mul")
_skeleton_fn = None


def load_skeletons(mas) -> bool:
    """Loads the benchmark's memory skeletons (libmas_bench.so, built beside the kernel library)."""
    global _skeleton_fn
    path = Path(mas.__file__).resolve().parent / "libmas_bench.so"
    if not path.exists():
        return False
    fn = ctypes.CDLL(str(path)).mas_bench_stream_skeleton
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64] * 4 + [ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]
    _skeleton_fn = fn
    return True


def skeleton_launcher(b, op):
    """A closure launching the memory skeleton of ``op`` on the buffers of ``b``: the kernel's
    streams (same rows, row strides and read / write mix) moved with no arithmetic. The KV store's
    skeleton writes the cache's first rows instead of the mapped slots; index arrays and the norm
    weight are not moved."""
    li, s = b.inputs, b.inputs.shape
    n = s.tokens
    if op == "fused_add_rmsnorm":
        h, r = li.hidden, li.residual
        args = (h, h.stride(0), r, r.stride(0), h, h.stride(0), r, r.stride(0), n, s.hidden)
    elif op == "silu_and_mul":
        g = li.gate_up
        up = g[:, s.inter:]
        args = (g, g.stride(0), up, g.stride(0), b.silu_out, b.silu_out.stride(0), None, 0, n, s.inter)
    elif op == "rope":
        q = li.q
        args = (q, q.stride(0), None, 0, q, q.stride(0), None, 0, n, (s.q_heads + s.kv_heads) * s.head_dim)
    elif op == "append_paged_kv_cache":
        k, v, row = li.k, li.v, s.kv_heads * s.head_dim
        args = (k, k.stride(0), v, v.stride(0), li.k_cache, row, li.v_cache, row, n, row)
    else:
        raise ValueError(op)
    ptrs = [a.data_ptr() if isinstance(a, torch.Tensor) else a for a in args]

    def launch():
        st = _skeleton_fn(*ptrs, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        if st != 0:
            raise RuntimeError(f"memory skeleton of {op} failed with status {st}")
    return launch


def op_launcher(mas, b, op):
    """A closure launching one kernel of the layer on the buffers of ``b`` (``skeleton:<op>``: its
    memory skeleton)."""
    if op.startswith("skeleton:"):
        return skeleton_launcher(b, op.split(":", 1)[1])
    li, s = b.inputs, b.inputs.shape
    if op == "fused_add_rmsnorm":
        return lambda: mas.norm.fused_add_rmsnorm(li.hidden, li.residual, li.norm_weight, s.eps)
    if op == "rope":
        return lambda: mas.rope.apply_rope_with_cos_sin_cache_inplace(li.positions, li.q, li.k, s.head_dim, li.table,
                                                                      True)
    if op == "append_paged_kv_cache":
        return lambda: mas.page.append_paged_kv_cache(b.k3, b.v3, li.batch_indices, li.positions,
                                                      (li.k_cache, li.v_cache), b.kv_indices, li.kv_indptr, None,
                                                      "NHD")
    if op == "silu_and_mul":
        return lambda: mas.activation.silu_and_mul(li.gate_up, out=b.silu_out)
    if op == "silu_and_mul_quant":
        return lambda: mas.activation.silu_and_mul_quant(li.gate_up, b.act_scale, out=b.silu_out)
    if op == "fused_add_rmsnorm_quant":
        return lambda: mas.norm.fused_add_rmsnorm_quant(b.norm_out, li.hidden, li.residual, li.norm_weight,
                                                        b.act_scale, s.eps)
    if op == "rope_append":
        return lambda: mas.fused.apply_rope_and_append_paged_kv_cache(
            li.positions, li.q, li.k, b.v3, s.head_dim, li.table, True, li.batch_indices, (li.k_cache, li.v_cache),
            b.kv_indices, li.kv_indptr, None, "NHD")
    raise ValueError(op)


def time_ops(mas, layer_sets, launches: int, ops: tuple[str, ...], replays: int = 5) -> dict[str, float]:
    """Average launch duration (µs) of each kernel: a HIP graph of ``launches`` back-to-back launches
    of that kernel alone, cycling the layer sets, bracketed by two HIP events on the stream the
    graph replays on. The graph is replayed once untimed, then ``replays`` times, each between its
    own pair of events; the median replay is reported (GPU clocks vary between phases of a run)."""
    out = {}
    for op in ops:
        fns = [op_launcher(mas, layer_sets[i % len(layer_sets)], op) for i in range(launches)]

        def body():
            for f in fns:
                f()

        g = capture(body)
        g.replay()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(replays)]
        for start, stop in events:
            start.record()
            g.replay()
            stop.record()
        torch.cuda.synchronize()
        times = sorted(start.elapsed_time(stop) for start, stop in events)
        out[op] = 1000.0 * times[len(times) // 2] / launches
        del g
    return out


def copy_ceiling_gbs(dev, nbytes: int = 1 << 30) -> float:
    """Device-to-device copy rate (read + write bytes per second), a practical streaming ceiling."""
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(10):
        b.copy_(a)
    stop.record()
    torch.cuda.synchronize()
    return 2 * nbytes * 10 / (start.elapsed_time(stop) * 1e-3) / 1e9


def capture(fn) -> torch.cuda.CUDAGraph:
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def cpu_baseline_layer(shape, seconds: float, fp8: bool) -> dict:
    """The oracle's five layer ops on a bounded sample of the workload, timed on the host."""
    from oracle import ops as oops

    mas = __graft_entry__.load_package()
    wl = mas.workloads
    tokens = shape.tokens
    # A sample of whole tokens: the full batch when it fits the time budget, else a row slice.
    if tokens * ((0 if shape.norm_only else shape.inter) + shape.hidden) > 64 * (32768 + 5120):
        tokens = 64
    li = wl.make_layer_inputs(shape, "cpu", seed=1, with_cache=False)

    def u16(t):
        return t[:tokens].contiguous().view(torch.int16).numpy().view(np.uint16)

    x, r, w = u16(li.hidden), u16(li.residual), li.norm_weight.view(torch.int16).numpy().view(np.uint16)
    a, w2 = u16(li.attn_out), li.post_norm_weight.view(torch.int16).numpy().view(np.uint16)
    gu = u16(li.gate_up)
    qkv = u16(li.qkv)
    hq, hk, d = shape.q_heads, shape.kv_heads, shape.head_dim
    q = qkv[:, : hq * d].reshape(tokens, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].reshape(tokens, hk, d)
    v = qkv[:, (hq + hk) * d:].reshape(tokens, hk, d)
    pos = li.positions[:tokens].numpy()
    table = li.table.numpy()
    slots = li.slot_mapping[:tokens].numpy()
    # the destination pages only; untouched pages play no part in the store
    pages_used = np.unique(slots // shape.page_size)
    remap = {p: j for j, p in enumerate(pages_used)}
    local_slots = np.array([remap[s // shape.page_size] * shape.page_size + s % shape.page_size for s in slots])
    kc = np.zeros((len(pages_used), shape.page_size, hk, d), np.uint16)
    vc = np.zeros_like(kc)

    def layer():
        nonlocal x, r, kc, vc
        if fp8:
            _, r = oops.fused_add_rmsnorm_quant(x, r, w, 0.05, shape.eps)
        else:
            _, r = oops.fused_add_rmsnorm(x, r, w, shape.eps)
        if shape.norm_only:
            return
        oops.rope(q, k, pos, table)
        kc, vc = oops.store_kv_slots(kc, vc, k, v, local_slots)
        if fp8:
            _, r = oops.fused_add_rmsnorm_quant(a, r, w2, 0.05, shape.eps)
            oops.silu_and_mul_quant(gu, 0.05)
        else:
            _, r = oops.fused_add_rmsnorm(a, r, w2, shape.eps)
            oops.silu_and_mul(gu)

    sample_shape = type(shape)(**{**shape.__dict__, "tokens": tokens})
    per_layer = wl.layer_credited_bytes(sample_shape, False, fp8)   # the oracle runs RoPE and the store separately
    layer()                                  # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        layer()
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": round(per_layer * reps / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{reps} single-threaded numpy passes of the step's ops on {tokens} of "
                      f"{shape.tokens} tokens ({dt:.1f} s)"}


def cpu_torch_layer(shape, seconds: float, fp8: bool) -> dict:
    """The same sample as the oracle baseline, as torch CPU code on all of the host's torch threads:
    the reference's math in torch (fp32 from bf16, rounded once), the kind of CPU path a user without
    the GPU kernels would run. Reported beside the single-threaded oracle baseline."""
    import torch.nn.functional as F

    mas = __graft_entry__.load_package()
    wl = mas.workloads
    tokens = shape.tokens
    if tokens * ((0 if shape.norm_only else shape.inter) + shape.hidden) > 64 * (32768 + 5120):
        tokens = 64
    li = wl.make_layer_inputs(shape, "cpu", seed=1, with_cache=False)
    hq, hk, d, eps = shape.q_heads, shape.kv_heads, shape.head_dim, shape.eps
    x, r = li.hidden[:tokens].clone(), li.residual[:tokens].clone()
    w, w2 = li.norm_weight.float(), li.post_norm_weight.float()
    a, gu = li.attn_out[:tokens].clone(), li.gate_up[:tokens].clone()
    qkv = li.qkv[:tokens].clone()
    q = qkv[:, : hq * d].view(tokens, hq, d)
    k = qkv[:, hq * d:(hq + hk) * d].view(tokens, hk, d)
    v = qkv[:, (hq + hk) * d:].view(tokens, hk, d)
    cs = li.table[li.positions[:tokens].long()]
    half = d // 2
    c, sn = cs[:, None, :half], cs[:, None, half:]
    slots = li.slot_mapping[:tokens].numpy()
    pages_used = np.unique(slots // shape.page_size)
    remap = {p: j for j, p in enumerate(pages_used)}
    local = torch.tensor([remap[s // shape.page_size] * shape.page_size + s % shape.page_size for s in slots])
    kc = torch.zeros(len(pages_used) * shape.page_size, hk, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    inter = shape.inter

    def norm(inp, res, weight):
        s_ = inp.float() + res.float()
        y = s_ * torch.rsqrt(s_.pow(2).mean(-1, keepdim=True) + eps) * weight
        return (y / 0.05).clamp(-448, 448).to(torch.float8_e4m3fn) if fp8 else y.bfloat16(), s_.bfloat16()

    op_s = {"fused_add_rmsnorm": 0.0, "rope": 0.0, "append_paged_kv_cache": 0.0, "silu_and_mul": 0.0}
    clock = time.perf_counter

    def layer():
        nonlocal r
        t = clock()
        _, r = norm(x, r, w)
        op_s["fused_add_rmsnorm"] += clock() - t
        if shape.norm_only:
            return
        t = clock()
        for u in (q, k):
            x1, x2 = u[..., :half].float(), u[..., half:].float()
            u[..., :half] = (x1 * c - x2 * sn).bfloat16()
            u[..., half:] = (x2 * c + x1 * sn).bfloat16()
        t2 = clock()
        kc[local] = k
        vc[local] = v
        t3 = clock()
        _, r = norm(a, r, w2)
        t4 = clock()
        y = (F.silu(gu[:, :inter].float()) * gu[:, inter:].float()).bfloat16()
        if fp8:
            (y.float() / 0.05).clamp(-448, 448).to(torch.float8_e4m3fn)
        t5 = clock()
        op_s["rope"] += t2 - t
        op_s["append_paged_kv_cache"] += t3 - t2
        op_s["fused_add_rmsnorm"] += t4 - t3
        op_s["silu_and_mul"] += t5 - t4

    sample_shape = type(shape)(**{**shape.__dict__, "tokens": tokens})
    per_layer = wl.layer_credited_bytes(sample_shape, False, fp8)
    layer()
    for key in op_s:
        op_s[key] = 0.0
    reps, t0 = 0, time.perf_counter()
    while True:
        layer()
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    calls = {"fused_add_rmsnorm": 1 if shape.norm_only else 2}
    return {"value": round(per_layer * reps / dt / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "torch",
            "sample": f"{reps} passes of the step's ops as torch CPU code on {tokens} of {shape.tokens} tokens "
                      f"({dt:.1f} s, {torch.get_num_threads()} threads)",
            # average µs per call of each op on the sample's tokens
            "op_us": {key: round(1e6 * v / (reps * calls.get(key, 1)), 1) for key, v in op_s.items() if v > 0}}


def run_layer_workload(mas, args, shape, dev) -> dict:
    wl, lp = mas.workloads, mas.layer_pass
    n_sets = 1 if args.protocol == "hot" else max(2, math.ceil(COLD_BYTES / footprint_bytes(shape)))
    table = mas.rope.cos_sin_cache(shape.max_position, shape.head_dim, shape.theta).to(dev)
    sets = [lp.LayerBuffers(wl.make_layer_inputs(shape, dev, seed=i, fill_on_device=True, table=table,
                                                     zero_cache=False),
                            fp8=args.fp8, fuse_rope_kv=not args.separate_rope_kv) for i in range(n_sets)]
    fused = not args.separate_rope_kv
    per_step = wl.layer_credited_bytes(shape, fused, args.fp8)
    steps = args.steps if args.steps is not None else (2000 if shape.decode else 40)
    warmup = args.warmup if args.warmup is not None else max(n_sets, steps // 10)

    def run_range(lo, hi):
        for i in range(lo, hi):
            lp.run_layer(sets[i % n_sets])

    def timed_steps(k: int, w: int) -> float:
        """Seconds for k steps replayed from HIP graphs after w warm-up steps. One replay runs a
        whole number of passes over the layer sets and at least 50 steps, amortising the launch."""
        per_graph = n_sets * max(1, math.ceil(50 / n_sets))
        graphs = {per_graph: capture(lambda: run_range(0, per_graph))}
        for count in (w, k):                          # every graph is captured before the timed region
            rem = count % per_graph
            if rem and rem not in graphs:
                graphs[rem] = capture(lambda: run_range(0, rem))

        def replay(count):
            for _ in range(count // per_graph):
                graphs[per_graph].replay()
            if count % per_graph:
                graphs[count % per_graph].replay()

        replay(w)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        replay(k)
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    elapsed = timed_steps(steps, warmup)
    other_us = None
    if not shape.norm_only:
        # the other RoPE / KV form, for comparison (same buffers, same step count)
        for b in sets:
            b.fuse_rope_kv = not fused
        other_us = timed_steps(steps, warmup) / steps * 1e6
        for b in sets:
            b.fuse_rope_kv = fused

    # stream-launched steps (no graph), for comparison
    stream_steps = min(steps, 10 * n_sets) if shape.decode else min(steps, 4 * n_sets)
    torch.cuda.synchronize()
    s0 = time.perf_counter()
    run_range(0, stream_steps)
    torch.cuda.synchronize()
    stream_us = (time.perf_counter() - s0) / stream_steps * 1e6

    launches = max(2 * n_sets, 100) if shape.decode else 4 * n_sets
    kernels = step_ops(shape, args.fp8)
    skeletons = tuple(f"skeleton:{op}" for op in kernels if op in SKELETON_OPS and shape.tokens <= 65535) \
        if _skeleton_fn is not None else ()
    op_us = time_ops(mas, sets, launches, kernels + skeletons)
    cb = wl.credited_bytes(shape)
    ops = {op: {"us": round(op_us[op], 3), "GB/s": round(cb[op] / op_us[op] / 1e3, 1),
                "frac": round(cb[op] / op_us[op] / 1e3 / PEAK_HBM_GBS, 4)} for op in kernels}
    for op in kernels:
        if f"skeleton:{op}" in op_us:
            sk = op_us[f"skeleton:{op}"]
            ops[op]["skeleton_us"] = round(sk, 3)
            ops[op]["of_skeleton"] = round(sk / op_us[op], 3)
    ms_per_step = elapsed / steps * 1e3
    dominant = step_ops(shape, args.fp8)[0 if shape.norm_only else 3]
    res = {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
           "value": per_step / (ms_per_step * 1e-3) / 1e9, "stream_us_per_step": stream_us, "ops": ops,
           "sets": n_sets, "dominant": dominant, "dominant_bytes": cb[dominant], "dominant_us": op_us[dominant]}
    if other_us is not None:
        res["separate_us_per_layer" if fused else "fused_us_per_layer"] = other_us
    return res


def run_pass_workload(mas, args, shape, dev) -> dict:
    lp, wl = mas.layer_pass, mas.workloads
    passes = [lp.DecodePass(shape, dev, seed=0, fp8=args.fp8, fuse_rope_kv=not args.separate_rope_kv)]
    per_step = passes[0].credited_bytes()
    steps = args.steps if args.steps is not None else 20
    warmup = args.warmup if args.warmup is not None else 3
    g = capture(passes[0].run)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ops_timed = step_ops(shape, args.fp8)
    op_us = time_ops(mas, passes[0].layers, shape.layers, ops_timed)
    cb = wl.credited_bytes(shape)
    ops = {op: {"us": round(us, 3), "GB/s": round(cb[op] / us / 1e3, 1),
                "frac": round(cb[op] / us / 1e3 / PEAK_HBM_GBS, 4)} for op, us in op_us.items()}
    ms_per_step = elapsed / steps * 1e3
    dominant = ops_timed[3]
    return {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
            "value": per_step / (ms_per_step * 1e-3) / 1e9, "ops": ops, "sets": 1, "dominant": dominant,
            "dominant_bytes": cb[dominant], "dominant_us": op_us[dominant],
            "us_per_layer": ms_per_step * 1e3 / shape.layers}


def run_attention_workload(mas, args, shape, dev) -> dict:
    """Paged decode attention (both kernels of one call) on the workload's rows; the step is one call."""
    wl = mas.workloads
    inp = wl.make_attention_inputs(shape, dev, seed=0)
    per_step = wl.attention_credited_bytes(inp)
    out = torch.empty_like(inp.q)
    scale = shape.head_dim ** -0.5

    def call():
        mas.attention.trtllm_batch_decode_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), inp.workspace,
                                                        inp.block_tables, inp.seq_lens, 0, scale, 1.0, out=out)

    steps = args.steps if args.steps is not None else 50
    warmup = args.warmup if args.warmup is not None else 5
    call()
    g = capture(call)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # per-call duration: HIP events around graphs of back-to-back calls, median of five replays
    graph_calls = 10
    gb = capture(lambda: [call() for _ in range(graph_calls)])
    gb.replay()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
    for start, stop in events:
        start.record()
        gb.replay()
        stop.record()
    torch.cuda.synchronize()
    call_us = 1000.0 * sorted(a.elapsed_time(b) for a, b in events)[2] / graph_calls
    ms_per_step = elapsed / steps * 1e3
    lens = inp.seq_lens.cpu()
    return {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
            "value": per_step / (ms_per_step * 1e-3) / 1e9, "sets": 1, "dominant": "paged_decode_attention",
            "dominant_bytes": per_step, "dominant_us": call_us,
            "ops": {"paged_decode_attention": {"us": round(call_us, 3), "GB/s": round(per_step / call_us / 1e3, 1),
                                               "frac": round(per_step / call_us / 1e3 / PEAK_HBM_GBS, 4)}},
            "attention": {"mean_len": round(float(lens.float().mean()), 1), "longest": int(lens.max()),
                          "positions": int(lens.sum()), "kv_pages": inp.k_cache.shape[0]},
            "inputs": inp}


def context_main(mas, args, shape, dev) -> int:
    """Causal context attention: a step is one call; the value is TFLOP/s of algorithmic flops."""
    wl = mas.workloads
    inp = wl.make_context_inputs(shape, dev, seed=0)
    out = torch.empty_like(inp.q)
    flops = wl.context_flops(shape)
    scale = shape.head_dim ** -0.5
    ws = torch.empty(16, dtype=torch.uint8, device=dev)

    def call():
        mas.attention.trtllm_batch_context_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), ws, inp.block_tables,
                                                         inp.seq_lens, shape.q_len, shape.q_len + shape.cached,
                                                         scale, 1.0, shape.rows, inp.cu_seqlens_q, None, out=out)

    steps = args.steps if args.steps is not None else 20
    warmup = args.warmup if args.warmup is not None else 3
    call()
    g = capture(call)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    gb = capture(lambda: [call() for _ in range(4)])
    gb.replay()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
    for start, stop in events:
        start.record()
        gb.replay()
        stop.record()
    torch.cuda.synchronize()
    call_us = 1000.0 * sorted(x.elapsed_time(y) for x, y in events)[2] / 4
    ms_per_step = elapsed / steps * 1e3
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    kernel_tflops = flops / (call_us * 1e-6) / 1e12
    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": shape.name, "rows": shape.rows, "q_len": shape.q_len, "cached": shape.cached,
                   "q_heads": shape.q_heads, "kv_heads": shape.kv_heads, "head_dim": shape.head_dim,
                   "page_size": shape.page_size, "flops": flops, "launch": "hip-graph"},
        "us_per_call": round(ms_per_step * 1e3, 3),
        "ops": {"paged_context_attention": {"us": round(call_us, 3), "TFLOP/s": round(kernel_tflops, 1),
                                            "frac": round(kernel_tflops / PEAK_BF16_TFLOPS, 4)}},
        "roofline": {"bound": "mfma", "kernel": "paged_context_attention", "achieved": round(kernel_tflops, 1),
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(kernel_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": None, "flops_per_launch": flops, "avg_launch_us": round(call_us, 3)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_context(inp, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


def cpu_baseline_context(inp, seconds: float) -> dict:
    """The oracle's causal attention on the host, on query tokens of the first row taken from its
    end (the longest reach), for about ``seconds``; algorithmic flops done per second."""
    from oracle import ops as oops

    s = inp.shape
    kv_len = s.cached + s.q_len
    q = inp.q.cpu().view(torch.int16).numpy().view(np.uint16)
    kc = inp.k_cache.cpu().view(torch.int16).numpy().view(np.uint16)
    vc = inp.v_cache.cpu().view(torch.int16).numpy().view(np.uint16)
    tables = inp.block_tables.cpu().numpy()[:1]
    done, tokens, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds and tokens < s.q_len:
        # one query token at a time (a row of one token whose kv_len is its position + 1)
        i = s.q_len - 1 - tokens
        pos = s.cached + i
        oops.paged_context_attention(q[i:i + 1], kc, vc, tables, np.array([pos + 1]), np.array([0, 1]),
                                     s.head_dim ** -0.5)
        done += (pos + 1) * s.q_heads * s.head_dim * 4
        tokens += 1
    elapsed = time.perf_counter() - t0
    return {"value": round(done / elapsed / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{tokens} query tokens of one row (longest reach first), single-threaded numpy ({elapsed:.1f} s)"}


def cpu_baseline_attention(inp, seconds: float) -> dict:
    """The oracle's decode attention on the host, one row at a time over the workload's rows (cycling),
    for about ``seconds``; credited bytes of the rows done per second."""
    from oracle import ops as oops

    s = inp.shape
    q = inp.q.cpu().view(torch.int16).numpy().view(np.uint16)
    kc = inp.k_cache.cpu().view(torch.int16).numpy().view(np.uint16)
    vc = inp.v_cache.cpu().view(torch.int16).numpy().view(np.uint16)
    tables = inp.block_tables.cpu().numpy()
    lens = inp.seq_lens.cpu().numpy()
    done_bytes, rows, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        b = rows % s.batch
        oops.paged_decode_attention(q[b:b + 1], kc, vc, tables[b:b + 1], lens[b:b + 1], s.head_dim ** -0.5)
        n = int(lens[b])
        done_bytes += n * s.kv_heads * s.head_dim * 4 + 2 * s.q_heads * s.head_dim * 2 + 4 * (-(-n // s.page_size)) + 4
        rows += 1
    elapsed = time.perf_counter() - t0
    return {"value": round(done_bytes / elapsed / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{rows} rows of the workload's decode attention, single-threaded numpy ({elapsed:.1f} s)"}


def pmc_probe(mas, args, shape, dev) -> None:
    """Launches only what a counter pass needs: the workload's dominant kernel (SiluAndMul, or the
    norm for the norm-only case) 20 times across the cold layer sets, then 4 copies of 256 MiB."""
    wl, lp = mas.workloads, mas.layer_pass
    n_sets = max(2, math.ceil(COLD_BYTES / footprint_bytes(shape)))
    table = mas.rope.cos_sin_cache(shape.max_position, shape.head_dim, shape.theta).to(dev)
    sets = [lp.LayerBuffers(wl.make_layer_inputs(shape, dev, seed=i, fill_on_device=True, table=table,
                                                 zero_cache=False)) for i in range(n_sets)]
    op = step_ops(shape, False)[0 if shape.norm_only else 3]
    for i in range(20):
        op_launcher(mas, sets[i % n_sets], op)()
    torch.cuda.synchronize()
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(4):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": op, "launches": 20, "bytes_per_launch": wl.credited_bytes(shape)[op],
                      "calibration_copy_bytes": 256 << 20}), flush=True)


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py runs on one GPU: these kernels have no multi-GPU path (asked for --gpus {args.gpus}, "
              f"WORLD_SIZE {world}); the layer kernels are token-parallel and would shard without exchange",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    mas = __graft_entry__.load_package()
    mas.load_library()
    load_skeletons(mas)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload in mas.workloads.CONTEXT_SHAPES:
        return context_main(mas, args, mas.workloads.CONTEXT_SHAPES[args.workload], dev)
    if args.workload in mas.workloads.ATTENTION_SHAPES:
        return attention_main(mas, args, mas.workloads.ATTENTION_SHAPES[args.workload], dev)
    shape = mas.workloads.SHAPES[args.workload]
    if args.pmc_probe:
        pmc_probe(mas, args, shape, dev)
        return 0
    if shape.layers > 1:
        res = run_pass_workload(mas, args, shape, dev)
    else:
        res = run_layer_workload(mas, args, shape, dev)

    dom_gbs = res["dominant_bytes"] / res["dominant_us"] / 1e3
    line = {
        "metric": METRIC,
        "value": round(res["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": res["warmup"],
        "ms_per_step": round(res["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": shape.name, "tokens": shape.tokens, "hidden": shape.hidden,
                   "intermediate": shape.inter, "q_heads": shape.q_heads, "kv_heads": shape.kv_heads,
                   "head_dim": shape.head_dim, "kv_pages": shape.num_pages, "page_size": shape.page_size,
                   "layers": shape.layers, "protocol": args.protocol, "layer_sets": res["sets"],
                   "launch": "hip-graph", "dataflow": "fp8" if args.fp8 else "bf16",
                   "rope_kv": "separate" if args.separate_rope_kv else "fused"},
        "us_per_layer": round(res.get("us_per_layer", res["ms_per_step"] * 1e3), 3),
        "frac_of_peak": round(res["value"] / PEAK_HBM_GBS, 4),
        "ops": res["ops"],
        "roofline": {"bound": "hbm", "kernel": res["dominant"], "achieved": round(dom_gbs, 1),
                     "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(dom_gbs / PEAK_HBM_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get((shape.name, res["dominant"])),
                     "bytes_per_launch": res["dominant_bytes"],
                     "avg_launch_us": round(res["dominant_us"], 3)},
    }
    dom = res["ops"].get(res["dominant"], {})
    if "skeleton_us" in dom:
        # the same bytes, buffers and launch shape moved by a kernel with no arithmetic, same run
        sk_gbs = res["dominant_bytes"] / dom["skeleton_us"] / 1e3
        line["roofline"]["skeleton"] = {"us": dom["skeleton_us"], "GB/s": round(sk_gbs, 1),
                                        "frac": round(sk_gbs / PEAK_HBM_GBS, 4)}
        line["roofline"]["frac_of_skeleton"] = dom["of_skeleton"]
    for key in ("separate_us_per_layer", "fused_us_per_layer", "stream_us_per_step"):
        if key in res:
            line[key] = round(res[key], 3)
    line["copy_ceiling_GBps"] = round(copy_ceiling_gbs(dev), 1)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_layer(shape, args.cpu_seconds, args.fp8)
        line["cpu_torch"] = cpu_torch_layer(shape, args.cpu_seconds / 2, args.fp8)
    print(json.dumps(line), flush=True)
    return 0


def attention_main(mas, args, shape, dev) -> int:
    if args.pmc_probe:
        # 5 calls of the op, then 4 copies of 256 MiB (the counters' calibration reference)
        wl = mas.workloads
        inp = wl.make_attention_inputs(shape, dev, seed=0)
        out = torch.empty_like(inp.q)
        for _ in range(5):
            mas.attention.trtllm_batch_decode_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), inp.workspace,
                                                            inp.block_tables, inp.seq_lens, 0,
                                                            shape.head_dim ** -0.5, 1.0, out=out)
        torch.cuda.synchronize()
        src = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "paged_decode_attention", "launches": 5,
                          "bytes_per_launch": wl.attention_credited_bytes(inp),
                          "calibration_copy_bytes": 256 << 20}), flush=True)
        return 0
    res = run_attention_workload(mas, args, shape, dev)
    dom_gbs = res["dominant_bytes"] / res["dominant_us"] / 1e3
    line = {
        "metric": METRIC, "value": round(res["value"], 2), "unit": "GB/s", "n_gpus": 1, "steps": res["steps"],
        "warmup": res["warmup"], "ms_per_step": round(res["ms_per_step"], 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": shape.name, "batch": shape.batch, "q_heads": shape.q_heads,
                   "kv_heads": shape.kv_heads, "head_dim": shape.head_dim, "page_size": shape.page_size,
                   "max_len": shape.max_len, **res["attention"], "launch": "hip-graph"},
        "us_per_call": round(res["ms_per_step"] * 1e3, 3),
        "frac_of_peak": round(res["value"] / PEAK_HBM_GBS, 4),
        "ops": res["ops"],
        "roofline": {"bound": "hbm", "kernel": res["dominant"], "achieved": round(dom_gbs, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(dom_gbs / PEAK_HBM_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get((shape.name, res["dominant"])),
                     "bytes_per_launch": res["dominant_bytes"], "avg_launch_us": round(res["dominant_us"], 3)},
        "copy_ceiling_GBps": round(copy_ceiling_gbs(dev), 1),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline_attention(res["inputs"], args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
