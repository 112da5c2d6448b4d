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

Timing: after the warm-up steps, the --steps timed steps run in chunks of at most 50; each chunk's
HIP graph runs untimed lead-in steps, a kernel that stores the GPU wall clock, the chunk's steps, a
second clock store and one more step. Each graph is replayed once untimed (a graph's first replay
also uploads it), then the chunks' stamped intervals are summed: exactly --steps steps, with no
graph launch or host gap inside (ROCm does not allow timing events inside graphs). Beside it: HIP events around replays of graphs of the timed steps
alone (graph launch included, ``graph_us_per_step``) and the host clock (``host_us_per_step``).
At decode sizes the line also carries the host time of one eager call of each op's wrapper
(``eager_host_us_per_call``): the reference runs steps past its graph sizes eagerly.

Printed on one JSON line: the metric (credited HBM bytes per step / time per step), microseconds
per layer, each kernel's average launch duration and bandwidth (HIP events around a graph of
back-to-back launches of that kernel, on the stream it runs on) beside the same for its memory
skeleton (a kernel moving the same streams of the same buffers with no arithmetic: the practical
ceiling at that size, launch ramp-up and drain included), the roofline of the dominant kernel, the
CPU baseline (the same ops as torch CPU code on all of torch's host threads, on a bounded sample of
the workload, thread count stated) and, beside it, the numpy oracle on one thread (`cpu_oracle`).

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
# Figures taken from committed rocprofv3 profiles (profiles/), each with the git blob hashes
# (`git hash-object <file>`) of the kernel sources it was measured on. `stale_sources` reports a
# figure whose sources have changed since: the bench line then carries it with "stale": true and
# takes its roofline from the live HIP-event timing instead.
KERNEL_SOURCES = {
    "silu_and_mul": ("csrc/silu_and_mul.hip", "csrc/device.h"),
    "fused_add_rmsnorm": ("csrc/rmsnorm.hip", "csrc/device.h"),
    "paged_decode_attention": ("csrc/attention.hip", "csrc/device.h"),
    "paged_context_attention": ("csrc/context_attention.hip", "csrc/device.h"),
}
# Git blob hashes of the kernel sources the profiled figures below were measured on.
_SILU_SOURCES = {"csrc/silu_and_mul.hip": "23b0260df03f552c5aeb3be5992d159ad4873f02",
                 "csrc/device.h": "4a649fbd27cb9b4a8503ee1b497b4df962d5650e"}
_NORM_SOURCES = {"csrc/rmsnorm.hip": "089cb088624451ba8a83f3bc292864153fe93b0d",
                 "csrc/device.h": "4a649fbd27cb9b4a8503ee1b497b4df962d5650e"}
_DECODE_ATTN_SOURCES = {"csrc/attention.hip": "dc9407d13c4dacbefa466e7aeb4a548403f5d5f6",
                        "csrc/device.h": "4a649fbd27cb9b4a8503ee1b497b4df962d5650e"}
# HBM bytes per launch of a workload's dominant kernel: two rocprofv3 counter passes (FETCH_SIZE,
# then WRITE_SIZE) over `bench.py --pmc-probe`, each calibrated by the same counter on a 256 MiB
# device copy.
MEASURED_TRAFFIC = {
    ("decode64_24b", "silu_and_mul"): {
        "bytes": 12_612_732, "profile": "profiles/silu_and_mul_decode64_hbm_traffic.md", "sources": _SILU_SOURCES},
    ("rmsnorm_256x5120", "fused_add_rmsnorm"): {
        "bytes": 10_607_023, "profile": "profiles/rmsnorm_256x5120_kernel_trace.md", "sources": _NORM_SOURCES},
    ("decode_pass_256x40", "silu_and_mul"): {
        "bytes": 50_357_113, "profile": "profiles/decode_pass_256x40_kernel_trace.md", "sources": _SILU_SOURCES},
    ("prefill8192_24b", "silu_and_mul"): {
        "bytes": 1_610_475_810, "profile": "profiles/silu_and_mul_prefill_hbm_traffic.md", "sources": _SILU_SOURCES},
    ("decode_attn_64x8192_24b", "paged_decode_attention"): {
        "bytes": 1_115_079_915, "profile": "profiles/decode_attention_64x8192_kernel_trace.md",
        "sources": _DECODE_ATTN_SOURCES},
    ("decode_attn_64x8192_123b", "paged_decode_attention"): {
        "bytes": 1_188_499_821, "profile": "profiles/decode_attention_64x8192_kernel_trace.md",
        "sources": _DECODE_ATTN_SOURCES},
}
# Average per-dispatch duration (µs) of a workload's dominant kernel in a committed kernel trace of
# `bench.py --trace-probe ops` (the same graph of back-to-back launches the bench times with HIP
# events, and nothing else). The roofline's `achieved` and `frac` use this duration.
TRACED_LAUNCH_US = {
    ("decode64_24b", "silu_and_mul"): {
        "us": 3.919, "profile": "profiles/layer_decode64_kernel_trace.md", "sources": _SILU_SOURCES},
    ("rmsnorm_256x5120", "fused_add_rmsnorm"): {
        "us": 3.899, "profile": "profiles/rmsnorm_256x5120_kernel_trace.md", "sources": _NORM_SOURCES},
    ("decode_pass_256x40", "silu_and_mul"): {
        "us": 9.562, "profile": "profiles/decode_pass_256x40_kernel_trace.md", "sources": _SILU_SOURCES},
    ("prefill8192_24b", "silu_and_mul"): {
        "us": 234.195, "profile": "profiles/layer_prefill8192_kernel_trace.md", "sources": _SILU_SOURCES},
    ("decode_attn_64x8192_24b", "paged_decode_attention"): {     # split + combine
        "us": 203.167 + 7.818, "profile": "profiles/decode_attention_64x8192_kernel_trace.md",
        "sources": _DECODE_ATTN_SOURCES},
    ("decode_attn_64x8192_123b", "paged_decode_attention"): {
        "us": 222.873 + 15.600, "profile": "profiles/decode_attention_64x8192_kernel_trace.md",
        "sources": _DECODE_ATTN_SOURCES},
}


def source_blob(rel: str) -> str:
    """Git blob hash of a package source file (what `git hash-object` prints), computed without git:
    sha1 of b"blob <size>\\0" followed by the file's bytes."""
    import hashlib
    data = (ROOT / "mini-agent-serve_amd" / rel).read_bytes()
    return hashlib.sha1(b"blob %d\0" % len(data) + data).hexdigest()


def stale_sources(entry: dict, kernel: str) -> list[str]:
    """Sources of ``kernel`` whose blob hash differs from the one ``entry`` (a profiled figure) was
    measured on; every source when the entry records none."""
    recorded = entry.get("sources", {})
    return [rel for rel in KERNEL_SOURCES.get(kernel, ()) if recorded.get(rel) != source_blob(rel)]


def roofline_entry(shape_name: str, kernel: str, amount: int, event_us: float, bound: str = "hbm") -> dict:
    """The `roofline` object of a line: `amount` is the kernel's algorithmic bytes (bound "hbm") or
    flops (bound "mfma") per launch. Achieved rate and frac come from the committed trace's
    per-dispatch duration when one exists for this kernel and workload and its sources are unchanged,
    else from the live HIP-event duration; both figures are carried."""
    key = (shape_name, kernel)
    hbm = bound == "hbm"
    peak, unit, scale = (PEAK_HBM_GBS, "GB/s", 1e3) if hbm else (PEAK_BF16_TFLOPS, "TFLOP/s", 1e6)
    out = {"bound": bound, "kernel": kernel}
    traced = TRACED_LAUNCH_US.get(key)
    traced_stale = stale_sources(traced, kernel) if traced else []
    use_trace = traced is not None and not traced_stale
    us = traced["us"] if use_trace else event_us
    rate = amount / us / scale
    out.update({"achieved": round(rate, 1), "peak": peak, "unit": unit, "frac": round(rate / peak, 4)})
    traffic = MEASURED_TRAFFIC.get(key)
    traffic_stale = stale_sources(traffic, kernel) if traffic else []
    out["traffic"] = traffic["bytes"] if traffic and not traffic_stale else None
    out["bytes_per_launch" if hbm else "flops_per_launch"] = amount
    out["avg_launch_us"] = round(us, 3)
    out["timing"] = f"rocprofv3 kernel trace, {traced['profile']}" if use_trace else "hip-events (live)"
    out["event_avg_launch_us"] = round(event_us, 3)
    out["frac_event"] = round(amount / event_us / scale / peak, 4)
    if traced is not None:
        out["traced_avg_launch_us"] = round(traced["us"], 3)
        out["traced_in"] = traced["profile"]
        out["trace_stale"] = bool(traced_stale)
    if traffic is not None:
        out["traffic_in"] = traffic["profile"]
        out["traffic_stale"] = bool(traffic_stale)
    return out


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
                   help="short run for rocprofv3 --pmc: one kernel (--pmc-op, default the dominant one) 20 times "
                        "on the cold layer sets, then a 256 MiB device copy (the calibration reference for "
                        "FETCH_SIZE / WRITE_SIZE); decode attention workloads: 5 calls, then the copies; context "
                        "attention workloads: 5 calls")
    p.add_argument("--trace-probe", choices=("ops", "steps"), default=None,
                   help="short run for rocprofv3 --kernel-trace: 'ops' launches only the per-kernel graphs of "
                        "back-to-back launches (and memory skeletons) the bench times with HIP events; 'steps' only "
                        "the stamped step graphs; prints the same run's HIP-event figures")
    p.add_argument("--pmc-op", default=None,
                   help="kernel for --pmc-probe: fused_add_rmsnorm, rope, append_paged_kv_cache, silu_and_mul, "
                        "rope_append, fused_add_rmsnorm_quant or silu_and_mul_quant")
    p.add_argument("--sets", type=int, default=None,
                   help="number of layer sets the cold protocol cycles (default: enough that one step's buffers "
                        "exceed 768 MB)")
    p.add_argument("--table-per-set", action="store_true",
                   help="give every cold layer set its own cos/sin table, so RoPE's table rows come from HBM as in a "
                        "forward pass whose weight traffic evicts the table between layers")
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


SKELETON_OPS = ("fused_add_rmsnorm", "rope", "append_paged_kv_cache", "silu_and_mul", "rope_append")
_skeleton_fn = None
_rope_append_skeleton_fn = None
_stamp_fn = None
_clock_khz = 0


def load_skeletons(mas) -> None:
    """Loads the benchmark's library (libmas_bench.so, built beside the kernel library): the memory
    skeletons and the wall-clock stamp kernel that brackets timed steps inside a graph."""
    global _skeleton_fn, _rope_append_skeleton_fn, _stamp_fn, _clock_khz
    path = Path(mas.__file__).resolve().parent / "libmas_bench.so"
    if not path.exists():
        raise RuntimeError(f"{path.name} is not built; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    fn = lib.mas_bench_stream_skeleton
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    _skeleton_fn = fn
    fn = lib.mas_bench_rope_append_skeleton
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 3 + [ctypes.c_void_p] * 2 + [ctypes.c_int64] * 3 + \
        [ctypes.c_void_p]
    _rope_append_skeleton_fn = fn
    _stamp_fn = lib.mas_bench_timestamp
    _stamp_fn.restype = ctypes.c_int
    _stamp_fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    khz = ctypes.c_int(0)
    lib.mas_bench_wall_clock_khz.restype = ctypes.c_int
    if lib.mas_bench_wall_clock_khz(ctypes.byref(khz)) != 0 or khz.value <= 0:
        raise RuntimeError("could not read the GPU wall-clock rate")
    _clock_khz = khz.value


def _stamp(ptr: int) -> None:
    if _stamp_fn(ptr, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) != 0:
        raise RuntimeError("timestamp kernel launch failed")


def time_steps(run_steps, k: int, w: int, lead: int, per_graph: int) -> dict:
    """Times exactly ``k`` steps. ``run_steps(lo, hi)`` enqueues steps lo..hi-1 (step i uses input
    set i modulo the sets, so consecutive ranges continue the cycle).

    The k steps run in chunks of at most ``per_graph``. Each chunk's HIP graph holds ``lead``
    untimed steps, a wall-clock stamp, the chunk's steps, a second stamp and one more step, so the
    stamps bracket exactly those steps inside one graph replay: no graph launch, host gap or
    synchronisation falls between them (one kernel boundary does: the second stamp's dispatch).
    After ``w`` warm-up steps (their own graph) and one untimed replay of each chunk graph (a
    graph's first replay on ROCm also uploads it, ~9% slower), the chunk graphs are replayed in
    turn and their intervals summed. Chunks keep graphs small: a single graph of a few thousand
    kernels ran ~7% slower per kernel than graphs of a few hundred. Also reported: HIP events
    around replays of graphs of the k steps alone (graph launch included) and the host clock
    around replay + synchronize."""
    stamps = torch.zeros(2, dtype=torch.int64, device="cuda")
    at = stamps.data_ptr()
    chunk = max(1, min(k, per_graph))
    sizes = [chunk] * (k // chunk) + ([k % chunk] if k % chunk else [])

    def stamped(count):
        def body():
            run_steps(0, lead)
            _stamp(at)
            run_steps(lead, lead + count)
            _stamp(at + 8)
            run_steps(lead + count, lead + count + 1)
        return capture(body)

    graphs = {count: stamped(count) for count in set(sizes)}
    warm = capture(lambda: run_steps(0, w)) if w > 0 else None
    torch.cuda.synchronize()
    if warm is not None:
        warm.replay()
    for g in graphs.values():
        g.replay()
    ticks = 0
    for count in sizes:
        graphs[count].replay()
        torch.cuda.synchronize()
        t0, t1 = stamps.tolist()
        ticks += t1 - t0
    del graphs, warm
    graph_s, host_s = timed_replays(lambda count: capture(lambda: run_steps(0, count)), per_graph, k, w)
    return {"device_s": ticks / (_clock_khz * 1e3), "graph_s": graph_s, "host_s": host_s, "chunks": len(sizes)}


def skeleton_launcher(b, op, block: int = 256):
    """A closure launching the memory skeleton of ``op`` on the buffers of ``b``: the kernel's
    streams (same rows, row strides and read / write mix) moved with no arithmetic, in workgroups of
    ``block`` threads. The KV store's skeleton writes the cache's first rows instead of the mapped
    slots; index arrays and the norm weight are not moved."""
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
    elif op == "rope_append":
        qkv, row = li.qkv, s.kv_heads * s.head_dim
        ptrs = (qkv.data_ptr(), qkv.stride(0), (s.q_heads + s.kv_heads) * s.head_dim, row, li.k_cache.data_ptr(),
                li.v_cache.data_ptr(), row, n, block)

        def launch_fused():
            st = _rope_append_skeleton_fn(*ptrs, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            if st != 0:
                raise RuntimeError(f"memory skeleton of {op} failed with status {st}")
        return launch_fused
    else:
        raise ValueError(op)
    ptrs = [a.data_ptr() if isinstance(a, torch.Tensor) else a for a in args] + [block]

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
    if op.startswith("skeleton64:"):
        return skeleton_launcher(b, op.split(":", 1)[1], block=64)
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


def eager_host_us(mas, layer_sets, ops: tuple[str, ...], calls: int = 500) -> dict[str, float]:
    """Host time (µs) of one eager call of each op's Python wrapper (argument checks, stream query,
    ctypes call and kernel launch): ``calls`` back-to-back calls on the launch stream, timed on the
    host clock without waiting for the GPU (these decode-sized kernels run shorter than a call), after
    50 untimed calls."""
    out = {}
    for op in ops:
        fns = [op_launcher(mas, layer_sets[i % len(layer_sets)], op) for i in range(calls + 50)]
        for f in fns[:50]:
            f()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for f in fns[50:]:
            f()
        out[op] = round((time.perf_counter() - t0) / calls * 1e6, 2)
        torch.cuda.synchronize()
    return out


def timed_replays(make_graph, per_graph: int, k: int, w: int) -> tuple[float, float]:
    """(device seconds, host seconds) for exactly ``k`` steps replayed from captured HIP graphs.

    ``make_graph(count)`` captures a graph of ``count`` consecutive steps starting from the first
    input set (``per_graph`` steps make whole passes over the sets). Device timing: ``w`` warm-up
    steps, then one untimed lead-in replay of ``per_graph`` steps, then the ``k`` timed steps (whole
    ``per_graph`` graphs and one remainder graph) between two HIP events on the stream. The timed
    graphs are enqueued while the lead-in still runs, so no graph launch or host gap falls inside
    the timed region, whatever ``k``. Host timing: the same ``k`` steps from an idle stream,
    ``time.perf_counter`` around replay and synchronize (graph launch and sync included)."""
    graphs = {per_graph: make_graph(per_graph)}
    for count in (w, k):                              # every graph is captured before the timed region
        rem = count % per_graph
        if rem and rem not in graphs:
            graphs[rem] = make_graph(rem)

    def replay(count):
        for _ in range(count // per_graph):
            graphs[per_graph].replay()
        if count % per_graph:
            graphs[count % per_graph].replay()

    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    replay(w)
    graphs[per_graph].replay()                        # lead-in, untimed
    start.record()
    replay(k)
    stop.record()
    torch.cuda.synchronize()
    device_s = start.elapsed_time(stop) * 1e-3
    t0 = time.perf_counter()
    replay(k)
    torch.cuda.synchronize()
    return device_s, time.perf_counter() - t0


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


def cpu_oracle_layer(shape, seconds: float, fp8: bool) -> dict:
    """The oracle's five layer ops (numpy, one thread) on a bounded sample of the workload, timed on
    the host; reported beside the torch CPU baseline."""
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
    """The CPU baseline: the step's ops as torch CPU code on all of torch's host threads (the thread
    count is reported), on a bounded sample of the workload - the reference's math in torch (fp32
    from bf16, rounded once), the CPU path a user without the GPU kernels would run."""
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
            "kind": "port",
            "sample": f"{reps} passes of the step's ops as torch CPU code on {tokens} of {shape.tokens} tokens "
                      f"({dt:.1f} s, {torch.get_num_threads()} threads)",
            # average µs per call of each op on the sample's tokens
            "op_us": {key: round(1e6 * v / (reps * calls.get(key, 1)), 1) for key, v in op_s.items() if v > 0}}


class EmbeddingBench:
    """The token-embedding gather (devstral2.py:282) on the shape's tokens, cold: ``launches`` launches
    each gather ``tokens`` distinct rows of a ``[vocab, hidden]`` bf16 table (no row repeats within a
    replay, which touches more than the 256 MB Infinity Cache), writing the sets' output rows in turn.

    Also the step-input path (model_runner.py:135,149-154 + devstral2.py:282): each step's ids are
    refreshed from a pristine copy (standing in for the runner's one host-to-device transfer, which
    rewrites the placeholders every step), then either the reference's torch sequence
    (``fill_placeholders`` as written, then ``F.embedding``) or this library's one launch resolving the
    placeholders inside the gather."""

    def __init__(self, mas, shape, dev, launches: int = 512, seed: int = 0):
        self.mas = mas
        n, h, v = shape.tokens, shape.hidden, shape.vocab
        self.tokens, self.hidden, self.vocab = n, h, v
        self.launches = min(launches, v // n)
        g = torch.Generator(device=dev).manual_seed(seed)
        self.table = torch.randn(v, h, generator=g, device=dev).to(torch.bfloat16)
        cpu = torch.Generator().manual_seed(seed)
        rows = torch.randperm(v, generator=cpu)[: self.launches * n].view(self.launches, n)
        self.ids = rows.to(dev)
        self.outs = [torch.empty(n, h, dtype=torch.bfloat16, device=dev) for _ in range(min(self.launches, 50))]
        # decode steps: every id is a placeholder -1 - r for the previous step's sample r
        self.placeholders = (-1 - torch.arange(n, dtype=torch.int64)).to(dev)
        self.step_ids = [torch.empty(n, dtype=torch.int64, device=dev) for _ in range(self.launches)]
        self.last = [r.to(torch.int32) for r in self.ids]

    def credited(self) -> int:
        return 4 * self.tokens * self.hidden + 8 * self.tokens

    def launcher(self, op: str, i: int):
        mas, out = self.mas, self.outs[i % len(self.outs)]
        ids, step_ids, last, ph = self.ids[i], self.step_ids[i], self.last[i], self.placeholders
        if op == "embedding":
            return lambda: mas.embedding.embedding(ids, self.table, out=out)
        if op in ("skeleton:embedding", "skeleton64:embedding"):
            # the same bytes with no id lookup: rows i, i + stride, ... of the table, in workgroups of
            # 256 or 64 threads
            stride = (self.vocab // self.tokens) * self.table.stride(0)
            src = self.table[i % (self.vocab // self.tokens)]
            block = 64 if op.startswith("skeleton64:") else 256
            ptrs = (src.data_ptr(), stride, None, 0, out.data_ptr(), out.stride(0), None, 0, self.tokens, self.hidden,
                    block)

            def launch():
                st = _skeleton_fn(*ptrs, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
                if st != 0:
                    raise RuntimeError(f"embedding skeleton failed with status {st}")
            return launch
        if op == "step_input_reset":
            return lambda: step_ids.copy_(ph)
        if op == "step_input_reference":
            def reference():
                step_ids.copy_(ph)
                # ModelRunner.fill_placeholders (model_runner.py:149-154), then embed_tokens (devstral2.py:282)
                is_placeholder = step_ids < 0
                rows = (-1 - step_ids).clamp(min=0)
                sampled = last[rows]
                step_ids.copy_(torch.where(is_placeholder, sampled, step_ids))
                torch.nn.functional.embedding(step_ids, self.table)
            return reference
        if op == "step_input_fused":
            def fused():
                step_ids.copy_(ph)
                mas.embedding.embedding(step_ids, self.table, out=out, last_tokens=last)
            return fused
        raise ValueError(op)

    def time(self, ops, replays: int = 5) -> dict[str, float]:
        """Average µs per launch (per step for the step-input sequences), as ``time_ops``."""
        res = {}
        for op in ops:
            fns = [self.launcher(op, i) for i in range(self.launches)]

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
            times = sorted(a.elapsed_time(b) for a, b in events)
            res[op] = 1000.0 * times[len(times) // 2] / self.launches
            del g
        return res

    def report(self) -> tuple[dict, dict]:
        """(the embedding's ``ops`` entry, the step-input comparison)."""
        ops = ("embedding", "step_input_reset", "step_input_reference", "step_input_fused")
        if _skeleton_fn is not None:
            ops = ops + ("skeleton:embedding", "skeleton64:embedding")
        t = self.time(ops)
        cb = self.credited()
        entry = {"us": round(t["embedding"], 3), "GB/s": round(cb / t["embedding"] / 1e3, 1),
                 "frac": round(cb / t["embedding"] / 1e3 / PEAK_HBM_GBS, 4), "launches_per_replay": self.launches}
        if "skeleton:embedding" in t:
            sk, block = skeleton_best(t, "embedding")
            entry["skeleton_us"] = round(sk, 3)
            entry["skeleton_block"] = block
            entry["of_skeleton"] = round(sk / t["embedding"], 3)
        steps = {"ids_refresh_us": round(t["step_input_reset"], 3),
                 "reference_us": round(t["step_input_reference"], 3),
                 "fused_us": round(t["step_input_fused"], 3),
                 "what": "per step: ids refreshed (device copy), then the reference's fill_placeholders + "
                         "F.embedding (6 launches) or one placeholder-resolving gather; graph-replayed, cold rows"}
        return entry, steps


def layer_sets(mas, args, shape, dev) -> list:
    """The layer buffer sets a one-layer workload cycles: enough distinct sets (each with its own KV
    cache) that no step finds its data in the Infinity Cache (cold), or one (hot)."""
    wl, lp = mas.workloads, mas.layer_pass
    n_sets = 1 if args.protocol == "hot" else max(2, math.ceil(COLD_BYTES / footprint_bytes(shape)))
    if args.sets is not None and args.protocol != "hot":
        n_sets = args.sets
    table = mas.rope.cos_sin_cache(shape.max_position, shape.head_dim, shape.theta).to(dev)
    return [lp.LayerBuffers(wl.make_layer_inputs(shape, dev, seed=i, fill_on_device=True,
                                                 table=table.clone() if args.table_per_set else table,
                                                 zero_cache=False),
                            fp8=args.fp8, fuse_rope_kv=not args.separate_rope_kv) for i in range(n_sets)]


def op_launches(shape, n_sets: int) -> int:
    """Launches per graph when each kernel is timed alone (decode: at least 100 back to back)."""
    if shape.layers > 1:
        return shape.layers
    return max(2 * n_sets, 100) if shape.decode else 4 * n_sets


def timed_kernels(shape, fp8: bool) -> tuple[str, ...]:
    """The step's kernels followed by the memory skeletons of those that have one."""
    kernels = step_ops(shape, fp8)
    skeletons = tuple(f"{kind}:{op}" for op in kernels if op in SKELETON_OPS and shape.tokens <= 65535
                      for kind in ("skeleton", "skeleton64")) if _skeleton_fn is not None else ()
    return kernels + skeletons


def op_table(mas, shape, kernels: tuple[str, ...], op_us: dict) -> dict:
    """Per-kernel µs, credited GB/s and fraction of peak, with the memory skeleton's µs and
    `of_skeleton` (skeleton µs / kernel µs) where the skeleton was timed."""
    cb = mas.workloads.credited_bytes(shape)
    ops = {op: {"us": round(op_us[op], 3), "GB/s": round(cb[op] / op_us[op] / 1e3, 1),
                "frac": round(cb[op] / op_us[op] / 1e3 / PEAK_HBM_GBS, 4)} for op in kernels}
    for op in kernels:
        if f"skeleton:{op}" in op_us:
            sk, block = skeleton_best(op_us, op)
            ops[op]["skeleton_us"] = round(sk, 3)
            ops[op]["skeleton_block"] = block
            ops[op]["of_skeleton"] = round(sk / op_us[op], 3)
    return ops


def skeleton_best(op_us: dict, op: str) -> tuple[float, int]:
    """The faster of an op's two skeleton shapes (workgroups of 256 or 64 threads; neither is the
    faster one at every size) and its block size."""
    sk, block = op_us[f"skeleton:{op}"], 256
    if op_us.get(f"skeleton64:{op}", float("inf")) < sk:
        sk, block = op_us[f"skeleton64:{op}"], 64
    return sk, block


def run_layer_workload(mas, args, shape, dev) -> dict:
    wl, lp = mas.workloads, mas.layer_pass
    sets = layer_sets(mas, args, shape, dev)
    n_sets = len(sets)
    fused = not args.separate_rope_kv
    per_step = wl.layer_credited_bytes(shape, fused, args.fp8)
    steps = args.steps if args.steps is not None else (2000 if shape.decode else 40)
    warmup = args.warmup if args.warmup is not None else max(n_sets, steps // 10)

    def run_range(lo, hi):
        for i in range(lo, hi):
            lp.run_layer(sets[i % n_sets])

    def timed_steps(k: int, w: int) -> dict:
        per_graph = n_sets * max(1, math.ceil(50 / n_sets))
        return time_steps(run_range, k, w, lead=per_graph, per_graph=per_graph)

    timing = timed_steps(steps, warmup)
    elapsed = timing["device_s"]
    other_us = None
    if not shape.norm_only:
        # the other RoPE / KV form, for comparison (same buffers, same step count)
        for b in sets:
            b.fuse_rope_kv = not fused
        other_us = timed_steps(steps, warmup)["device_s"] / steps * 1e6
        for b in sets:
            b.fuse_rope_kv = fused

    # stream-launched steps (no graph), for comparison
    stream_steps = min(steps, 10 * n_sets) if shape.decode else min(steps, 4 * n_sets)
    torch.cuda.synchronize()
    s0 = time.perf_counter()
    run_range(0, stream_steps)
    torch.cuda.synchronize()
    stream_us = (time.perf_counter() - s0) / stream_steps * 1e6

    kernels = step_ops(shape, args.fp8)
    eager = eager_host_us(mas, sets, kernels) if shape.decode else None
    op_us = time_ops(mas, sets, op_launches(shape, n_sets), timed_kernels(shape, args.fp8))
    ops = op_table(mas, shape, kernels, op_us)
    cb = wl.credited_bytes(shape)
    step_inputs = None
    if shape.decode and not shape.norm_only:
        ops["embedding"], step_inputs = EmbeddingBench(mas, shape, dev).report()
    ms_per_step = elapsed / steps * 1e3
    dominant = step_ops(shape, args.fp8)[0 if shape.norm_only else 3]
    res = {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
           "value": per_step / (ms_per_step * 1e-3) / 1e9, "stream_us_per_step": stream_us, "ops": ops,
           "sets": n_sets, "dominant": dominant, "dominant_bytes": cb[dominant], "dominant_us": op_us[dominant],
           "graph_us_per_step": timing["graph_s"] / steps * 1e6, "host_us_per_step": timing["host_s"] / steps * 1e6,
           "step_inputs": step_inputs, "eager_host_us_per_call": eager}
    if other_us is not None:
        res["separate_us_per_layer" if fused else "fused_us_per_layer"] = other_us
    return res


def run_pass_workload(mas, args, shape, dev) -> dict:
    lp, wl = mas.layer_pass, mas.workloads
    passes = [lp.DecodePass(shape, dev, seed=0, fp8=args.fp8, fuse_rope_kv=not args.separate_rope_kv)]
    per_step = passes[0].credited_bytes()
    steps = args.steps if args.steps is not None else 20
    warmup = args.warmup if args.warmup is not None else 3
    timing = time_steps(lambda lo, hi: [passes[0].run() for _ in range(lo, hi)], steps, warmup, lead=1, per_graph=10)
    elapsed = timing["device_s"]
    ops_timed = step_ops(shape, args.fp8)
    op_us = time_ops(mas, passes[0].layers, op_launches(shape, 1), timed_kernels(shape, args.fp8))
    ops = op_table(mas, shape, ops_timed, op_us)
    cb = wl.credited_bytes(shape)
    ops["embedding"], step_inputs = EmbeddingBench(mas, shape, dev).report()
    ms_per_step = elapsed / steps * 1e3
    dominant = ops_timed[3]
    return {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
            "value": per_step / (ms_per_step * 1e-3) / 1e9, "ops": ops, "sets": 1, "dominant": dominant,
            "dominant_bytes": cb[dominant], "dominant_us": op_us[dominant],
            "us_per_layer": ms_per_step * 1e3 / shape.layers, "graph_us_per_step": timing["graph_s"] / steps * 1e6,
            "host_us_per_step": timing["host_s"] / steps * 1e6, "step_inputs": step_inputs}


def graph_call_us(call, calls: int) -> float:
    """Per-call µs of an attention call: HIP events around a graph of ``calls`` back-to-back calls,
    replayed once untimed, then the median of five timed replays."""
    gb = capture(lambda: [call() for _ in range(calls)])
    gb.replay()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
    for start, stop in events:
        start.record()
        gb.replay()
        stop.record()
    torch.cuda.synchronize()
    return 1000.0 * sorted(a.elapsed_time(b) for a, b in events)[2] / calls


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
    timing = time_steps(lambda lo, hi: [call() for _ in range(lo, hi)], steps, warmup, lead=4, per_graph=10)
    elapsed = timing["device_s"]
    call_us = graph_call_us(call, 10)
    ms_per_step = elapsed / steps * 1e3
    lens = inp.seq_lens.cpu()
    return {"steps": steps, "warmup": warmup, "ms_per_step": ms_per_step, "per_step_bytes": per_step,
            "value": per_step / (ms_per_step * 1e-3) / 1e9, "sets": 1, "dominant": "paged_decode_attention",
            "dominant_bytes": per_step, "dominant_us": call_us,
            "ops": {"paged_decode_attention": {"us": round(call_us, 3), "GB/s": round(per_step / call_us / 1e3, 1),
                                               "frac": round(per_step / call_us / 1e3 / PEAK_HBM_GBS, 4)}},
            "attention": {"mean_len": round(float(lens.float().mean()), 1), "longest": int(lens.max()),
                          "positions": int(lens.sum()), "kv_pages": inp.k_cache.shape[0]},
            "inputs": inp, "graph_us_per_step": timing["graph_s"] / steps * 1e6,
            "host_us_per_step": timing["host_s"] / steps * 1e6}


def context_main(mas, args, shape, dev) -> int:
    """Causal context attention: a step is one call; the value is TFLOP/s of algorithmic flops."""
    wl = mas.workloads
    inp = wl.make_context_inputs(shape, dev, seed=0)
    out = torch.empty_like(inp.q)
    flops = wl.context_flops(shape)
    scale = shape.head_dim ** -0.5
    ws = torch.empty(128 << 20, dtype=torch.uint8, device=dev)  # the reference's workspace (devstral2.py:35)

    def call():
        mas.attention.trtllm_batch_context_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), ws, inp.block_tables,
                                                         inp.seq_lens, inp.max_q_len, inp.max_kv_len, scale, 1.0,
                                                         inp.cu_seqlens_q.numel() - 1, inp.cu_seqlens_q, None, out=out)

    if args.pmc_probe:
        # 5 calls of the op and nothing else: a counter pass then sees only its dispatches
        for _ in range(5):
            call()
        torch.cuda.synchronize()
        print(json.dumps({"pmc_probe": "paged_context_attention", "launches": 5, "flops_per_launch": flops}),
              flush=True)
        return 0
    if args.trace_probe:
        call()
        print(json.dumps({"trace_probe": "ops", "workload": shape.name, "calls_per_graph": 4,
                          "event_us_per_call": round(graph_call_us(call, 4), 3)}), flush=True)
        return 0
    steps = args.steps if args.steps is not None else 20
    warmup = args.warmup if args.warmup is not None else 3
    call()
    timing = time_steps(lambda lo, hi: [call() for _ in range(lo, hi)], steps, warmup, lead=1, per_graph=4)
    elapsed = timing["device_s"]
    call_us = graph_call_us(call, 4)
    one_kernel_us = None
    if shape.graph_rows:
        # the same inputs with a workspace too small for any split: the one-kernel grid launch
        tiny = torch.empty(16, dtype=torch.uint8, device=dev)

        def one_kernel():
            mas.attention.trtllm_batch_context_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), tiny, inp.block_tables,
                                                             inp.seq_lens, inp.max_q_len, inp.max_kv_len, scale, 1.0,
                                                             inp.cu_seqlens_q.numel() - 1, inp.cu_seqlens_q, None,
                                                             out=out)
        one_kernel()
        one_kernel_us = graph_call_us(one_kernel, 4)
    ms_per_step = elapsed / steps * 1e3
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    kernel_tflops = flops / (call_us * 1e-6) / 1e12
    line = {
        "metric": METRIC, "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": steps,
        "warmup": warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": shape.name, "rows": shape.rows, "q_len": shape.q_len, "cached": shape.cached,
                   "q_heads": shape.q_heads, "kv_heads": shape.kv_heads, "head_dim": shape.head_dim,
                   "page_size": shape.page_size, "flops": flops, "launch": "hip-graph",
                   **({"graph_rows": shape.graph_rows, "max_q_len": inp.max_q_len, "max_kv_len": inp.max_kv_len}
                      if shape.graph_rows else {})},
        "us_per_call": round(ms_per_step * 1e3, 3), "graph_us_per_call": round(timing["graph_s"] / steps * 1e6, 3),
        "host_us_per_call": round(timing["host_s"] / steps * 1e6, 3),
        "ops": {"paged_context_attention": {"us": round(call_us, 3), "TFLOP/s": round(kernel_tflops, 1),
                                            "frac": round(kernel_tflops / PEAK_BF16_TFLOPS, 4),
                                            **({"one_kernel_us": round(one_kernel_us, 3)} if one_kernel_us else {})}},
        "roofline": roofline_entry(shape.name, "paged_context_attention", flops, call_us, bound="mfma"),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_torch_context(inp, args.cpu_seconds)
        line["cpu_oracle"] = cpu_oracle_context(inp, args.cpu_seconds / 2)
    print(json.dumps(line), flush=True)
    return 0


def _cpu_kv(inp):
    """The workload's caches on the host, as fp32 [pages * page_size, kv_heads, head_dim]."""
    s = inp.shape
    return (inp.k_cache.cpu().float().view(-1, s.kv_heads, s.head_dim),
            inp.v_cache.cpu().float().view(-1, s.kv_heads, s.head_dim))


def _cpu_rows(tables_row, n: int, page_size: int) -> torch.Tensor:
    """Cache rows of positions 0..n-1 through one block-table row."""
    p = torch.arange(n)
    return tables_row[p // page_size].long() * page_size + p % page_size


def cpu_torch_attention(inp, seconds: float) -> dict:
    """The CPU baseline for decode attention: each row's attention as torch CPU code in fp32 (keys and
    values gathered through its block table, grouped query heads batched per kv head) on all of
    torch's host threads, cycling over the workload's rows for about ``seconds``; credited bytes of
    the rows done per second."""
    s = inp.shape
    q = inp.q.cpu().float()
    kc, vc = _cpu_kv(inp)
    tables, lens = inp.block_tables.cpu(), inp.seq_lens.cpu()
    g = s.q_heads // s.kv_heads
    scale = s.head_dim ** -0.5
    done_bytes, rows, t0 = 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        b = rows % s.batch
        n = int(lens[b])
        idx = _cpu_rows(tables[b], n, s.page_size)
        k = kc[idx].permute(1, 2, 0)                                   # [Hk, D, n]
        v = vc[idx].permute(1, 0, 2)                                   # [Hk, n, D]
        p = torch.softmax((q[b].view(s.kv_heads, g, s.head_dim) @ k) * scale, dim=-1)
        (p @ v).to(torch.bfloat16)
        done_bytes += n * s.kv_heads * s.head_dim * 4 + 2 * s.q_heads * s.head_dim * 2 + 4 * (-(-n // s.page_size)) + 4
        rows += 1
    elapsed = time.perf_counter() - t0
    return {"value": round(done_bytes / elapsed / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{rows} rows of the workload's decode attention as torch CPU code, fp32 "
                                      f"({elapsed:.1f} s, {torch.get_num_threads()} threads)"}


def cpu_torch_context(inp, seconds: float) -> dict:
    """The CPU baseline for context attention: causal attention of the prompt rows' query tokens in
    blocks of 64 from each row's end (the longest reach first) as torch CPU code in fp32 on all of
    torch's host threads, cycling over the rows (and again from the first) for about ``seconds``;
    algorithmic flops done per second."""
    s = inp.shape
    kv_len = s.cached + s.q_len
    kc, vc = _cpu_kv(inp)
    q_all = inp.q.cpu().float()
    tables = inp.block_tables.cpu()
    g = s.q_heads // s.kv_heads
    scale = s.head_dim ** -0.5
    rows = []
    for r in range(s.rows):
        idx = _cpu_rows(tables[r], kv_len, s.page_size)
        rows.append((q_all[r * s.q_len:(r + 1) * s.q_len], kc[idx].permute(1, 2, 0), vc[idx].permute(1, 0, 2)))
    done, tokens, blocks, t0 = 0, 0, 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        q, k, v = rows[(blocks // -(-s.q_len // 64)) % s.rows]          # [tokens, Hq, D], [Hk, D, kv], [Hk, kv, D]
        hi = s.q_len - (blocks % -(-s.q_len // 64)) * 64
        lo = max(0, hi - 64)
        reach = s.cached + hi                                           # positions the block's last token sees
        qb = q[lo:hi].view(hi - lo, s.kv_heads, g, s.head_dim).permute(1, 2, 0, 3).reshape(s.kv_heads, -1, s.head_dim)
        sc = (qb @ k[:, :, :reach]) * scale                             # [Hk, g * tokens, reach]
        pos = s.cached + torch.arange(lo, hi).repeat(g)
        sc.masked_fill_(torch.arange(reach)[None, None, :] > pos[None, :, None], float("-inf"))
        (torch.softmax(sc, dim=-1) @ v[:, :reach]).to(torch.bfloat16)
        done += sum(s.cached + i + 1 for i in range(lo, hi)) * s.q_heads * s.head_dim * 4
        tokens += hi - lo
        blocks += 1
    elapsed = time.perf_counter() - t0
    return {"value": round(done / elapsed / 1e12, 6), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{tokens} query tokens of the workload's prompt rows, cycled (longest reach "
                                      f"first in each row) as torch CPU code, fp32 ({elapsed:.1f} s, "
                                      f"{torch.get_num_threads()} threads)"}


def cpu_oracle_context(inp, seconds: float) -> dict:
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


def cpu_oracle_attention(inp, seconds: float) -> dict:
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
    """Launches only what a counter pass needs: one kernel (``--pmc-op``; default the workload's
    dominant kernel, SiluAndMul or the norm for the norm-only case) 20 times across the cold layer
    sets, then 4 copies of 256 MiB."""
    wl, lp = mas.workloads, mas.layer_pass
    n_sets = max(2, math.ceil(COLD_BYTES / footprint_bytes(shape)))
    table = mas.rope.cos_sin_cache(shape.max_position, shape.head_dim, shape.theta).to(dev)
    sets = [lp.LayerBuffers(wl.make_layer_inputs(shape, dev, seed=i, fill_on_device=True, table=table,
                                                 zero_cache=False), fp8=args.fp8) for i in range(n_sets)]
    op = args.pmc_op or step_ops(shape, False)[0 if shape.norm_only else 3]
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


def trace_probe(mas, args, shape, dev) -> None:
    """Launches only what a kernel trace of the bench's own timing needs, so the trace's per-dispatch
    durations come from the same graphs the line's HIP-event figures do: ``ops`` - each kernel's
    graph of back-to-back launches (and its memory skeleton's), replayed once untimed and five
    times timed; ``steps`` - the stamped step graphs alone. Prints the HIP-event figures."""
    if shape.layers > 1:
        p = mas.layer_pass.DecodePass(shape, dev, seed=0, fp8=args.fp8, fuse_rope_kv=not args.separate_rope_kv)
        sets = p.layers

        def run_range(lo, hi):
            for _ in range(lo, hi):
                p.run()
        steps, warmup, lead, per_graph = args.steps or 20, args.warmup or 3, 1, 10
    else:
        sets = layer_sets(mas, args, shape, dev)

        def run_range(lo, hi):
            for i in range(lo, hi):
                mas.layer_pass.run_layer(sets[i % len(sets)])
        per_graph = len(sets) * max(1, math.ceil(50 / len(sets)))
        steps, warmup, lead = args.steps or (200 if shape.decode else 20), args.warmup or len(sets), per_graph
    out = {"trace_probe": args.trace_probe, "workload": shape.name, "layer_sets": len(sets)}
    if args.trace_probe == "ops":
        launches = op_launches(shape, len(sets))
        op_us = time_ops(mas, sets, launches, timed_kernels(shape, args.fp8))
        out.update({"launches_per_graph": launches, "replays": 6, "event_us": {k: round(v, 3) for k, v in op_us.items()}})
    else:
        timing = time_steps(run_range, steps, warmup, lead=lead, per_graph=per_graph)
        out.update({"steps": steps, "us_per_step": round(timing["device_s"] / steps * 1e6, 3)})
    print(json.dumps(out), flush=True)


def step_credited_bytes(fs) -> dict[str, int]:
    """Credited bytes of each kernel of a whole forward step (one launch; per layer for the layer
    ops): every mandatory input element read once and every output written once, index arrays and
    norm weights included, the cos/sin table and attention partials not."""
    ls, lay = fs.shape.layer, fs.layout
    n, d, h, i = fs.num_tokens, fs.num_decodes, ls.hidden, ls.inter
    hq, hk, dim, ps = ls.q_heads, ls.kv_heads, ls.head_dim, fs.shape.page_size
    lens = lay.seq_lens.long()
    dec_pages = int(((lens[:d] + ps - 1) // ps).sum())
    prompt_positions = sum(q + c for q, c in fs.shape.prompts)
    prompt_tokens = sum(q for q, _ in fs.shape.prompts)
    return {
        "embedding": n * (4 * h + 8),
        "norm_in": 7 * n * h + 2 * h,
        "rope_append": n * (4 * (hq + hk) * dim + 6 * hk * dim + 8),
        "decode_attention": (lay.decode_positions * hk * dim * 4 + d * hq * dim * 3 + dec_pages * 4 + d * 4
                             if d else 0),
        "context_attention": (prompt_positions * hk * dim * 4 + prompt_tokens * hq * dim * 3 + 8 * len(fs.shape.prompts)
                              if fs.shape.prompts else 0),
        "norm_post": 7 * n * h + 2 * h,
        "silu": 5 * n * i,
        "final_norm": 8 * n * h + 2 * h,
    }


def step_main(mas, args, shape, dev) -> int:
    """A whole forward step (embedding, every layer's kernels with its attention, final norm) in the
    reference's fp8 dataflow, graph-replayed; the value is credited bytes per second. Beside it, each
    kernel's µs per launch over the step's layers (a graph of back-to-back launches, one per layer)
    and its share of the step."""
    fs = mas.layer_pass.ForwardStep(shape, dev, seed=0)
    cb = step_credited_bytes(fs)
    layer_ops = [op for op in fs.LAYER_OPS if cb[op] > 0]
    per_step = cb["embedding"] + cb["final_norm"] + shape.layers * sum(cb[op] for op in layer_ops)
    steps = args.steps if args.steps is not None else 10
    warmup = args.warmup if args.warmup is not None else 2
    fs.run()
    torch.cuda.synchronize()

    def run_range(lo, hi):
        for _ in range(lo, hi):
            fs.run()

    if args.trace_probe == "steps":
        timing = time_steps(run_range, steps, warmup, lead=1, per_graph=2)
        print(json.dumps({"trace_probe": "steps", "workload": shape.name, "steps": steps,
                          "us_per_step": round(timing["device_s"] / steps * 1e6, 3)}), flush=True)
        return 0

    def per_launch_us(fn, launches) -> float:
        g = capture(lambda: [fn(x) for x in launches])
        g.replay()
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        for start, stop in events:
            start.record()
            g.replay()
            stop.record()
        torch.cuda.synchronize()
        return 1000.0 * sorted(a.elapsed_time(b) for a, b in events)[2] / len(launches)

    op_us = {op: per_launch_us(getattr(fs, "run_" + op), fs.layers) for op in layer_ops}
    op_us["embedding"] = per_launch_us(lambda _: fs.run_embedding(), range(shape.layers))
    op_us["final_norm"] = per_launch_us(lambda _: fs.run_final_norm(), range(shape.layers))
    if args.trace_probe == "ops":
        print(json.dumps({"trace_probe": "ops", "workload": shape.name, "launches_per_graph": shape.layers,
                          "event_us": {k: round(v, 3) for k, v in op_us.items()}}), flush=True)
        return 0
    timing = time_steps(run_range, steps, warmup, lead=1, per_graph=2)
    ms_per_step = timing["device_s"] / steps * 1e3
    step_us = ms_per_step * 1e3
    ops = {}
    for op, us in op_us.items():
        count = shape.layers if op in layer_ops else 1
        ops[op] = {"us": round(us, 3), "launches": count, "us_per_step": round(us * count, 1),
                   "share": round(us * count / step_us, 4), "GB/s": round(cb[op] / us / 1e3, 1),
                   "frac": round(cb[op] / us / 1e3 / PEAK_HBM_GBS, 4)}
    value = per_step / (ms_per_step * 1e-3) / 1e9
    ls = shape.layer
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_per_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic",
        "config": {"workload": shape.name, "tokens": fs.num_tokens, "decode_rows": fs.num_decodes,
                   "decode_positions": fs.layout.decode_positions, "prompts": [list(p) for p in shape.prompts],
                   "prefill_rows": fs.num_prefills, "layers": shape.layers, "hidden": ls.hidden,
                   "intermediate": ls.inter, "q_heads": ls.q_heads, "kv_heads": ls.kv_heads, "head_dim": ls.head_dim,
                   "page_size": shape.page_size, "block_table_width": shape.reach // shape.page_size,
                   "kv_pages_per_layer": fs.layout.pages, "launch": "hip-graph", "dataflow": "fp8",
                   "gemms": "N(0,1) stand-in outputs"},
        "us_per_layer": round(step_us / shape.layers, 3), "frac_of_peak": round(value / PEAK_HBM_GBS, 4),
        "credited_bytes_per_step": per_step, "ops": ops,
        "ops_sum_us": round(sum(o["us_per_step"] for o in ops.values()), 1),
        "graph_us_per_step": round(timing["graph_s"] / steps * 1e6, 3),
        "host_us_per_step": round(timing["host_s"] / steps * 1e6, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


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
    if args.workload in mas.workloads.STEP_SHAPES:
        return step_main(mas, args, mas.workloads.STEP_SHAPES[args.workload], dev)
    shape = mas.workloads.SHAPES[args.workload]
    if args.pmc_probe:
        pmc_probe(mas, args, shape, dev)
        return 0
    if args.trace_probe:
        trace_probe(mas, args, shape, dev)
        return 0
    if shape.layers > 1:
        res = run_pass_workload(mas, args, shape, dev)
    else:
        res = run_layer_workload(mas, args, shape, dev)

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
        "roofline": roofline_entry(shape.name, res["dominant"], res["dominant_bytes"], res["dominant_us"]),
    }
    dom = res["ops"].get(res["dominant"], {})
    if "skeleton_us" in dom:
        # the same bytes, buffers and launch shape moved by a kernel with no arithmetic, same run
        sk_gbs = res["dominant_bytes"] / dom["skeleton_us"] / 1e3
        line["roofline"]["skeleton"] = {"us": dom["skeleton_us"], "GB/s": round(sk_gbs, 1),
                                        "frac": round(sk_gbs / PEAK_HBM_GBS, 4)}
        line["roofline"]["frac_of_skeleton"] = dom["of_skeleton"]
    for key in ("separate_us_per_layer", "fused_us_per_layer", "stream_us_per_step", "graph_us_per_step",
                "host_us_per_step"):
        if key in res:
            line[key] = round(res[key], 3)
    if res.get("step_inputs"):
        line["step_inputs"] = res["step_inputs"]
    if res.get("eager_host_us_per_call"):
        line["eager_host_us_per_call"] = res["eager_host_us_per_call"]
    line["copy_ceiling_GBps"] = round(copy_ceiling_gbs(dev), 1)
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_torch_layer(shape, args.cpu_seconds, args.fp8)
        line["cpu_oracle"] = cpu_oracle_layer(shape, args.cpu_seconds / 2, args.fp8)
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
    if args.trace_probe:
        wl = mas.workloads
        inp = wl.make_attention_inputs(shape, dev, seed=0)
        out = torch.empty_like(inp.q)

        def call():
            mas.attention.trtllm_batch_decode_with_kv_cache(inp.q, (inp.k_cache, inp.v_cache), inp.workspace,
                                                            inp.block_tables, inp.seq_lens, 0,
                                                            shape.head_dim ** -0.5, 1.0, out=out)
        call()
        print(json.dumps({"trace_probe": "ops", "workload": shape.name, "calls_per_graph": 10,
                          "event_us_per_call": round(graph_call_us(call, 10), 3)}), flush=True)
        return 0
    res = run_attention_workload(mas, args, shape, dev)
    line = {
        "metric": METRIC, "value": round(res["value"], 2), "unit": "GB/s", "n_gpus": 1, "steps": res["steps"],
        "warmup": res["warmup"], "ms_per_step": round(res["ms_per_step"], 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": shape.name, "batch": shape.batch, "q_heads": shape.q_heads,
                   "kv_heads": shape.kv_heads, "head_dim": shape.head_dim, "page_size": shape.page_size,
                   "max_len": shape.max_len, **res["attention"], "launch": "hip-graph"},
        "us_per_call": round(res["ms_per_step"] * 1e3, 3),
        "graph_us_per_call": round(res["graph_us_per_step"], 3), "host_us_per_call": round(res["host_us_per_step"], 3),
        "frac_of_peak": round(res["value"] / PEAK_HBM_GBS, 4),
        "ops": res["ops"],
        "roofline": roofline_entry(shape.name, res["dominant"], res["dominant_bytes"], res["dominant_us"]),
        "copy_ceiling_GBps": round(copy_ceiling_gbs(dev), 1),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_torch_attention(res["inputs"], args.cpu_seconds)
        line["cpu_oracle"] = cpu_oracle_attention(res["inputs"], args.cpu_seconds / 2)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
