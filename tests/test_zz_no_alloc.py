"""The allocation-free decode attention entry point (mas_paged_decode_attention_bf16_noalloc),
called through the C ABI, against the workspace entry point on the same inputs.

With a workspace of exactly the static scratch's size, both entry points pick the same splits and
run the same kernels, so the outputs must match bit for bit. Two calls in a row, the second on a
smaller input, check that the shared scratch carries nothing between calls; a call too large for
the scratch must be rejected with MAS_ERR_SCRATCH before anything is enqueued.
"""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20          # MAS_DECODE_ATTENTION_SCRATCH_BYTES
MAS_ERR_SCRATCH = -5
MAS_ERR_NOT_READY = -6


def _inputs(dev, batch, hq, hk, d, page_size, max_len, seed):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, max_len + 1, (batch,), generator=g)
    width = -(-max_len // page_size)
    pages = batch * width + 1
    tables = torch.randperm(pages, generator=g)[: batch * width].reshape(batch, width).to(torch.int32)
    dg = torch.Generator(device=dev).manual_seed(seed)
    kv = (pages, page_size, hk, d)
    return (torch.randn(batch, hq, d, generator=dg, device=dev).bfloat16(),
            torch.randn(kv, generator=dg, device=dev).bfloat16(), torch.randn(kv, generator=dg, device=dev).bfloat16(),
            tables.to(dev), lens.to(torch.int32).to(dev))


def _call(lib, noalloc, q, kc, vc, tables, lens, out, ws=None, err=None):
    b, hq, d = q.shape
    args = [out.data_ptr(), out.stride(0), out.stride(1), q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(),
            vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), kc.shape[0], kc.shape[1], tables.data_ptr(),
            tables.stride(0), tables.shape[1], lens.data_ptr(), b, hq, kc.shape[2], d, d ** -0.5, 1.0, 0, None, 0.0]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        return lib.mas_paged_decode_attention_bf16_noalloc(*args, err, stream)
    return lib.mas_paged_decode_attention_bf16(*args, ws.data_ptr(), ws.numel(), err, stream)


@pytest.mark.parametrize("shape", [
    # (batch, q heads, kv heads, head_dim, page_size, max_len): the second of each pair is smaller
    ((64, 32, 8, 128, 256, 8192), (16, 32, 8, 128, 256, 2048)),
    ((8, 96, 8, 128, 16, 4096), (3, 96, 8, 128, 16, 700)),
])
def test_noalloc_matches_workspace_entry_point(mas, dev, shape):
    lib = mas._lib.load()
    ws = torch.empty(SCRATCH_BYTES, dtype=torch.uint8, device=dev)
    for i, s in enumerate(shape):
        q, kc, vc, tables, lens = _inputs(dev, *s, seed=10 + i)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        assert _call(lib, False, q, kc, vc, tables, lens, want, ws) == 0
        assert _call(lib, True, q, kc, vc, tables, lens, got) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"call {i} ({s})"


def test_noalloc_rejects_calls_beyond_its_scratch(mas, dev):
    lib = mas._lib.load()
    # one split per row needs batch * hq * (d + 2) * 4 bytes: 1024 * 128 * 130 * 4 > 64 MiB
    q, kc, vc, tables, lens = _inputs(dev, 1024, 128, 8, 128, 256, 256, seed=3)
    out = torch.zeros_like(q)
    assert _call(lib, True, q, kc, vc, tables, lens, out) == MAS_ERR_SCRATCH
    torch.cuda.synchronize()
    assert not out.any()
    assert "no-allocation" in lib.mas_status_string(MAS_ERR_SCRATCH).decode()


def test_noalloc_through_the_wrapper_and_a_graph(mas, dev):
    """workspace_buffer=None selects the entry point; captured in a graph, replays match eager."""
    q, kc, vc, tables, lens = _inputs(dev, 16, 32, 8, 128, 256, 3000, seed=5)
    want = mas.attention.trtllm_batch_decode_with_kv_cache(q, (kc, vc), torch.empty(SCRATCH_BYTES, dtype=torch.uint8,
                                                           device=dev), tables, lens, 0, 128 ** -0.5, 1.0)
    out = torch.empty_like(q)
    mas.attention.trtllm_batch_decode_with_kv_cache(q, (kc, vc), None, tables, lens, 0, 128 ** -0.5, 1.0, out=out)
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        mas.attention.trtllm_batch_decode_with_kv_cache(q, (kc, vc), None, tables, lens, 0, 128 ** -0.5, 1.0, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want)


_FIRST_CALL_UNDER_CAPTURE = r"""
import json, sys
import torch
sys.path.insert(0, sys.argv[1])
sys.path.insert(0, sys.argv[1] + "/tests")
import __graft_entry__
from test_zz_no_alloc import _call, _inputs
mas = __graft_entry__.load_package()
lib = mas._lib.load()
dev = torch.device("cuda:0")
q, kc, vc, tables, lens = _inputs(dev, 8, 32, 8, 128, 256, 2000, seed=7)
want = torch.empty_like(q)
ws = torch.empty(64 << 20, dtype=torch.uint8, device=dev)
assert _call(lib, False, q, kc, vc, tables, lens, want, ws) == 0
out = torch.zeros_like(q)
torch.cuda.synchronize()
codes = []
g0 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g0):           # the entry point's first call in this process, under capture
    codes.append(_call(lib, True, q, kc, vc, tables, lens, out))
torch.cuda.synchronize()
untouched = not out.any().item()
codes.append(_call(lib, True, q, kc, vc, tables, lens, out))      # outside capture: sets up the scratch
torch.cuda.synchronize()
eager_ok = torch.equal(out, want)
out.zero_()
g1 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g1):
    codes.append(_call(lib, True, q, kc, vc, tables, lens, out))
replays_ok = []
for _ in range(2):
    out.zero_()
    torch.cuda.synchronize()
    g1.replay()
    torch.cuda.synchronize()
    replays_ok.append(torch.equal(out, want))
print(json.dumps({"codes": codes, "untouched": untouched, "eager_ok": eager_ok, "replays_ok": replays_ok,
                  "text": lib.mas_status_string(codes[0]).decode()}))
"""


def test_noalloc_first_call_under_capture_in_a_fresh_process(mas, dev):
    """In a process that has not called the entry point yet, a first call under graph capture is
    rejected with MAS_ERR_NOT_READY and enqueues nothing; one eager call sets the scratch up, after
    which a captured call works and its replays match the workspace entry point."""
    import json
    import subprocess
    import sys
    from conftest import ROOT
    proc = subprocess.run([sys.executable, "-c", _FIRST_CALL_UNDER_CAPTURE, str(ROOT)], capture_output=True,
                          text=True, timeout=300)
    assert proc.returncode == 0, proc.stderr[-2000:]
    res = json.loads(proc.stdout.strip().splitlines()[-1])
    assert res["codes"] == [MAS_ERR_NOT_READY, 0, 0], res
    assert res["untouched"] and res["eager_ok"] and all(res["replays_ok"]), res
    assert "outside capture" in res["text"]
