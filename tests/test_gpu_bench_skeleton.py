"""The benchmark's memory skeletons (libmas_bench.so) move exactly the streams they stand for: the
ceilings bench.py reports beside each kernel are only honest if the skeleton really reads and writes
those bytes."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from conftest import bits

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def skeleton(mas):
    if not mas._build.BENCH_LIBRARY_PATH.exists():
        pytest.fail("libmas_bench.so is not built (run __graft_entry__.build())")
    fn = ctypes.CDLL(str(mas._build.BENCH_LIBRARY_PATH)).mas_bench_stream_skeleton
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_void_p]

    def run(src0, src1, dst0, dst1, rows, elems, block=256):
        args = []
        for t in (src0, src1, dst0, dst1):
            args += [t.data_ptr() if t is not None else None, t.stride(0) if t is not None else 0]
        st = fn(*args, rows, elems, block, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        return st
    return run


def _rand(rows, cols, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(rows, cols, generator=g, device=dev).bfloat16()


@pytest.mark.parametrize("block", [64, 256])
def test_copy_moves_each_row_and_nothing_else(skeleton, dev, block):
    src = _rand(70, 48 * 16, dev, 1)
    dst = torch.zeros(70, 64 * 16, dtype=torch.bfloat16, device=dev)
    assert skeleton(src, None, dst, None, 70, 40 * 16, block) == 0
    assert np.array_equal(bits(dst[:, :640]), bits(src[:, :640]))
    assert not bits(dst[:, 640:]).any()


@pytest.mark.parametrize("block", [64, 256])
def test_pairwise_copy_in_place_and_to_other_buffers(skeleton, dev, block):
    a, b = _rand(9, 1024, dev, 2), _rand(9, 1024, dev, 3)
    a0, b0 = a.clone(), b.clone()
    assert skeleton(a, b, a, b, 9, 1024, block) == 0     # the norm's in-place mix: unchanged
    assert np.array_equal(bits(a), bits(a0)) and np.array_equal(bits(b), bits(b0))
    x, y = torch.zeros_like(a), torch.zeros_like(b)
    assert skeleton(a, b, x, y, 9, 1024, block) == 0
    assert np.array_equal(bits(x), bits(a0)) and np.array_equal(bits(y), bits(b0))


@pytest.mark.parametrize("block", [64, 256])
def test_two_sources_to_one_destination_reads_both(skeleton, dev, block):
    gate_up = _rand(33, 2 * 2048, dev, 4)
    out = torch.zeros(33, 2048, dtype=torch.bfloat16, device=dev)
    assert skeleton(gate_up, gate_up[:, 2048:], out, None, 33, 2048, block) == 0
    expect = bits(gate_up[:, :2048]) ^ bits(gate_up[:, 2048:])
    assert np.array_equal(bits(out), expect)


def test_rejects_what_it_cannot_launch(skeleton, dev):
    src = _rand(4, 16, dev, 5)
    dst = torch.zeros(4, 16, dtype=torch.bfloat16, device=dev)
    assert skeleton(src, None, dst, None, 4, 12) != 0      # not a whole number of 16-byte vectors
    assert skeleton(src, None, dst, None, 65536, 16) != 0  # more rows than one grid column holds
    assert skeleton(src, None, dst, None, 4, 16, 128) != 0  # workgroups of 64 or 256 threads only
