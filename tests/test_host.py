"""Host-side checks that need no GPU: the C-ABI library loads and exports every entry point that
include/mas_kernels.h declares, status reporting, argument validation (raised before anything is
enqueued), the torch.library registrations and their fake kernels, and the golden fixtures."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import GOLDEN_DIR, ROOT

HEADER = ROOT / "include" / "mas_kernels.h"


def declared_entry_points() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:int64_t|int|const char\s*\*)\s+(mas_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_bound_entry_points(mas):
    declared = declared_entry_points()
    assert len(declared) >= 9
    assert sorted(declared) == sorted(mas._lib.exported_symbols())


def test_library_loads_and_exports_every_declared_symbol(mas):
    lib = mas.load_library()
    raw = ctypes.CDLL(str(mas._build.LIBRARY_PATH))
    for name in declared_entry_points():
        assert hasattr(raw, name), f"{name} not exported"
        assert getattr(lib, name) is not None


def test_benchmark_skeletons_live_in_their_own_library(mas):
    kernels = ctypes.CDLL(str(mas._build.LIBRARY_PATH))
    assert not hasattr(kernels, "mas_bench_stream_skeleton")
    if not mas._build.BENCH_LIBRARY_PATH.exists():
        pytest.skip("libmas_bench.so not built")
    fn = ctypes.CDLL(str(mas._build.BENCH_LIBRARY_PATH)).mas_bench_stream_skeleton
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    assert fn(None, 0, None, 0, None, 0, None, 0, 0, 8, 256, None) == 0          # empty: nothing launched
    assert fn(None, 0, None, 0, None, 0, None, 0, 0, 8, 64, None) == 0
    assert fn(16, 8, None, 0, 32, 8, None, 0, 70000, 8, 256, None) == -1        # rows past one grid row each
    assert fn(16, 8, None, 0, 32, 8, 48, 8, 4, 8, 256, None) == -1              # two destinations, one source
    assert fn(16, 8, None, 0, 40, 8, None, 0, 4, 8, 256, None) == -1            # misaligned destination
    assert fn(16, 8, None, 0, 32, 8, None, 0, 4, 8, 128, None) == -1            # neither 64 nor 256 threads


def test_context_workspace_bytes(mas):
    """Bytes for 32 splits' fp32 partials, (head_dim + 2) floats per (row, token slot, head, split),
    the token slots rounded up to whole token tiles: 32 tokens per wavefront of a workgroup of four
    (eight for 8+ query heads per kv head) wavefronts shared among up to 4 heads."""
    f = mas.attention.context_workspace_bytes
    # one head per kv head: 4 wavefronts x 32 tokens = 128-token tiles; 40 tokens -> one tile
    assert f(1, 40, 8, 8, 128) == 128 * 8 * 32 * 130 * 4
    assert f(1, 128, 8, 8, 128) == f(1, 40, 8, 8, 128)
    assert f(1, 129, 8, 8, 128) == 2 * f(1, 128, 8, 8, 128)
    # 4 heads per kv head share a workgroup: 32-token tiles
    assert f(3, 33, 32, 8, 128) == 3 * 64 * 32 * 32 * 130 * 4
    # 12 per kv head (eight wavefronts, 4 heads each): 64-token tiles; head_dim 64
    assert f(1, 64, 96, 8, 64) == 64 * 96 * 32 * 66 * 4
    assert f(0, 64, 96, 8, 64) == 0
    for bad in ((1, 64, 96, 7, 128), (1, 64, 32, 8, 256), (-1, 64, 32, 8, 128), (1, 64, 32, 0, 128)):
        with pytest.raises(ValueError):
            f(*bad)


def test_fused_rope_append_rejects_an_empty_table(mas):
    """Every token's table row is loaded before its position is judged, so an empty table is an
    argument error (returned before anything is enqueued) rather than a per-token error bit."""
    fn = mas.load_library().mas_rope_append_paged_kv_cache_bf16
    p = 256                                     # any non-null address: nothing is dereferenced

    def call(table_rows, rows):
        return fn(p, 128, 128, 1, p, 128, 128, p, 128, 128, 1, p, p, 128, table_rows, rows, 128, 1,
                  p, p, 16 * 128, 128, 128, 4, 16, p, p, 4, p, 1, None, 0, 0, p, None)
    assert call(0, 3) == -1
    assert call(0, 0) == 0                      # nothing to do: not an error
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():                      # the wrapper says so before the library is called
        cuda = dict(device="cuda")
        qkv = torch.empty(3, 6 * 128, dtype=torch.bfloat16, **cuda)
        cache = torch.empty(4, 16, 2, 128, dtype=torch.bfloat16, **cuda)
        i32 = torch.zeros(3, dtype=torch.int32, **cuda)
        with pytest.raises(ValueError, match="cos_sin_cache has no rows"):
            mas.fused.apply_rope_and_append_paged_kv_cache(
                i32, qkv[:, :256], qkv[:, 256:512], qkv[:, 512:], 128, torch.empty(0, 128, **cuda), True, i32,
                (cache, cache.clone()), torch.zeros(4, dtype=torch.int32, **cuda), torch.zeros(2, dtype=torch.int32,
                                                                                               **cuda))


def test_library_links_against_one_hip_runtime(mas):
    mas.load_library()
    maps = Path("/proc/self/maps").read_text()
    runtimes = set(re.findall(r"\S*libamdhip64\S*", maps))
    assert len(runtimes) == 1, runtimes


def test_status_strings_and_version(mas):
    lib = mas.load_library()
    assert lib.mas_status_string(0) == b"ok"
    assert b"unsupported" in lib.mas_status_string(-2)
    assert b"alignment" in lib.mas_status_string(-3)
    assert mas.library_version() == (0, 1, 0)
    with pytest.raises(mas._lib.KernelError, match="status -1"):
        mas._lib.check(-1, "op")
    assert mas._lib.describe_error_bits(1 | 8) == "token id outside [0, vocab); " \
                                                 "page slot past kv_indices or page id outside the cache"


def test_rows_view(mas):
    from mini_agent_serve_amd._tensors import rows_view
    t = torch.empty(6, 10)
    assert rows_view(t, "t") == (6, 10)
    assert rows_view(torch.empty(4, 3, 10), "t") == (12, 10)
    qkv = torch.empty(5, 24)
    assert rows_view(qkv[:, 8:16], "q") == (5, 24)
    assert rows_view(torch.empty(1, 1, 7), "t") == (1, 7)
    assert rows_view(torch.empty(4, 1, 7).as_strided((4, 1, 7), (7, 99, 1)), "t") == (4, 7)
    with pytest.raises(ValueError, match="contiguous in its last dimension"):
        rows_view(torch.empty(10, 6).t(), "t")
    assert rows_view(torch.empty(3, 4, 8)[:, ::2], "t") == (6, 16)     # every other row: one stride
    with pytest.raises(ValueError, match="one row index"):
        rows_view(torch.empty(3, 4, 8)[:, :2], "t")


def test_rows_view_against_brute_force(mas):
    """Random shapes and strides: rows_view accepts exactly the layouts whose rows, enumerated in
    row-major order of the leading dimensions, start at r * row_stride, and returns that stride."""
    import itertools
    import random
    from mini_agent_serve_amd._tensors import rows_view
    rng = random.Random(7)
    storage = torch.empty(1 << 16)
    checked = rejected = 0
    for _ in range(3000):
        nd = rng.randint(1, 4)
        shape = [rng.choice([1, 1, 2, 3, 4]) for _ in range(nd - 1)] + [rng.choice([1, 2, 5, 8])]
        strides = [rng.choice([0, 1, 3, 8, 16, 40, 64, 99]) for _ in range(nd - 1)] + [rng.choice([1, 1, 1, 2])]
        t = storage.as_strided(shape, strides)
        w = shape[-1]
        offsets = [sum(i * s for i, s in zip(idx, strides[:-1]))
                   for idx in itertools.product(*[range(n) for n in shape[:-1]])]
        rows = len(offsets)
        if w > 1 and strides[-1] != 1:
            want = None
        elif rows == 1:
            want = (1, max(w, 1))
        else:
            step = offsets[1] - offsets[0]
            want = (rows, step) if all(o == r * step + offsets[0] for r, o in enumerate(offsets)) else None
        if want is None:
            with pytest.raises(ValueError):
                rows_view(t, "t")
            rejected += 1
        else:
            assert rows_view(t, "t") == want, (shape, strides)
            checked += 1
    assert checked > 500 and rejected > 500


def test_device_checks_compare_device_indices(mas):
    from torch._subclasses.fake_tensor import FakeTensorMode
    from mini_agent_serve_amd._tensors import require_gpu, require_same_device
    a, b = torch.empty(2), torch.empty(3)
    assert require_same_device(("a", a), ("b", b)) == torch.device("cpu")
    with pytest.raises(ValueError, match="GPU"):
        require_gpu(a, "a")
    with pytest.raises(TypeError, match="torch.Tensor"):
        require_gpu([1, 2], "a")
    class OnOtherGpu:
        """Stands for a tensor on a second GPU, which a one-GPU machine cannot make even as a fake
        tensor: what the check reads of a tensor."""
        device, is_cuda = torch.device("cuda", 1), True

        def get_device(self):
            return 1

    with FakeTensorMode():
        g0 = torch.empty(2, device="cuda:0")
        g1 = OnOtherGpu()
        require_gpu(g0, "g0")
        assert require_same_device(("x", g0), ("y", torch.empty(5, device="cuda:0"))) == torch.device("cuda:0")
        with pytest.raises(ValueError, match="y is on cuda:1"):
            require_same_device(("x", g0), ("y", g1))
        with pytest.raises(ValueError, match="y is on cpu"):
            require_same_device(("x", g0), ("y", a))


def test_arguments_are_validated_before_launch(mas):
    cpu = torch.zeros(4, 64, dtype=torch.bfloat16)
    w = torch.ones(64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        mas.fused_add_rmsnorm(cpu, cpu.clone(), w)
    with pytest.raises(ValueError, match="GPU"):
        mas.silu_and_mul(cpu)
    with pytest.raises(ValueError, match="GPU"):
        mas.embedding.embedding(torch.zeros(3, dtype=torch.int64), cpu)
    with pytest.raises(ValueError, match="GPU"):
        mas.apply_rope_with_cos_sin_cache_inplace(torch.zeros(4, dtype=torch.int32), cpu, cpu, 64,
                                                  torch.zeros(8, 64))
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():                      # GPU-device tensors without a GPU: checks run, nothing launches
        h = torch.empty(4, 64, dtype=torch.bfloat16, device="cuda")
        wd = torch.empty(64, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(TypeError, match="bfloat16"):
            mas.fused_add_rmsnorm(h.float(), h.float(), wd)
        with pytest.raises(ValueError, match="weight must be a contiguous"):
            mas.fused_add_rmsnorm(h, h.clone(), torch.empty(32, dtype=torch.bfloat16, device="cuda"))
        with pytest.raises(ValueError, match="even"):
            mas.silu_and_mul(torch.empty(4, 63, dtype=torch.bfloat16, device="cuda"))
        with pytest.raises(ValueError, match="rotary_dim"):
            mas.apply_rope_with_cos_sin_cache_inplace(torch.empty(4, dtype=torch.int32, device="cuda"), h, h, 64,
                                                      torch.empty(8, 48, device="cuda"))
        with pytest.raises(ValueError, match="kv_layout"):
            mas.append_paged_kv_cache(h, h, None, None, (h, h), None, None, None, "NDH")
        with pytest.raises(TypeError, match="int64"):
            mas.embedding.embedding(torch.empty(3, dtype=torch.int32, device="cuda"), h)


def test_fake_kernels_under_fake_tensor_mode(mas):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(7, 2 * 96, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.mas.silu_and_mul(x).shape == (7, 96)
        ids = torch.empty(2, 5, dtype=torch.int64, device="cuda")
        table = torch.empty(10, 32, dtype=torch.bfloat16, device="cuda")
        assert torch.ops.mas.embedding(ids, table, None).shape == (2, 5, 32)
        h = torch.empty(3, 64, dtype=torch.bfloat16, device="cuda")
        torch.ops.mas.fused_add_rmsnorm(h, h.clone(), torch.empty(64, dtype=torch.bfloat16, device="cuda"), 1e-6)
    expected = {"fused_add_rmsnorm", "fused_add_rmsnorm_quant", "fused_add_rmsnorm_quant_hs", "silu_and_mul",
                "silu_and_mul_out", "apply_rope_with_cos_sin_cache_inplace", "append_paged_kv_cache",
                "store_kv_slots", "embedding", "embedding_out", "embedding_fill_placeholders",
                "embedding_fill_placeholders_out", "fill_placeholders", "silu_and_mul_quant", "silu_and_mul_quant_hs",
                "apply_rope_and_append_paged_kv_cache", "paged_decode_attention", "paged_context_attention"}
    assert expected <= {name for name in dir(torch.ops.mas) if not name.startswith("_")}


def test_golden_fixtures_reproduce():
    """The committed fixtures are what the oracle computes today."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_golden", GOLDEN_DIR / "gen_golden.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    fresh = gen.build()
    stored = np.load(GOLDEN_DIR / "layer_ops.npz")
    assert set(stored.files) == set(fresh)
    for key in stored.files:
        assert np.array_equal(stored[key], fresh[key]), key


def test_graph_context_workload_layout(mas):
    """The bench's graph-step context workloads follow the reference runner's layout
    (model_runner.py:155-221): 17 prompt rows, the real prompts first, then one padding row holding
    the padding tokens (the step's token count rounded up to 64; its kv_len their count, every
    block-table entry the sink page) and empty rows (seq_len 1, the sink in column 0); max_q_len the
    padded token count, max_kv_len the table's reach."""
    inp = mas.workloads.make_context_inputs("context_attn_graph_3x100_after2000_24b")
    s = inp.shape
    cu, seq, tables = inp.cu_seqlens_q.tolist(), inp.seq_lens.tolist(), inp.block_tables
    assert len(seq) == 17 and len(cu) == 18 and tables.shape == (17, 8192 // 16)
    assert cu[:4] == [0, 100, 200, 300] and cu[4:] == [320] * 14
    assert seq[:3] == [2100] * 3 and seq[3] == 20 and seq[4:] == [1] * 13
    assert (inp.max_q_len, inp.max_kv_len) == (320, 8192) and inp.q.shape == (320, s.q_heads, s.head_dim)
    sink = inp.k_cache.shape[0] - 1
    width = -(-2100 // 16)
    real = tables[:3, :width]
    assert int(real.min()) >= 0 and int(real.max()) < sink and real.unique().numel() == real.numel()
    assert torch.all(tables[3] == sink) and torch.all(tables[4:, 0] == sink)
    assert mas.workloads.context_flops(s) == 3 * sum(2000 + i + 1 for i in range(100)) * 32 * 128 * 4


# ---- the bench line's profiled figures --------------------------------------------------------------

def _bench():
    import sys
    sys.path.insert(0, str(ROOT))
    import bench
    return bench


def test_source_blob_is_git_hash_object():
    """The staleness check hashes a source as `git hash-object` does: sha1 of "blob <size>\\0" + bytes."""
    import hashlib
    bench = _bench()
    rel = "csrc/silu_and_mul.hip"
    data = (ROOT / "mini-agent-serve_amd" / rel).read_bytes()
    want = hashlib.sha1(b"blob " + str(len(data)).encode() + b"\0" + data).hexdigest()
    assert bench.source_blob(rel) == want


def test_roofline_follows_a_fresh_trace_and_flags_a_stale_one(monkeypatch):
    """With its sources unchanged, the roofline's rate and frac come from the committed trace; with
    a source hash that no longer matches, from the live HIP-event time, flagged stale."""
    bench = _bench()
    key = ("decode64_24b", "silu_and_mul")
    traced = bench.TRACED_LAUNCH_US[key]
    fresh = dict(traced, sources={rel: bench.source_blob(rel) for rel in bench.KERNEL_SOURCES["silu_and_mul"]})
    monkeypatch.setitem(bench.TRACED_LAUNCH_US, key, fresh)
    e = bench.roofline_entry(*key, 12_582_912, 3.5)
    assert e["avg_launch_us"] == round(fresh["us"], 3) and not e["trace_stale"]
    assert e["frac"] == round(12_582_912 / fresh["us"] / 1e3 / 8000.0, 4)
    assert e["frac_event"] == round(12_582_912 / 3.5 / 1e3 / 8000.0, 4)
    stale = dict(fresh, sources={**fresh["sources"], "csrc/silu_and_mul.hip": "0" * 40})
    monkeypatch.setitem(bench.TRACED_LAUNCH_US, key, stale)
    e = bench.roofline_entry(*key, 12_582_912, 3.5)
    assert e["trace_stale"] and e["avg_launch_us"] == 3.5 and e["timing"] == "hip-events (live)"
    # flops-bound lines use the same rule
    m = bench.roofline_entry("no_such_workload", "paged_context_attention", 1e12, 500.0, bound="mfma")
    assert m["unit"] == "TFLOP/s" and m["frac"] == round(1e12 / 500.0 / 1e6 / 2500.0, 4)


def test_profiled_figures_name_existing_profiles_that_hold_them():
    """Every profiled figure cites a committed profile that states it, and records the hash of every
    source its kernel is built from."""
    bench = _bench()
    for table, field, fmt in ((bench.TRACED_LAUNCH_US, "us", None), (bench.MEASURED_TRAFFIC, "bytes", "{:,}")):
        for (workload, kernel), entry in table.items():
            text = (ROOT / entry["profile"]).read_text()
            assert set(entry["sources"]) == set(bench.KERNEL_SOURCES[kernel]), (workload, kernel)
            if fmt is not None:
                assert fmt.format(entry[field]) in text, (workload, kernel, entry[field])
