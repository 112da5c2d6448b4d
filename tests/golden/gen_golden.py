"""Writes tests/golden/layer_ops.npz: small seeded inputs of every hot-path op with the oracle's outputs.

The reference has no tests and no fixtures, and its arithmetic lives in flashinfer, which is absent
here, so these vectors come from this repository's oracle (itself pinned against torch and
transformers routines in tests/test_oracle_*.py). They are regression data: the CPU suite checks that
the oracle still reproduces them, the GPU suite checks the kernels against them.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import numerics as on  # noqa: E402
from oracle import ops  # noqa: E402

OUT = Path(__file__).resolve().parent / "layer_ops.npz"


def bf16(rng, *shape, scale=1.0, shift=0.0):
    return on.f32_to_bf16((shift + scale * rng.standard_normal(shape)).astype(np.float32))


def build() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    g: dict[str, np.ndarray] = {}
    # RMSNorm + residual (both epilogues): 6 rows x 264 (not a multiple of 64 lanes x 8), special rows
    x = bf16(rng, 6, 264, scale=2.0)
    r = bf16(rng, 6, 264)
    x[1] = on.f32_to_bf16(np.zeros(264, np.float32))
    r[1] = on.f32_to_bf16(np.zeros(264, np.float32))            # zero row
    x[2] = on.f32_to_bf16(np.full(264, 3.0, np.float32))
    r[2] = on.f32_to_bf16(np.zeros(264, np.float32))            # constant row
    x[3, :8] = on.f32_to_bf16(np.array([1e4, -1e4, 3e-3, 0, 65504, -2.5, 7, 1e-30], np.float32))
    w = bf16(rng, 264, scale=0.1, shift=1.0)
    g["norm_x"], g["norm_r"], g["norm_w"] = x, r, w
    g["norm_eps"] = np.array(1e-5, np.float32)
    g["norm_out"], g["norm_res"] = ops.fused_add_rmsnorm(x, r, w, 1e-5)
    g["quant_scale"] = np.array(0.0123, np.float32)
    g["quant_out"], g["quant_res"] = ops.fused_add_rmsnorm_quant(x, r, w, 0.0123, 1e-5)
    # SiluAndMul: 5 rows x 2*72 with limits in row 0
    gu = bf16(rng, 5, 144, scale=4.0)
    gu[0, :6] = on.f32_to_bf16(np.array([0.0, -0.0, 30.0, -30.0, 90.0, -90.0], np.float32))
    g["silu_in"] = gu
    g["silu_out"] = ops.silu_and_mul(gu)
    # RoPE: 7 tokens, 3 q + 2 k heads of 128, plain table theta 1e6 over 512 positions, both layouts
    table = ops.cos_sin_table(512, ops.rope_inv_freq(128, 1e6))
    pos = np.array([0, 1, 511, 300, 5, 5, 277], np.int32)
    q = bf16(rng, 7, 3, 128)
    k = bf16(rng, 7, 2, 128)
    g["rope_q"], g["rope_k"], g["rope_pos"], g["rope_table"] = q, k, pos, table
    g["rope_neox_q"], g["rope_neox_k"] = ops.rope(q, k, pos, table, is_neox=True)
    g["rope_gptj_q"], g["rope_gptj_k"] = ops.rope(q, k, pos, table, is_neox=False)
    # Paged KV append: 3 sequences, page size 4, 2 heads of 16, pool of 10 pages (last = sink)
    tables = np.array([[3, 7, 1], [0, 9, 9], [5, 2, 8]], np.int32)
    indptr = np.array([0, 3, 6, 9], np.int32)
    bidx = np.array([0, 0, 0, 0, 0, 0, 1, 2, 2, 2], np.int32)
    kpos = np.array([0, 1, 2, 3, 4, 9, 0, 10, 11, 3], np.int32)
    kk = bf16(rng, 10, 2, 16)
    vv = bf16(rng, 10, 2, 16)
    kc0 = bf16(rng, 10, 4, 2, 16)
    vc0 = bf16(rng, 10, 4, 2, 16)
    g.update(kv_tables=tables, kv_indptr=indptr, kv_bidx=bidx, kv_pos=kpos, kv_k=kk, kv_v=vv, kv_kc0=kc0, kv_vc0=vc0)
    g["kv_kc"], g["kv_vc"] = ops.append_paged_kv_cache(kc0, vc0, kk, vv, bidx, kpos, tables.flatten(), indptr)
    # Embedding: 9 ids over a 40 x 48 table, repeats and both ends
    tab = bf16(rng, 40, 48)
    ids = np.array([0, 39, 7, 7, 12, 0, 33, 39, 1], np.int64)
    g["emb_table"], g["emb_ids"] = tab, ids
    g["emb_out"] = ops.embedding(tab, ids)
    return g


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
