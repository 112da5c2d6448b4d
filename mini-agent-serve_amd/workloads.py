"""Seeded synthetic inputs for the five layer-kernel workloads (the shapes of mini-agent-serve's
Devstral-Small-2 24B and Devstral-2 123B decoders), and the credited-byte model used to report
HBM bandwidth.

Tensors are drawn as N(0, 1) in fp32 and cast to bf16; norm weights are 1 + 0.1 N(0, 1). q, k and v
are column views of one fused qkv buffer ``[N, (Hq + 2 Hk) D]``, exactly as the reference splits its
qkv GEMM output (miniagentserve/models/devstral2/devstral2.py:158-161). Index tensors use the
reference's dtypes: positions / batch indices / page tables int32, token ids int64
(miniagentserve/engine/model_runner.py:43-47).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .rope import cos_sin_cache

__all__ = ["Shape", "SHAPES", "LayerInputs", "make_layer_inputs", "credited_bytes", "layer_credited_bytes",
           "AttentionShape", "ATTENTION_SHAPES", "AttentionInputs", "make_attention_inputs",
           "attention_credited_bytes", "ContextShape", "CONTEXT_SHAPES", "ContextInputs", "make_context_inputs",
           "context_flops", "StepShape", "STEP_SHAPES", "StepLayout", "make_step_layout"]


@dataclass(frozen=True)
class Shape:
    name: str
    tokens: int
    hidden: int
    inter: int
    q_heads: int
    kv_heads: int
    head_dim: int
    num_pages: int
    page_size: int
    seqs: int                   # sequences in the batch (decode: one token each)
    decode: bool                # decode: random positions; prefill: contiguous 0..len-1 per sequence
    max_position: int = 32768
    theta: float = 1e6
    eps: float = 1e-5
    layers: int = 1
    vocab: int = 131072
    norm_only: bool = False     # the step is one RMSNorm + residual (the single-op CPU case)

    @property
    def qkv_width(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim


SHAPES: dict[str, Shape] = {s.name: s for s in [
    # the CPU-runnable single-op case: RMSNorm + residual on [256, 5120]
    Shape("rmsnorm_256x5120", 256, 5120, 32768, 32, 8, 128, 1, 256, 256, True, norm_only=True),
    # Devstral-Small-2 decode step, one layer, 64 tokens; 2048 pages x 256 slots
    Shape("decode64_24b", 64, 5120, 32768, 32, 8, 128, 2048, 256, 64, True),
    # Devstral-Small-2 chunked prefill, one layer, 4 x 2048 tokens; 4096-page pool
    Shape("prefill8192_24b", 8192, 5120, 32768, 32, 8, 128, 4096, 256, 4, False),
    # Devstral-2 123B prefill, one layer, 4 x 4096 tokens; 8192-page pool
    Shape("prefill16384_123b", 16384, 12288, 28672, 96, 8, 128, 8192, 256, 4, False),
    # 40-layer decode pass over 256 sequences (GEMM and attention outputs replaced by N(0,1));
    # 512 pages x 256 slots per layer, each sequence's current page distinct
    Shape("decode_pass_256x40", 256, 5120, 32768, 32, 8, 128, 512, 256, 256, True, layers=40),
    # the same decode and prefill layers on the reference engine's default 16-slot pages
    # (miniagentserve/engine/serving_engine.py:24), pools of the same capacity
    Shape("decode64_24b_p16", 64, 5120, 32768, 32, 8, 128, 32768, 16, 64, True),
    Shape("prefill8192_24b_p16", 8192, 5120, 32768, 32, 8, 128, 65536, 16, 4, False),
]}


@dataclass
class LayerInputs:
    shape: Shape
    hidden: torch.Tensor        # [N, H] bf16, the previous sublayer's output entering the first norm
    residual: torch.Tensor      # [N, H] bf16
    norm_weight: torch.Tensor   # [H] bf16, input_layernorm
    attn_out: torch.Tensor      # [N, H] bf16, stand-in for the o_proj output entering the second norm
    post_norm_weight: torch.Tensor  # [H] bf16, post_attention_layernorm
    gate_up: torch.Tensor       # [N, 2I] bf16
    qkv: torch.Tensor           # [N, (Hq + 2Hk) D] bf16
    positions: torch.Tensor     # [N] int32
    batch_indices: torch.Tensor  # [N] int32
    block_tables: torch.Tensor  # [batch, width] int32
    kv_indptr: torch.Tensor     # [batch + 1] int32
    slot_mapping: torch.Tensor  # [N] int64, the same destinations as the block-table form
    table: torch.Tensor         # [max_position, D] fp32 cos/sin
    k_cache: torch.Tensor | None = None
    v_cache: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)

    @property
    def q(self) -> torch.Tensor:
        s = self.shape
        return self.qkv[:, : s.q_heads * s.head_dim]

    @property
    def k(self) -> torch.Tensor:
        s = self.shape
        return self.qkv[:, s.q_heads * s.head_dim: (s.q_heads + s.kv_heads) * s.head_dim]

    @property
    def v(self) -> torch.Tensor:
        s = self.shape
        return self.qkv[:, (s.q_heads + s.kv_heads) * s.head_dim:]


def _indices(shape: Shape, gen: torch.Generator):
    """Positions, batch indices, block tables, indptr and slots on the CPU."""
    n, ps = shape.tokens, shape.page_size
    if shape.decode:
        # one token per sequence at a random position; every sequence's current page is distinct
        positions = torch.randint(0, shape.max_position, (n,), generator=gen, dtype=torch.int64)
        width = -(-shape.max_position // ps)
        pages = torch.randperm(shape.num_pages, generator=gen)[:n]
        tables = torch.randint(0, shape.num_pages, (n, width), generator=gen, dtype=torch.int64)
        tables[torch.arange(n), positions // ps] = pages
        batch = torch.arange(n)
    else:
        per_seq = n // shape.seqs
        width = -(-per_seq // ps)
        positions = torch.arange(per_seq).repeat(shape.seqs)
        batch = torch.arange(shape.seqs).repeat_interleave(per_seq)
        tables = torch.randperm(shape.num_pages, generator=gen)[: shape.seqs * width].reshape(shape.seqs, width)
    slots = tables[batch, positions // ps] * ps + positions % ps
    indptr = torch.arange(tables.shape[0] + 1) * tables.shape[1]
    return (positions.to(torch.int32), batch.to(torch.int32), tables.to(torch.int32), indptr.to(torch.int32),
            slots.to(torch.int64))


def make_layer_inputs(shape: Shape | str, device: torch.device | str = "cpu", seed: int = 0,
                      with_cache: bool = True, fill_on_device: bool = False,
                      table: torch.Tensor | None = None, zero_cache: bool = True) -> LayerInputs:
    """One layer's inputs. ``fill_on_device`` draws the big tensors with the device's generator
    (fast for the prefill shapes); otherwise everything is drawn on the CPU and copied, so the
    oracle can see the same values. ``zero_cache=False`` leaves the KV cache uninitialised (timing
    runs, where only the slots a step writes matter)."""
    if isinstance(shape, str):
        shape = SHAPES[shape]
    device = torch.device(device)
    cpu_gen = torch.Generator().manual_seed(seed)
    dev_gen = torch.Generator(device=device).manual_seed(seed) if fill_on_device else None
    n = shape.tokens

    def normal(*size, scale=1.0, shift=0.0):
        if fill_on_device:
            t = torch.randn(*size, generator=dev_gen, device=device)
        else:
            t = torch.randn(*size, generator=cpu_gen).to(device)
        return (shift + scale * t).to(torch.bfloat16) if (scale != 1.0 or shift != 0.0) else t.to(torch.bfloat16)

    hidden = normal(n, shape.hidden)
    residual = normal(n, shape.hidden)
    weight = normal(shape.hidden, scale=0.1, shift=1.0)
    attn_out = normal(n, shape.hidden)
    post_weight = normal(shape.hidden, scale=0.1, shift=1.0)
    gate_up = normal(n, 2 * shape.inter)
    qkv = normal(n, shape.qkv_width)
    positions, batch, tables, indptr, slots = _indices(shape, cpu_gen)
    if table is None:
        table = cos_sin_cache(shape.max_position, shape.head_dim, shape.theta)
    inputs = LayerInputs(shape, hidden, residual, weight, attn_out, post_weight, gate_up, qkv, positions.to(device),
                         batch.to(device), tables.to(device), indptr.to(device), slots.to(device), table.to(device))
    if with_cache:
        cache_shape = (shape.num_pages, shape.page_size, shape.kv_heads, shape.head_dim)
        alloc = torch.zeros if zero_cache else torch.empty
        inputs.k_cache = alloc(cache_shape, dtype=torch.bfloat16, device=device)
        inputs.v_cache = alloc(cache_shape, dtype=torch.bfloat16, device=device)
    return inputs


def layer_credited_bytes(shape: Shape, fused_rope_kv: bool = False, fp8: bool = False) -> int:
    """One decoder layer's kernels: two norms, SiluAndMul, RoPE, KV store (one norm for a norm-only
    shape). With RoPE and the store fused, k is read once: 2·N·Hk·D bytes fewer. ``fp8``: the
    reference's FP8 dataflow - norms write fp8 (7·N·H) and SiluAndMul writes the quantized down_proj
    input (5·N·I)."""
    b = credited_bytes(shape)
    norm = b["fused_add_rmsnorm_quant"] if fp8 else b["fused_add_rmsnorm"]
    if shape.norm_only:
        return norm
    rope_kv = b["rope_append"] if fused_rope_kv else b["rope"] + b["append_paged_kv_cache"]
    return 2 * norm + (b["silu_and_mul_quant"] if fp8 else b["silu_and_mul"]) + rope_kv


def credited_bytes(shape: Shape) -> dict[str, int]:
    """Algorithmic HBM bytes per launch: each mandatory input element read once, each output
    element written once, index arrays included, the norm weight once, the cos/sin table not
    credited (it could be computed in the kernel)."""
    n, h, i = shape.tokens, shape.hidden, shape.inter
    heads = shape.q_heads + shape.kv_heads
    d = shape.head_dim
    return {
        "fused_add_rmsnorm": 8 * n * h + 2 * h,
        "fused_add_rmsnorm_quant": 7 * n * h + 2 * h,
        "silu_and_mul": 6 * n * i,
        "silu_and_mul_quant": 5 * n * i,
        "rope": 4 * n * heads * d + 4 * n,
        "append_paged_kv_cache": 8 * n * shape.kv_heads * d + 8 * n,
        # fused RoPE + KV append: q, k read and written; v read; k and v written to the cache
        "rope_append": 4 * n * heads * d + 4 * n + 6 * n * shape.kv_heads * d + 4 * n,
        "embedding": 4 * n * h + 8 * n,
    }


# ---- paged decode attention -------------------------------------------------------------------------

@dataclass(frozen=True)
class AttentionShape:
    name: str
    batch: int                  # decode rows, one query token each
    q_heads: int
    kv_heads: int
    head_dim: int
    page_size: int
    max_len: int                # seq_lens drawn uniformly from [1, max_len]; block-table width max_len / page_size


ATTENTION_SHAPES: dict[str, AttentionShape] = {s.name: s for s in [
    # Devstral-Small-2 decode attention: 64 rows, lengths up to 8192 (the runner's graph width,
    # max_model_len 8192 / 256-slot blocks), 4 query heads per kv head
    AttentionShape("decode_attn_64x8192_24b", 64, 32, 8, 128, 256, 8192),
    # Devstral-2 123B: 12 query heads per kv head
    AttentionShape("decode_attn_64x8192_123b", 64, 96, 8, 128, 256, 8192),
    # the reference engine's default 16-slot pages (serving_engine.py:24)
    AttentionShape("decode_attn_64x8192_24b_p16", 64, 32, 8, 128, 16, 8192),
]}


@dataclass
class AttentionInputs:
    shape: AttentionShape
    q: torch.Tensor             # [batch, Hq, D] bf16
    k_cache: torch.Tensor       # [pages, page_size, Hk, D] bf16 (NHD)
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [batch, max_len / page_size] int32
    seq_lens: torch.Tensor      # [batch] int32
    workspace: torch.Tensor     # uint8, the reference's 128 MiB


def make_attention_inputs(shape: AttentionShape | str, device="cpu", seed: int = 0) -> AttentionInputs:
    """Each row gets ceil(len / page_size) distinct pages of a pool sized to hold them all (pages in
    random order); caches, q ~ N(0, 1), drawn on ``device``."""
    if isinstance(shape, str):
        shape = ATTENTION_SHAPES[shape]
    device = torch.device(device)
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, shape.max_len + 1, (shape.batch,), generator=g)
    width = shape.max_len // shape.page_size
    need = [-(-int(n) // shape.page_size) for n in lens]
    pages = sum(need) + 1
    perm = torch.randperm(pages, generator=g)
    tables = torch.zeros(shape.batch, width, dtype=torch.int32)
    at = 0
    for b, k in enumerate(need):
        tables[b, :k] = perm[at:at + k].to(torch.int32)
        at += k
    dg = torch.Generator(device=device).manual_seed(seed)
    kv = (pages, shape.page_size, shape.kv_heads, shape.head_dim)
    return AttentionInputs(
        shape=shape,
        q=torch.randn(shape.batch, shape.q_heads, shape.head_dim, generator=dg, device=device).bfloat16(),
        k_cache=torch.randn(kv, generator=dg, device=device).bfloat16(),
        v_cache=torch.randn(kv, generator=dg, device=device).bfloat16(),
        block_tables=tables.to(device), seq_lens=lens.to(torch.int32).to(device),
        workspace=torch.zeros(128 << 20, dtype=torch.uint8, device=device))


def attention_credited_bytes(inputs: AttentionInputs) -> int:
    """Each key and value row of every position read once (2 * Hk * D * 2 bytes per position), q
    read and out written once, one block-table entry per page and one seq_len per row. The split
    partials in the workspace are not credited."""
    s = inputs.shape
    lens = inputs.seq_lens.cpu().long()
    positions = int(lens.sum())
    pages = int(((lens + s.page_size - 1) // s.page_size).sum())
    return positions * s.kv_heads * s.head_dim * 4 + 2 * s.batch * s.q_heads * s.head_dim * 2 + pages * 4 + s.batch * 4


# ---- paged context (prefill) attention ---------------------------------------------------------------

@dataclass(frozen=True)
class ContextShape:
    name: str
    rows: int                   # prompt rows
    q_len: int                  # new tokens per row
    cached: int                 # positions already in the cache before them (kv_len = cached + q_len)
    q_heads: int
    kv_heads: int
    head_dim: int
    page_size: int
    # The layout of the reference's captured graphs (model_runner.py:155-221) when graph_rows > 0:
    # graph_rows prompt rows, the real ones first, then one padding row holding the padding tokens
    # (the step's token count rounded up to 64; their kv_len = their count, every block-table entry
    # the sink page) and empty rows (seq_len 1); max_q_len = the step's tokens, padding included
    # (devstral2.py:295), and the block table reach positions wide (the graphs' max_blocks), passed
    # as max_kv_len (devstral2.py:296).
    graph_rows: int = 0
    reach: int = 0


CONTEXT_SHAPES: dict[str, ContextShape] = {s.name: s for s in [
    # the prefill-8192 step's attention: 4 prompts of 2048 tokens, Devstral-Small-2 heads
    ContextShape("context_attn_4x2048_24b", 4, 2048, 0, 32, 8, 128, 256),
    # the prefill-16384 step's attention: 4 prompts of 4096 tokens, Devstral-2 123B heads
    ContextShape("context_attn_4x4096_123b", 4, 4096, 0, 96, 8, 128, 256),
    # the reference engine's default 16-slot pages (serving_engine.py:24)
    ContextShape("context_attn_4x2048_24b_p16", 4, 2048, 0, 32, 8, 128, 16),
    # an agent turn: a few new tokens after a long cached conversation prefix (few token tiles, long
    # key ranges: the split-KV shapes), 16-slot pages
    ContextShape("context_attn_1x128_after4096_24b", 1, 128, 4096, 32, 8, 128, 16),
    ContextShape("context_attn_4x256_after8192_24b", 4, 256, 8192, 32, 8, 128, 16),
    ContextShape("context_attn_1x128_after4096_123b", 1, 128, 4096, 96, 8, 128, 16),
    # the same kind of turn inside the reference's graphs (17 prompt rows, 128 tokens, an 8192-position
    # table: its engine's defaults, serving_engine.py:23-27): split-KV decided on the device
    ContextShape("context_attn_graph_1x100_after4000_24b", 1, 100, 4000, 32, 8, 128, 16, graph_rows=17, reach=8192),
    ContextShape("context_attn_graph_1x100_after4000_123b", 1, 100, 4000, 96, 8, 128, 16, graph_rows=17,
                 reach=8192),
    ContextShape("context_attn_graph_3x100_after2000_24b", 3, 100, 2000, 32, 8, 128, 16, graph_rows=17, reach=8192),
    # a graph step where no split pays (a fresh prompt): the planned launch against the one-kernel grid
    ContextShape("context_attn_graph_1x120_after0_24b", 1, 120, 0, 32, 8, 128, 16, graph_rows=17, reach=8192),
]}


@dataclass
class ContextInputs:
    shape: ContextShape
    q: torch.Tensor             # [rows * q_len, Hq, D]
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_tables: torch.Tensor  # [rows, pages per row] int32 (the real rows first)
    seq_lens: torch.Tensor      # [rows] int32 (kv_len)
    cu_seqlens_q: torch.Tensor  # [rows + 1] int32
    max_q_len: int
    max_kv_len: int


def make_context_inputs(shape: ContextShape | str, device="cpu", seed: int = 0) -> ContextInputs:
    if isinstance(shape, str):
        shape = CONTEXT_SHAPES[shape]
    device = torch.device(device)
    kv_len = shape.cached + shape.q_len
    width = -(-kv_len // shape.page_size)
    pages = shape.rows * width + 1   # the last page: the graphs' sink for padding rows
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(pages - 1 if shape.graph_rows else pages, generator=g)
    real = perm[: shape.rows * width].reshape(shape.rows, width).to(torch.int32)
    lens = [kv_len] * shape.rows
    cu = [r * shape.q_len for r in range(shape.rows + 1)]
    tokens, max_q, max_kv = shape.rows * shape.q_len, shape.q_len, kv_len
    tables = real
    if shape.graph_rows:
        total = -(-tokens // 64) * 64
        pad = total - tokens
        tables = torch.full((shape.graph_rows, max(shape.reach // shape.page_size, width)), pages - 1,
                            dtype=torch.int32)
        tables[: shape.rows, :width] = real
        tables[: shape.rows, width:] = -1   # past seq_lens: never read
        lens += [max(pad, 1)] + [1] * (shape.graph_rows - shape.rows - 1)
        cu += [total] * (shape.graph_rows - shape.rows)
        tokens, max_q, max_kv = total, total, tables.shape[1] * shape.page_size
    dg = torch.Generator(device=device).manual_seed(seed)
    kv = (pages, shape.page_size, shape.kv_heads, shape.head_dim)
    return ContextInputs(
        shape=shape,
        q=torch.randn(tokens, shape.q_heads, shape.head_dim, generator=dg, device=device).bfloat16(),
        k_cache=torch.randn(kv, generator=dg, device=device).bfloat16(),
        v_cache=torch.randn(kv, generator=dg, device=device).bfloat16(),
        block_tables=tables.to(device),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        cu_seqlens_q=torch.tensor(cu, dtype=torch.int32, device=device),
        max_q_len=max_q, max_kv_len=max_kv)


def context_flops(shape: ContextShape) -> int:
    """Algorithmic flops of causal attention: each (query token, head) scores and weighs the
    positions up to its own, 2 * D flops each for Q.K and for P.V (the real rows only, not a graph's
    padding)."""
    positions = sum(shape.cached + i + 1 for i in range(shape.q_len))
    return shape.rows * positions * shape.q_heads * shape.head_dim * 4


# ---- whole forward steps (decode rows and prompt rows, as the runner lays a graph step out) -----------

@dataclass(frozen=True)
class StepShape:
    """One step of the reference's captured forward (Devstral2Model.forward, devstral2.py:265-307)
    at Devstral-Small-2's sizes: ``decode_rows`` decode sequences with lengths drawn from U[1,
    max_len] (each appends its one new token at position len - 1) and, when ``prompts`` is not
    empty, the runner's 17 prompt rows: the prompts ((new tokens, cached positions) each), one
    padding row and empty rows (model_runner.py:179-221). Pages of ``page_size`` slots and block
    tables ``reach / page_size`` columns wide: the reference engine's defaults (serving_engine.py:23-27,
    model_runner.py:79)."""
    name: str
    decode_rows: int
    max_len: int
    prompts: tuple = ()
    layers: int = 40
    page_size: int = 16
    reach: int = 8192
    layer: Shape = SHAPES["decode64_24b"]     # hidden / intermediate / head sizes
    prefill_rows: int = 17                    # model_runner.py:21
    token_step: int = 64                      # model_runner.py:19: graph token counts are multiples of it


STEP_SHAPES: dict[str, StepShape] = {s.name: s for s in [
    # a decode step of 64 sequences up to 8192 positions through all 40 layers
    StepShape("decode_step_64x8192_40", 64, 8192),
    # the same decode rows with an agent turn's prompt chunk in the same step: 100 new tokens after
    # 4000 cached (a 192-token graph step: 64 decode tokens, 100 prompt tokens, 28 padding tokens)
    StepShape("mixed_step_64x8192_1x100_40", 64, 8192, prompts=((100, 4000),)),
]}


@dataclass
class StepLayout:
    """A step's index tensors on the CPU, as the runner's prepare() fills them for a graph step:
    decode rows first (decode row i owns token i), then the prompt rows; tokens of the padding row at
    positions 0.. of the sink page (the pool's last page)."""
    num_tokens: int
    num_decodes: int
    positions: torch.Tensor     # [num_tokens] int32
    batch_indices: torch.Tensor  # [num_tokens] int32
    seq_lens: torch.Tensor      # [rows] int32
    cu_seqlens_q: torch.Tensor  # [prefill rows + 1] int32 (prompt tokens, counted after the decode tokens)
    block_tables: torch.Tensor  # [rows, reach / page_size] int32
    pages: int                  # pages in the pool, the sink page last
    decode_positions: int       # positions the decode rows attend (their seq_lens summed)


def make_step_layout(shape: StepShape, seed: int = 0) -> StepLayout:
    g = torch.Generator().manual_seed(seed)
    ps, width = shape.page_size, shape.reach // shape.page_size
    d = shape.decode_rows
    dec_lens = torch.randint(1, shape.max_len + 1, (d,), generator=g)
    npf = len(shape.prompts)
    tokens = d + sum(q for q, _ in shape.prompts)
    if npf:
        tokens = -(-tokens // shape.token_step) * shape.token_step
    prefill_rows = shape.prefill_rows if npf else 0
    rows = d + prefill_rows
    row_lens = [int(n) for n in dec_lens] + [q + c for q, c in shape.prompts]
    need = [-(-n // ps) for n in row_lens]
    if max(need) > width:
        raise ValueError("a row reaches past the block table")
    pages = sum(need) + 1
    sink = pages - 1
    perm = torch.randperm(pages - 1, generator=g).to(torch.int32)
    tables = torch.full((rows, width), sink, dtype=torch.int32)   # past seq_lens: never read
    at = 0
    for r, k in enumerate(need):
        tables[r, :k] = perm[at:at + k]
        at += k
    positions = torch.zeros(tokens, dtype=torch.int32)
    batch = torch.zeros(tokens, dtype=torch.int32)
    lens = torch.ones(rows, dtype=torch.int32)
    cu = torch.zeros(prefill_rows + 1, dtype=torch.int32)
    positions[:d] = (dec_lens - 1).to(torch.int32)
    batch[:d] = torch.arange(d, dtype=torch.int32)
    lens[:d] = dec_lens.to(torch.int32)
    t = 0
    for j, (q, c) in enumerate(shape.prompts):
        cu[j] = t
        positions[d + t:d + t + q] = torch.arange(c, c + q, dtype=torch.int32)
        batch[d + t:d + t + q] = d + j
        lens[d + j] = c + q
        t += q
    if prefill_rows > npf:
        first, start = d + npf, d + t
        positions[start:] = torch.arange(tokens - start, dtype=torch.int32)
        batch[start:] = first
        lens[first:] = 1
        lens[first] = max(tokens - start, 1)
        cu[npf] = t
        cu[npf + 1:] = tokens - d
        tables[first:, :] = sink
    if prefill_rows:
        cu[prefill_rows] = tokens - d
    return StepLayout(tokens, d, positions, batch, lens, cu, tables, pages, int(dec_lens.sum()))
