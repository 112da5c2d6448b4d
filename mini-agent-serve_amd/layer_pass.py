"""The reference decoder layer's kernel sequence, with the GEMM and attention outputs supplied as
inputs (they are outside this library).

Per layer, in the order of miniagentserve/models/devstral2/devstral2.py:237-253 and 155-224:
  1. fused add + RMSNorm of the previous sublayer output into the residual stream    (:241-246)
  2. RoPE on the q/k column views of the fused qkv output                            (:163-166)
  3. paged KV append of k/v                                                          (:170-173)
     (``fuse_rope_kv`` runs 2 and 3 as one kernel, with the same results)
  4. fused add + RMSNorm of the attention output                                     (:248-252)
  5. SiluAndMul of the gate_up output                                                (:224)
The reference's in-layer norms emit fp8 for its FP8 GEMMs and its down_proj quantizes the
SiluAndMul output; ``fp8`` selects that dataflow (fp8 norm epilogue, SiluAndMul with the quantize
fused in). Otherwise the norms write bf16 in place and SiluAndMul writes bf16 (the variant the
layer-kernel workloads are quoted on).
``DecodePass`` chains 40 such layers behind the embedding gather over one residual stream, as
``Devstral2Model.forward`` does (:282-304). ``ForwardStep`` is a whole step of the reference's
forward in its fp8 dataflow with the attention inside every layer: decode rows and the runner's
prompt rows laid out as a captured graph step, each layer's decode attention and context attention
on its own KV cache, and the final norm (:265-307).
"""
from __future__ import annotations

import torch

from . import activation, attention, embedding, fused, norm, page, rope
from .workloads import (LayerInputs, Shape, StepShape, credited_bytes, layer_credited_bytes, make_layer_inputs,
                        make_step_layout)

__all__ = ["LayerBuffers", "run_layer", "DecodePass", "ForwardStep"]


class LayerBuffers:
    """One layer's inputs plus the outputs the kernels write (SiluAndMul output, fp8 norm output)."""

    def __init__(self, inputs: LayerInputs, fp8: bool = False, act_scale: float = 0.05, fuse_rope_kv: bool = False):
        s = inputs.shape
        self.inputs = inputs
        self.fuse_rope_kv = fuse_rope_kv
        dev = inputs.hidden.device
        self.fp8 = fp8
        self.silu_out = torch.empty(s.tokens, s.inter, dtype=torch.float8_e4m3fn if fp8 else torch.bfloat16,
                                    device=dev)
        if fp8:
            self.norm_out = torch.empty(s.tokens, s.hidden, dtype=torch.float8_e4m3fn, device=dev)
            self.act_scale = torch.tensor(act_scale, dtype=torch.float32, device=dev)
        s3 = (s.tokens, s.kv_heads, s.head_dim)
        self.k3 = inputs.k.view(s3)
        self.v3 = inputs.v.view(s3)
        self.kv_indices = inputs.block_tables.flatten()


def run_layer(b: LayerBuffers) -> None:
    li = b.inputs
    s = li.shape
    if b.fp8:
        norm.fused_add_rmsnorm_quant(b.norm_out, li.hidden, li.residual, li.norm_weight, b.act_scale, s.eps)
    else:
        norm.fused_add_rmsnorm(li.hidden, li.residual, li.norm_weight, s.eps)
    if s.norm_only:
        return
    if b.fuse_rope_kv:
        fused.apply_rope_and_append_paged_kv_cache(li.positions, li.q, li.k, b.v3, s.head_dim, li.table, True,
                                                   li.batch_indices, (li.k_cache, li.v_cache), b.kv_indices,
                                                   li.kv_indptr, None, "NHD")
    else:
        rope.apply_rope_with_cos_sin_cache_inplace(li.positions, li.q, li.k, s.head_dim, li.table, True)
        page.append_paged_kv_cache(b.k3, b.v3, li.batch_indices, li.positions, (li.k_cache, li.v_cache),
                                   b.kv_indices, li.kv_indptr, None, "NHD")
    if b.fp8:
        norm.fused_add_rmsnorm_quant(b.norm_out, li.attn_out, li.residual, li.post_norm_weight, b.act_scale, s.eps)
        activation.silu_and_mul_quant(li.gate_up, b.act_scale, out=b.silu_out)
    else:
        norm.fused_add_rmsnorm(li.attn_out, li.residual, li.post_norm_weight, s.eps)
        activation.silu_and_mul(li.gate_up, out=b.silu_out)


class DecodePass:
    """Embedding gather + ``shape.layers`` layers over one shared residual stream.

    Layer 0's first norm reads the embedding output; every other sublayer output is an N(0, 1)
    stand-in. Each layer has its own KV cache, as the reference's per-layer slices of
    ``[layers, pages, page_size, kv_heads, head_dim]`` (model_runner.py:83-85).
    """

    def __init__(self, shape: Shape, device: torch.device, seed: int = 0, fp8: bool = False,
                 fuse_rope_kv: bool = False):
        self.shape = shape
        self.device = device
        table = rope.cos_sin_cache(shape.max_position, shape.head_dim, shape.theta).to(device)
        self.layers: list[LayerBuffers] = []
        residual = None
        for i in range(shape.layers):
            li = make_layer_inputs(shape, device, seed=seed * 1000 + i, fill_on_device=True, table=table)
            if residual is None:
                residual = li.residual
                residual.zero_()          # devstral2.py:302: the stream starts at zero
            else:
                li.residual = residual
            self.layers.append(LayerBuffers(li, fp8, fuse_rope_kv=fuse_rope_kv))
        gen = torch.Generator(device=device).manual_seed(seed)
        self.embed_table = torch.randn(shape.vocab, shape.hidden, generator=gen, device=device).to(torch.bfloat16)
        cpu = torch.Generator().manual_seed(seed)
        self.ids = torch.randint(0, shape.vocab, (shape.tokens,), generator=cpu).to(device)
        self.embed_out = self.layers[0].inputs.hidden

    def run(self) -> None:
        embedding.embedding(self.ids, self.embed_table, out=self.embed_out)
        for b in self.layers:
            run_layer(b)

    def credited_bytes(self) -> int:
        b = self.layers[0]
        return credited_bytes(self.shape)["embedding"] + self.shape.layers * layer_credited_bytes(
            self.shape, b.fuse_rope_kv, b.fp8)


class ForwardStep:
    """One captured forward step of the reference (Devstral2Model.forward, devstral2.py:265-307) with
    its GEMMs replaced by N(0, 1) stand-in outputs: the embedding gather of the step's tokens, then per
    layer (:237-253, :155-224)
      1. fused add + RMSNorm, fp8 out (the qkv_proj input)
      2. RoPE + paged KV append + llama-4 query scale, one kernel, on the qkv stand-in
      3. decode attention on the decode rows' query tokens and context attention on the prompt rows'
         (the runner's 17 rows, max_q_len = the step's prompt-side tokens, max_kv_len = the block
         table's reach: :287-296), both writing the o_proj input quantize
      4. fused add + RMSNorm of the o_proj stand-in, fp8 out (the gate_up input)
      5. SiluAndMul + quantize of the gate_up stand-in (the down_proj input)
    and the final bf16 norm. Each layer has its own KV cache (one pool of 16-slot pages holding
    every row's positions), its own stand-ins and norm weights; one residual stream runs through all
    of them. Rows and tokens follow the runner's prepare() (make_step_layout). The workspace is the
    reference's 128 MiB buffer (devstral2.py:35), shared by both attention calls.
    """

    LLAMA_4_BETA = 0.1
    LLAMA_4_ORIGINAL_MAX = 8192

    def __init__(self, shape: StepShape, device: torch.device, seed: int = 0, act_scale: float = 0.05):
        self.shape = shape
        ls = shape.layer
        self.device = device
        lay = make_step_layout(shape, seed)
        self.layout = lay
        n, d = lay.num_tokens, lay.num_decodes
        self.num_tokens, self.num_decodes = n, d
        self.positions = lay.positions.to(device)
        self.batch_indices = lay.batch_indices.to(device)
        self.seq_lens = lay.seq_lens.to(device)
        self.cu_seqlens_q = lay.cu_seqlens_q.to(device)
        self.block_tables = lay.block_tables.to(device)
        self.kv_indices = self.block_tables.flatten()
        rows = self.block_tables.shape[0]
        self.kv_indptr = torch.arange(rows + 1, dtype=torch.int32, device=device) * self.block_tables.shape[1]
        self.num_prefills = self.cu_seqlens_q.numel() - 1
        self.max_q_len = n - d
        self.max_kv_len = shape.reach
        self.table = rope.cos_sin_cache(ls.max_position, ls.head_dim, ls.theta).to(device)
        self.scale = ls.head_dim ** -0.5
        self.act_scale = torch.tensor(act_scale, dtype=torch.float32, device=device)
        self.workspace = torch.zeros(128 << 20, dtype=torch.uint8, device=device)
        gen = torch.Generator(device=device).manual_seed(seed)

        def normal(*size, scale=1.0, shift=0.0):
            t = torch.randn(*size, generator=gen, device=device)
            return (shift + scale * t).to(torch.bfloat16) if (scale != 1.0 or shift != 0.0) else t.to(torch.bfloat16)

        cache_shape = (lay.pages, shape.page_size, ls.kv_heads, ls.head_dim)
        k0, v0 = normal(*cache_shape), normal(*cache_shape)
        self.residual = torch.zeros(n, ls.hidden, dtype=torch.bfloat16, device=device)  # devstral2.py:302
        self.layers = []
        for _ in range(shape.layers):
            self.layers.append({
                "hidden": normal(n, ls.hidden),            # the previous down_proj output (layer 0: the embedding)
                "w_in": normal(ls.hidden, scale=0.1, shift=1.0),
                "qkv": normal(n, ls.qkv_width),
                "o_proj": normal(n, ls.hidden),
                "w_post": normal(ls.hidden, scale=0.1, shift=1.0),
                "gate_up": normal(n, 2 * ls.inter),
                "k_cache": k0.clone(), "v_cache": v0.clone(),
            })
        del k0, v0
        self.final_in = normal(n, ls.hidden)               # the last down_proj output
        self.final_weight = normal(ls.hidden, scale=0.1, shift=1.0)
        self.norm_out = torch.empty(n, ls.hidden, dtype=torch.float8_e4m3fn, device=device)
        self.attn_out = torch.empty(n, ls.q_heads, ls.head_dim, dtype=torch.float8_e4m3fn, device=device)
        self.silu_out = torch.empty(n, ls.inter, dtype=torch.float8_e4m3fn, device=device)
        self.embed_table = normal(ls.vocab, ls.hidden)
        cpu = torch.Generator().manual_seed(seed)
        self.ids = torch.randint(0, ls.vocab, (n,), generator=cpu).to(device)

    def views(self, layer: dict):
        """q [tokens, Hq, D], k [tokens, Hk * D] and v [tokens, Hk, D]: column views of the qkv stand-in
        (devstral2.py:158-168)."""
        ls = self.shape.layer
        qkv = layer["qkv"]
        qd, kd = ls.q_heads * ls.head_dim, ls.kv_heads * ls.head_dim
        return (qkv[:, :qd], qkv[:, qd:qd + kd], qkv[:, qd + kd:].unflatten(-1, (ls.kv_heads, ls.head_dim)))

    def run_norm_in(self, layer: dict) -> None:
        ls = self.shape.layer
        norm.fused_add_rmsnorm_quant(self.norm_out, layer["hidden"], self.residual, layer["w_in"], self.act_scale,
                                     ls.eps)

    def run_rope_append(self, layer: dict) -> None:
        ls = self.shape.layer
        q, k, v = self.views(layer)
        fused.apply_rope_and_append_paged_kv_cache(
            self.positions, q, k, v, ls.head_dim, self.table, True, self.batch_indices,
            (layer["k_cache"], layer["v_cache"]), self.kv_indices, self.kv_indptr, None, "NHD",
            llama_4_scaling_beta=self.LLAMA_4_BETA, original_max_position_embeddings=self.LLAMA_4_ORIGINAL_MAX)

    def run_decode_attention(self, layer: dict) -> None:
        ls, d = self.shape.layer, self.num_decodes
        if d == 0:
            return
        q = self.views(layer)[0].unflatten(-1, (ls.q_heads, ls.head_dim))
        attention.trtllm_batch_decode_with_kv_cache(
            q[:d], (layer["k_cache"], layer["v_cache"]), self.workspace, self.block_tables[:d], self.seq_lens[:d],
            self.max_kv_len, self.scale, 1.0, out=self.attn_out[:d], out_quant_scale=self.act_scale)

    def run_context_attention(self, layer: dict) -> None:
        ls, d = self.shape.layer, self.num_decodes
        if self.num_prefills == 0:
            return
        q = self.views(layer)[0].unflatten(-1, (ls.q_heads, ls.head_dim))
        attention.trtllm_batch_context_with_kv_cache(
            q[d:], (layer["k_cache"], layer["v_cache"]), self.workspace, self.block_tables[d:], self.seq_lens[d:],
            self.max_q_len, self.max_kv_len, self.scale, 1.0, self.num_prefills, self.cu_seqlens_q, None,
            out=self.attn_out[d:], out_quant_scale=self.act_scale)

    def run_norm_post(self, layer: dict) -> None:
        ls = self.shape.layer
        norm.fused_add_rmsnorm_quant(self.norm_out, layer["o_proj"], self.residual, layer["w_post"], self.act_scale,
                                     ls.eps)

    def run_silu(self, layer: dict) -> None:
        activation.silu_and_mul_quant(layer["gate_up"], self.act_scale, out=self.silu_out)

    def run_embedding(self) -> None:
        embedding.embedding(self.ids, self.embed_table, out=self.layers[0]["hidden"])

    def run_final_norm(self) -> None:
        norm.fused_add_rmsnorm(self.final_in, self.residual, self.final_weight, self.shape.layer.eps)

    LAYER_OPS = ("norm_in", "rope_append", "decode_attention", "context_attention", "norm_post", "silu")

    def run(self) -> None:
        self.run_embedding()
        for layer in self.layers:
            for op in self.LAYER_OPS:
                getattr(self, "run_" + op)(layer)
        self.run_final_norm()
