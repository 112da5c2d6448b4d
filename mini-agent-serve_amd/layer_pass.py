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
``Devstral2Model.forward`` does (:282-304).
"""
from __future__ import annotations

import torch

from . import activation, embedding, fused, norm, page, rope
from .workloads import LayerInputs, Shape, credited_bytes, layer_credited_bytes, make_layer_inputs

__all__ = ["LayerBuffers", "run_layer", "DecodePass"]


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
