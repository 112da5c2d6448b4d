"""MI355X (gfx950) per-layer kernels of mini-agent-serve's Devstral/Mistral decoder.

Drop-ins for the calls the reference's layer modules make
(miniagentserve/models/devstral2/devstral2.py):

- ``norm.fused_add_rmsnorm`` / ``norm.fused_add_rmsnorm_quant``   (flashinfer.norm, :241-252, :305-307)
- ``activation.silu_and_mul``                                       (flashinfer.activation, :224)
- ``activation.silu_and_mul_quant``                                 (:224 with down_proj's fp8 quantize, :93-95)
- ``rope.apply_rope_with_cos_sin_cache_inplace``                    (flashinfer.rope, :163-166)
- ``page.append_paged_kv_cache`` (+ ``page.store_kv_slots``)        (flashinfer.page, :170-173)
- ``embedding.embedding`` / ``embedding.Embedding``                 (nn.Embedding, :260, :282)
- ``embedding.fill_placeholders`` / ``embedding(..., last_tokens=)`` (ModelRunner.fill_placeholders,
  miniagentserve/engine/model_runner.py:149-154, alone or fused with the gather)
- ``attention.trtllm_batch_decode_with_kv_cache``                   (flashinfer.decode, :184-196)
- ``attention.trtllm_batch_context_with_kv_cache``                  (flashinfer.prefill, :198-213)
- ``fused.apply_rope_and_append_paged_kv_cache``                    (:163-166 + :170-173 + the llama-4
  query scale at :175-179, one kernel)

Each op validates its tensors, then calls hand-written HIP kernels in ``libmas_kernels.so``
through the C ABI of ``include/mas_kernels.h`` on torch's current stream. There is no CPU or
PyTorch fallback: without the built library every op raises.

The directory name is not a Python identifier; the repository's ``__graft_entry__.load_package``
imports it as ``mini_agent_serve_amd``.
"""
from __future__ import annotations

from . import _compile_fix, _lib, activation, attention, embedding, fused, norm, page, rope, workloads
from . import layer_pass
from . import _ops  # noqa: F401  (registers the torch.library ops)

_compile_fix.arm()  # Inductor's missing sym_storage_offset lowering, installed when Inductor loads
from .activation import silu_and_mul, silu_and_mul_quant
from .embedding import Embedding
from .fused import apply_rope_and_append_paged_kv_cache
from .norm import fused_add_rmsnorm, fused_add_rmsnorm_quant
from .page import append_paged_kv_cache, store_kv_slots
from .rope import apply_rope_with_cos_sin_cache_inplace

__all__ = [
    "activation", "attention", "embedding", "fused", "norm", "page", "rope", "workloads", "layer_pass",
    "apply_rope_and_append_paged_kv_cache",
    "silu_and_mul", "silu_and_mul_quant", "Embedding", "fused_add_rmsnorm", "fused_add_rmsnorm_quant", "append_paged_kv_cache",
    "store_kv_slots", "apply_rope_with_cos_sin_cache_inplace", "load_library", "library_version",
]


def load_library():
    """Loads libmas_kernels.so (raises if it is not built)."""
    return _lib.load()


def library_version() -> tuple[int, int, int]:
    v = _lib.load().mas_version()
    return (v >> 16) & 0xFF, (v >> 8) & 0xFF, v & 0xFF
