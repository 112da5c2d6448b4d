"""CPU oracle for the per-layer kernels - TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A numpy restatement of what the reference computes on its hot path
(miniagentserve/models/devstral2/devstral2.py), written from the semantics of the calls the
reference makes, not from any kernel source:

- ``numerics``: bf16 and fp8-e4m3fn encode/decode at the bit level.
- ``ops``: fused residual-add RMSNorm (bf16 and fp8 outputs), SiluAndMul (and with the fp8
  quantize of the down_proj input), the activation quantize, NeoX/GPT-J RoPE from a cos/sin table,
  the llama-4 query scale, the paged KV append (block-table and slot forms), the embedding gather
  and the step-input placeholder fill, paged decode and causal context attention, and the RoPE
  table builders.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the reference that results are compared against or as the timed
CPU baseline; the library in ``mini-agent-serve_amd/`` never calls it.

How each function is pinned (the tests under tests/test_oracle_*.py):
- bf16 / fp8 codecs: bit-exact against torch's own dtype conversions over exhaustive or dense
  sweeps, including ties, subnormals, saturation and NaN.
- RMSNorm: against torch.nn.functional.rms_norm and transformers' Ministral3RMSNorm, plus closed
  forms (w = 1, constant rows, zero rows); the residual output bit-exact against torch's bf16 add.
- SiluAndMul: against torch.nn.functional.silu, plus silu(0) = 0 and the large-|g| limits.
- RoPE: against transformers' apply_rotary_pos_emb / rotate_half (NeoX) and a complex multiply
  (GPT-J); position 0 is the identity bit for bit; pair norms are preserved.
- KV store / embedding: against brute-force loops and torch indexing; the block-table and slot
  forms agree.
- Tables: against transformers' default and YaRN inverse frequencies and attention factor.
- Activation quantize: bit for bit against the reference's own torch expression (y / scale, clamp
  to +-448, cast to e4m3fn) on every finite bf16 value; SiluAndMul + quantize: against SiluAndMul
  followed by that expression.
- llama-4 query scale: bit for bit against transformers' get_llama_4_attn_scale after the bf16 cast.
- Placeholder fill: the closed-form cases of the runner's rule (-1 - r -> last token of row r).
- Decode and context attention: against torch's scaled_dot_product_attention in fp32 on the
  gathered rows (grouped heads; for context rows an explicit causal mask aligned to the end of
  each row); decode also against closed forms (one position returns its value row, scale 0 the
  mean of the value rows, an empty row zeros).
flashinfer's own rounding choices (which the reference inherits) cannot be observed here: the
library is absent and the reference has no tests or fixtures, so agreement with flashinfer
bit for bit is "parity unpinned"; the oracle fixes one documented rounding order per op and the
GPU parity tests hold the kernels to it within the stated tolerances.
"""
from . import numerics, ops  # noqa: F401
