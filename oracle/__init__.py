"""CPU oracle for the per-layer kernels - TEST INFRASTRUCTURE, NOT PRODUCT CODE.

A numpy restatement of what the reference computes on its hot path
(miniagentserve/models/devstral2/devstral2.py), written from the semantics of the calls the
reference makes, not from any kernel source:

- ``numerics``: bf16 and fp8-e4m3fn encode/decode at the bit level.
- ``ops``: fused residual-add RMSNorm (bf16 and fp8 outputs), SiluAndMul, NeoX/GPT-J RoPE from
  a cos/sin table, the paged KV append (block-table and slot forms), the embedding gather, and
  the RoPE table builders.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or as the timed CPU baseline; the library in
``mini-agent-serve_amd/`` never calls it.

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
flashinfer's own rounding choices (which the reference inherits) cannot be observed here: the
library is absent and the reference has no tests or fixtures, so agreement with flashinfer
bit for bit is "parity unpinned"; the oracle fixes one documented rounding order per op and the
GPU parity tests hold the kernels to it within the stated tolerances.
"""
from . import numerics, ops  # noqa: F401
