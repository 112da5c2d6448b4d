"""The whole-step workload (layer_pass.ForwardStep, the bench's decode and mixed steps) at a small
size, after one run of the step: the residual stream equals the oracle's chain of fused adds over
the embedding and every layer's stand-ins, bit for bit; the last layer's KV cache holds every real
token's rotated key and its value at the slot its row's block table gives; the attention output
(the o_proj input quantize) of the decode rows and of the prompt rows is the oracle's attention of
the rotated queries over that cache, quantized, within one e4m3 step plus the bf16 tolerance
(rtol 1.6e-2, atol 1e-2) divided by the scale; and so is the last SiluAndMul + quantize output.
The residual chain, the cache rows and the layout are the bit-exact checks. Two fixed steps (5
decode rows, with and without a prompt) and six seeded ones (1-12 decode rows, 0-3 prompts, pages
of 16-256 slots)."""
from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from conftest import bits, fp8_codes
from oracle import numerics as on
from oracle import ops

pytestmark = pytest.mark.gpu


def _step(mas, dev, prompts, decode_rows=5, max_len=300, page_size=16, reach=512, seed=3):
    wl = mas.workloads
    layer = dataclasses.replace(wl.SHAPES["decode64_24b"], vocab=4096)
    shape = wl.StepShape("test_step", decode_rows=decode_rows, max_len=max_len, prompts=prompts, layers=2,
                         page_size=page_size, reach=reach, layer=layer)
    fs = mas.layer_pass.ForwardStep(shape, dev, seed=seed)
    final_in = bits(fs.final_in)   # the final norm writes its output over its input
    fs.run()
    torch.cuda.synchronize()
    return fs, final_in


def _fp8_close(got_codes, want_codes, scale):
    """Within one e4m3 step of the oracle's quantize, plus the bf16 tolerance of the value before the
    quantize (rtol 1.6e-2, atol 1e-2) carried through the division by the scale."""
    got, want = on.fp8_to_f32(got_codes), on.fp8_to_f32(want_codes)
    step = np.maximum(np.abs(want) * 2.0 ** -3, 2.0 ** -9) + 1.6e-2 * np.abs(want) + 1e-2 / scale
    assert np.all(np.abs(got - want) <= step)


def _random_step(seed):
    """1-12 decode rows up to 40-600 positions, 0-3 prompts of 1-60 new tokens after 0-400 cached,
    pages of 16, 64 or 256 slots, a 1024-position table."""
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 4)) if rng.random() < 0.75 else 0
    prompts = tuple((int(rng.integers(1, 61)), int(rng.integers(0, 401))) for _ in range(n))
    return dict(prompts=prompts, decode_rows=int(rng.integers(1, 13)), max_len=int(rng.integers(40, 601)),
                page_size=int(rng.choice([16, 64, 256])), reach=1024, seed=seed)


CASES = [dict(prompts=()), dict(prompts=((20, 50),))] + [_random_step(700 + k) for k in range(6)]


@pytest.mark.parametrize("case", CASES, ids=["decode", "mixed"] + [f"seed{700 + k}" for k in range(6)])
def test_forward_step_against_the_oracle(mas, dev, case):
    fs, final_in = _step(mas, dev, **case)
    ls, lay = fs.shape.layer, fs.layout
    n, d = fs.num_tokens, fs.num_decodes
    scale = float(fs.act_scale)
    # the residual stream: embedding, then per layer the two sublayer stand-ins, then the final input
    ids = fs.ids.cpu().numpy()
    r = np.zeros((n, ls.hidden), dtype=np.uint16)
    inputs = [ops.embedding(bits(fs.embed_table), ids)]
    for i, layer in enumerate(fs.layers):
        if i > 0:
            inputs.append(bits(layer["hidden"]))
        inputs.append(bits(layer["o_proj"]))
    inputs.append(final_in)
    for x in inputs[:-1]:
        r = on.f32_to_bf16(on.bf16_to_f32(r) + on.bf16_to_f32(x))
    assert np.array_equal(bits(fs.layers[0]["hidden"]), inputs[0])   # the gather's output, layer 0's input
    want_r = on.f32_to_bf16(on.bf16_to_f32(r) + on.bf16_to_f32(inputs[-1]))
    assert np.array_equal(bits(fs.residual), want_r)
    # the last layer's cache and attention
    last = fs.layers[-1]
    q, k, v = fs.views(last)
    kc, vc = bits(last["k_cache"]), bits(last["v_cache"])
    tables, lens = lay.block_tables.numpy(), lay.seq_lens.numpy()
    pos, idx = lay.positions.numpy(), lay.batch_indices.numpy()
    real = d + sum(qn for qn, _ in fs.shape.prompts)
    ps = fs.shape.page_size
    kb, vb = bits(k).reshape(n, ls.kv_heads, ls.head_dim), bits(v)
    for t in range(real):
        page, e = tables[idx[t], pos[t] // ps], pos[t] % ps
        assert np.array_equal(kc[page, e], kb[t]) and np.array_equal(vc[page, e], vb[t])
    qb = bits(q).reshape(n, ls.q_heads, ls.head_dim)
    got = fp8_codes(fs.attn_out)
    if d:
        att = ops.paged_decode_attention(qb[:d], kc, vc, tables[:d], lens[:d], fs.scale)
        _fp8_close(got[:d], ops.quantize_activation(att, scale), scale)
    if fs.shape.prompts:
        att = ops.paged_context_attention(qb[d:], kc, vc, tables[d:], lens[d:], lay.cu_seqlens_q.numpy(), fs.scale)
        _fp8_close(got[d:real], ops.quantize_activation(att, scale)[:real - d], scale)
    _fp8_close(fp8_codes(fs.silu_out), ops.silu_and_mul_quant(bits(last["gate_up"]), scale), scale)
