"""The ops on the model runner's own data formats: the one-transfer packed step-input buffer
(miniagentserve/engine/model_runner.py:31-63, filled at 176-225) and the per-layer slices of the
5-D KV cache (model_runner.py:82-85). Results must equal those of the same ops on standalone
contiguous tensors, bit for bit."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import bits
from oracle import ops

pytestmark = pytest.mark.gpu


def _layout(num_tokens, batch, num_prefills, max_blocks):
    """Field dtypes and shapes in the runner's order (widest dtype first, so every view is aligned):
    input_ids, positions, batch_indices, seq_lens, cu_seqlens_q, block_tables, temperatures."""
    return [(torch.int64, (num_tokens,)), (torch.int32, (num_tokens,)), (torch.int32, (num_tokens,)),
            (torch.int32, (batch,)), (torch.int32, (num_prefills + 1,)), (torch.int32, (batch, max_blocks)),
            (torch.float32, (batch,))]


def _unpack(buffer, dims):
    views, offset = [], 0
    for dtype, shape in _layout(*dims):
        n = dtype.itemsize * math.prod(shape)
        views.append(buffer[offset:offset + n].view(dtype).view(shape))
        offset += n
    return views


def test_decode_step_on_packed_inputs_and_layer_cache_slices(mas, dev):
    g = torch.Generator().manual_seed(17)
    layers, blocks, bs, hk, hq, d, hidden, vocab = 3, 64, 16, 2, 8, 128, 256, 1000
    batch = 8                                   # decode rows, one token each
    max_blocks = 6
    dims = (batch, batch, 0, max_blocks)
    size = sum(dt.itemsize * math.prod(sh) for dt, sh in _layout(*dims))
    host = torch.zeros(size, dtype=torch.uint8)
    ids, pos, idx, lens, cu, tables, temps = _unpack(host, dims)
    seq_lens = torch.randint(1, max_blocks * bs, (batch,), generator=g)
    ids.copy_(-1 - torch.arange(batch))                        # every token is the previous step's sample
    pos.copy_(seq_lens - 1)
    idx.copy_(torch.arange(batch))
    lens.copy_(seq_lens)
    tables.copy_(torch.randperm(blocks, generator=g)[: batch * max_blocks].reshape(batch, max_blocks))
    temps.fill_(1.0)
    buf = host.to(dev)
    ids_d, pos_d, idx_d, _, _, tables_d, _ = _unpack(buf, dims)

    last = torch.randint(0, vocab, (batch,), generator=g).to(torch.int32).to(dev)
    weight = torch.randn(vocab, hidden, generator=g).bfloat16().to(dev)
    emb = mas.embedding.embedding(ids_d, weight, last_tokens=last)
    want_ids = ops.fill_placeholders((-1 - np.arange(batch)), last.cpu().numpy())
    assert np.array_equal(ids_d.cpu().numpy(), want_ids)
    assert np.array_equal(bits(emb), ops.embedding(bits(weight.cpu()), want_ids))

    k_cache = torch.zeros(layers, blocks + 1, bs, hk, d, dtype=torch.bfloat16, device=dev)
    v_cache = torch.zeros_like(k_cache)
    kv_indptr = torch.arange(batch + 1, dtype=torch.int32, device=dev) * max_blocks   # devstral2.py:289
    table = mas.rope.cos_sin_cache(max_blocks * bs, d, 1e6).to(dev)
    qkv0 = torch.randn(batch, (hq + 2 * hk) * d, generator=g).bfloat16().to(dev)
    layer = 1
    qkv = qkv0.clone()
    q, k, v = qkv.split([hq * d, hk * d, hk * d], dim=-1)
    mas.apply_rope_and_append_paged_kv_cache(pos_d, q, k, v.view(batch, hk, d), d, table, True, idx_d,
                                             (k_cache[layer], v_cache[layer]), tables_d.flatten(), kv_indptr)

    # the same on standalone tensors
    kc = torch.zeros(blocks + 1, bs, hk, d, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    qkv2 = qkv0.clone()
    q2, k2, v2 = qkv2.split([hq * d, hk * d, hk * d], dim=-1)
    mas.apply_rope_and_append_paged_kv_cache(pos_d.clone(), q2, k2, v2.view(batch, hk, d), d, table, True,
                                             idx_d.clone(), (kc, vc), tables_d.flatten().clone(), kv_indptr)
    assert torch.equal(qkv, qkv2)
    assert torch.equal(k_cache[layer], kc) and torch.equal(v_cache[layer], vc)
    assert not k_cache[0].any() and not k_cache[2].any()      # other layers untouched
    # and the cache holds each token's rotated k at its page slot
    for t in range(batch):
        p = int(seq_lens[t]) - 1
        page = int(tables[t, p // bs])
        assert torch.equal(k_cache[layer, page, p % bs], k.view(batch, hk, d)[t])
