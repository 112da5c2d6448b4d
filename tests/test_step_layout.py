"""The forward-step workloads' layout (workloads.make_step_layout) against the rules of the
reference runner's prepare() for a captured graph step (model_runner.py:179-221): decode row i owns
token i at position seq_len - 1; prompt row j owns tokens num_decodes + cu[j] .. cu[j + 1] at its
cached positions onward; the step's token count rounds up to 64 when prompts are present, the
padding tokens going to the padding row at positions 0.. of the sink page; 17 prompt rows; every
real token's cache slot distinct and off the sink page."""
from __future__ import annotations

import dataclasses

import pytest
import torch

from conftest import __graft_entry__

wl = __graft_entry__.load_package().workloads


def _slots(lay, page_size):
    tables, pos, idx = lay.block_tables.long(), lay.positions.long(), lay.batch_indices.long()
    return tables[idx, pos // page_size] * page_size + pos % page_size


@pytest.mark.parametrize("name", sorted(wl.STEP_SHAPES))
def test_step_layout_follows_prepare(name):
    shape = wl.STEP_SHAPES[name]
    lay = wl.make_step_layout(shape, seed=0)
    d, ps = shape.decode_rows, shape.page_size
    real_prompt_tokens = sum(q for q, _ in shape.prompts)
    if shape.prompts:
        assert lay.num_tokens % 64 == 0 and lay.num_tokens >= d + real_prompt_tokens
        assert lay.num_tokens - (d + real_prompt_tokens) < 64
        assert lay.block_tables.shape[0] == d + 17 and lay.cu_seqlens_q.numel() == 18
    else:
        assert lay.num_tokens == d and lay.block_tables.shape[0] == d and lay.cu_seqlens_q.tolist() == [0]
    assert lay.block_tables.shape[1] == shape.reach // ps
    lens = lay.seq_lens.long()
    # decode rows
    assert torch.equal(lay.positions[:d].long(), lens[:d] - 1)
    assert torch.equal(lay.batch_indices[:d].long(), torch.arange(d))
    assert int(lens[:d].sum()) == lay.decode_positions and int(lens[:d].max()) <= shape.max_len
    # prompt rows: tokens after the decode tokens, at their cached positions onward
    cu = lay.cu_seqlens_q.long()
    for j, (q, c) in enumerate(shape.prompts):
        lo, hi = d + int(cu[j]), d + int(cu[j + 1])
        assert hi - lo == q and int(lens[d + j]) == q + c
        assert torch.equal(lay.positions[lo:hi].long(), torch.arange(c, c + q))
        assert bool((lay.batch_indices[lo:hi] == d + j).all())
    sink = lay.pages - 1
    if shape.prompts:
        npf, first = len(shape.prompts), d + len(shape.prompts)
        start = d + int(cu[npf])
        pad = lay.num_tokens - start
        assert int(lens[first]) == max(pad, 1) and bool((lens[first + 1:] == 1).all())
        assert bool((lay.batch_indices[start:] == first).all())
        assert torch.equal(lay.positions[start:].long(), torch.arange(pad))
        assert bool((cu[npf + 1:] == lay.num_tokens - d).all())
        assert bool((lay.block_tables[first:] == sink).all())
    # real tokens: distinct slots, none on the sink page; padding tokens on the sink page
    real = d + real_prompt_tokens
    slots = _slots(lay, ps)
    assert slots[:real].unique().numel() == real
    assert bool((slots[:real] // ps != sink).all()) and bool((slots[real:] // ps == sink).all())
    # every row's pages lie in the pool, and no two rows share a page
    used = []
    for r in range(d + len(shape.prompts)):
        k = -(-int(lens[r]) // ps)
        used.append(lay.block_tables[r, :k])
    used = torch.cat(used)
    assert used.unique().numel() == used.numel() and int(used.max()) < sink


def test_step_layout_rejects_rows_past_the_table():
    shape = dataclasses.replace(wl.STEP_SHAPES["decode_step_64x8192_40"], reach=4096)
    with pytest.raises(ValueError):
        wl.make_step_layout(shape)
