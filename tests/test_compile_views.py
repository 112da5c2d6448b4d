"""torch.compile(dynamic=True) and custom ops that mutate views of the model's inputs, on the CPU.

The reference compiles its model with dynamic shapes (miniagentserve/engine/model_runner.py:98) and
hands each layer the slice ``k_cache[layer]`` of the 5-D cache it receives
(miniagentserve/models/devstral2/devstral2.py:303-304), which the KV append mutates (:170-173).
torch 2.10's Inductor has no lowering for ``aten.sym_storage_offset`` and rebuilds such slices at
offset 0, so every layer's append lands in layer 0; importing the package installs the lowering
(``_compile_fix``). These tests use small CPU custom ops shaped like the cache ops (the real ones
need a GPU) and check compiled results against eager ones for the reference's pattern and the other
view layouts the wrappers see.
"""
from __future__ import annotations

import pytest
import torch
from torch.library import custom_op


@custom_op("mas_test::append", mutates_args=("kc", "vc"))
def _append(k: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor) -> None:
    kc[0].copy_(k)
    vc[0].copy_(k * 3)


@_append.register_fake
def _(k, kc, vc):
    return None


def _layered(x, K, V):
    outs = []
    for layer in range(K.shape[0]):
        _append(x * (layer + 1), K[layer], V[layer])
        outs.append(K[layer][0] + V[layer][0])       # a reader after each layer's write
    return torch.stack(outs)


def _combined(x, KV):
    for layer in range(KV.shape[0]):
        kv = KV[layer]
        _append(x * (layer + 1), kv[:, 0], kv[:, 1])
    return KV[-1] * 2


def _whole(x, K, V):
    _append(x, K, V)
    return K + V


def _run(fn, make, x):
    want_in = make()
    want = fn(x, *want_in)
    got_in = make()
    got = torch.compile(fn, dynamic=True, fullgraph=True)(x, *got_in)
    torch._dynamo.reset()
    return want, got, want_in, got_in


@pytest.fixture(scope="module", autouse=True)
def _package(mas):
    """The package import arms the lowering fix."""
    return mas


@pytest.mark.parametrize("name,fn,make", [
    ("per_layer_slices", _layered, lambda: (torch.zeros(3, 4, 3), torch.zeros(3, 4, 3))),
    ("combined_per_layer", _combined, lambda: (torch.zeros(3, 4, 2, 3),)),
    ("whole_tensors", _whole, lambda: (torch.zeros(4, 3), torch.zeros(4, 3))),
])
def test_compiled_view_mutations_match_eager(name, fn, make):
    x = torch.randn(3, generator=torch.Generator().manual_seed(1))
    want, got, want_in, got_in = _run(fn, make, x)
    assert torch.equal(want, got), name
    for a, b in zip(want_in, got_in):
        assert torch.equal(a, b), name


def test_compiled_input_views_match_eager():
    """Inputs that are themselves slices of one storage (the per-layer call of a compiled layer)."""
    x = torch.randn(3, generator=torch.Generator().manual_seed(2))
    for pick in (lambda K, V: (K[1], V[2]), lambda K, V: (K[1], K[2])):
        K, V = torch.zeros(3, 4, 3), torch.zeros(3, 4, 3)
        K2, V2 = K.clone(), V.clone()
        _whole(x, *pick(K, V))
        torch.compile(_whole, dynamic=True, fullgraph=True)(x, *pick(K2, V2))
        torch._dynamo.reset()
        assert torch.equal(K, K2) and torch.equal(V, V2)
