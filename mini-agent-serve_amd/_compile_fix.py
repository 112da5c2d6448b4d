"""Inductor lowering for ``aten.sym_storage_offset``, which torch 2.10's Inductor lacks.

Under ``torch.compile(dynamic=True)`` (the reference's mode, miniagentserve/engine/model_runner.py:98),
a custom op that mutates a view of a graph input - the per-layer cache slice ``k_cache[layer]`` of
the 5-D cache the model receives (miniagentserve/models/devstral2/devstral2.py:303-304, :170-173) -
is functionalized with the view's metadata, and the view is rebuilt before the op runs as
``as_strided(base, size, stride, sym_storage_offset(select(base, 0, layer)))``. Inductor has
lowerings for ``sym_size`` and ``sym_stride`` but none for ``sym_storage_offset``, so it falls back
to running that op on an example tensor rebuilt from the view's layout, whose offset is always 0:
every layer's slice then aliases layer 0, and the KV append of layer l silently overwrites layer 0.

The lowering added here returns the view's offset as Inductor itself accounts offsets: relative to
the buffer the view's storage starts at (a graph input's own storage offset is not part of its
buffer layout), read from the view's layout once it is expressed as a reinterpretation of that
buffer. It is installed only if torch has no lowering for the op, and only when Inductor's lowering
module is loaded (right away if it already is, else by a one-shot import hook), so importing this
package does not import the compiler.

Not covered (a torch limitation, with or without this lowering): a compiled function whose *input*
is itself a view with a nonzero storage offset, and which passes sub-views of that input to a
mutating custom op. The view metadata then carries the sub-view's absolute offset as a constant,
which Inductor reads as relative to the input. Per-layer slices taken inside the compiled model, as
the reference takes them, and inputs passed whole are handled; the wrappers pass a combined
``[pages, 2, ...]`` cache whole and split it inside the op, so they create no such sub-view.
"""
from __future__ import annotations

import importlib.abc
import importlib.machinery
import sys
import threading

import torch

_MODULE = "torch._inductor.lowering"
_lock = threading.Lock()
_installed = False


def install() -> bool:
    """Registers the lowering if Inductor has none for the op; returns whether one is now present."""
    global _installed
    with _lock:
        if _installed:
            return True
        from torch._inductor import ir, lowering

        op = torch.ops.aten.sym_storage_offset.default
        if op not in lowering.lowerings:
            @lowering.register_lowering(op)
            def _sym_storage_offset(a):
                x = a.data if isinstance(a, ir.TensorBox) else a
                if isinstance(x, ir.BaseView):
                    x = ir.ExternKernel.convert_to_reinterpret_view(x)
                return x.get_layout().offset
        _installed = True
        return True


class _Loader(importlib.abc.Loader):
    def __init__(self, inner):
        self._inner = inner

    def create_module(self, spec):
        return self._inner.create_module(spec)

    def exec_module(self, module):
        self._inner.exec_module(module)
        install()


class _Finder(importlib.abc.MetaPathFinder):
    """Wraps the loader of Inductor's lowering module so ``install`` runs right after it loads."""

    def find_spec(self, name, path, target=None):
        if name != _MODULE:
            return None
        sys.meta_path.remove(self)
        spec = importlib.machinery.PathFinder.find_spec(name, path)
        if spec is not None and spec.loader is not None:
            spec.loader = _Loader(spec.loader)
        return spec


def arm() -> None:
    """Installs the lowering now if Inductor is loaded, else when it is first imported."""
    if _MODULE in sys.modules:
        install()
    elif not any(isinstance(f, _Finder) for f in sys.meta_path):
        sys.meta_path.insert(0, _Finder())
