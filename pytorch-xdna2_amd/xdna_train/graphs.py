"""Graph capture for the xdna device.

A training step of hundreds of small operators is bound by launch and dispatch cost on
the host; captured once as a HIP graph it replays with one launch.  ``Graph`` pairs a
``torch.cuda.CUDAGraph`` (which captures PyTorch-ROCm's stream and keeps a private pool of
its caching allocator for the operators served by the ROCm fallback) with a private pool
of the xdna caching allocator (``xdna_hip_cache_pool_*`` in include/xdna_hip.h), so the
memory the captured kernels use is not handed to other work while the graph can replay.

The reference has no graph capture (its NPU path is host-driven); the usage mirrors
``torch.cuda.graph``:

    g = torch.xdna.Graph()
    step()                              # warm up eagerly (library plans, lazy state)
    with torch.xdna.graph(g):
        loss = step()                   # captured, not run
    for _ in range(n):
        g.replay()                      # loss now holds this replay's value

Captured work must be stream-ordered device work only: no host reads of device values
(``.item()``, prints), no host-side branching on them, constant shapes.
"""

from __future__ import annotations

import contextlib
import weakref

import torch

from . import device as _device


def _release(cuda_graph, pool: int) -> None:
    try:
        cuda_graph.reset()
    finally:
        _device.native().release_graph_weights(pool)
        _device.native().pool_release(pool)


class Graph:
    """A captured sequence of xdna (and PyTorch-ROCm) work, replayed with ``replay()``."""

    def __init__(self):
        ext = _device.native()
        self._cuda = torch.cuda.CUDAGraph()
        self._pool = int(ext.pool_create())
        self._release = weakref.finalize(self, _release, self._cuda, self._pool)

    @property
    def pool(self) -> int:
        """Id of the private xdna allocator pool of this graph."""
        return self._pool

    def replay(self) -> None:
        """Launches the captured work on the current stream.  First, the prepared forms of
        frozen conv weights the graph adopted are prepared again where the weight was
        written since.  The backend's host caches of forms derived from tensors (prepared
        conv weights, kept packs) stop serving entries made before the replay, whose
        tensors the graph may have rewritten."""
        ext = _device.native()
        ext.refresh_graph_weights(self._pool)
        ext.note_graph_replay()
        self._cuda.replay()

    def reset(self) -> None:
        """Frees the graph and returns its memory to the shared pools."""
        self._release()


@contextlib.contextmanager
def graph(g: Graph, stream: torch.cuda.Stream | None = None, capture_error_mode: str = "global"):
    """Captures the xdna work of the ``with`` body into ``g`` (see the module docstring)."""
    if not isinstance(g, Graph):
        raise TypeError("torch.xdna.graph expects a torch.xdna.Graph")
    _device.synchronize()
    with torch.cuda.graph(g._cuda, stream=stream, capture_error_mode=capture_error_mode):
        _device.native().pool_begin(g.pool)
        try:
            yield g
        finally:
            _device.native().pool_end()


# torch.xdna.Graph / torch.xdna.graph, next to torch.xdna.synchronize and the others
_device._device_module.Graph = Graph
_device._device_module.graph = graph
