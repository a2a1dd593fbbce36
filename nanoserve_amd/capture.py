"""HIP-graph capture with Python's cycle collector held off.

While a stream is being captured (torch's default "global" capture mode),
HIP refuses work on other streams that could make an implicit dependency,
and torch turns the refusal into an exception.  Some destructors issue such
work: freeing a pinned host tensor that served a `non_blocking` copy records
a completion event on every stream the copy used (torch's caching host
allocator), and an exception thrown from a storage deleter terminates the
process.  Tensors owned by objects in a reference cycle are freed whenever
the cycle collector happens to run -- possibly in the middle of a capture.

`no_cycle_collection` collects pending garbage first and then disables the
automatic collector, so the only frees during the block are the
deterministic reference-count ones of the code inside it; `graph_capture`
wraps `torch.cuda.graph` in it.
"""

from __future__ import annotations

import contextlib
import gc

import torch


@contextlib.contextmanager
def no_cycle_collection():
    """Run the block with every cycle collected up front and the collector off."""
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was_enabled:
            gc.enable()


@contextlib.contextmanager
def graph_capture(graph: "torch.cuda.CUDAGraph", stream: "torch.cuda.Stream | None" = None, pool=None):
    """`torch.cuda.graph(graph, pool=pool, stream=stream)` inside `no_cycle_collection`."""
    with no_cycle_collection():
        with torch.cuda.graph(graph, pool=pool, stream=stream):
            yield
