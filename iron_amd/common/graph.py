"""hipGraph capture of a launch sequence (torch.cuda.CUDAGraph on ROCm).

Garbage collection is run before and suspended during the capture: a cyclic
collection inside it can free a pinned host tensor whose pending-copy event
the host allocator then queries, which is not allowed while a stream is
capturing and ends the process. The capture error mode is thread-local, so
other threads' runtime calls are not attributed to the capture.
"""

from __future__ import annotations

import gc

import torch


def capture_graph(fn, device) -> torch.cuda.CUDAGraph:
    """Capture everything ``fn()`` launches on the current stream into a graph.

    ``fn`` must already have run eagerly once (code objects loaded, lazily
    allocated scratch in place); the captured work is not executed here.
    """
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        torch.cuda.synchronize(device)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
                fn()
        torch.cuda.current_stream(device).wait_stream(side)
        torch.cuda.synchronize(device)
    finally:
        if was_enabled:
            gc.enable()
    return graph
