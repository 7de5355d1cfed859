"""hipGraph capture shared by the whole-step and model_graph runners (the role of
fastmd/engine/_graph_capture.py:21-47, ``capture_graph`` and ``CAPTURE_ERROR_MODE``).

* Thread-local capture mode: the trajectory logger's worker thread waits on its copy events while
  the MD thread captures a window after a capacity growth; in the global mode HIP would reject that
  wait from any thread during the capture and invalidate it. The captured work is the same.
* The garbage collector is paused for the capture: a collection there may finalize an earlier,
  unreachable runner's graph, whose destruction during a capture invalidates the capture.
"""
from __future__ import annotations

import contextlib
import gc

import torch

from fastmd_amd._roctx import roctx_range

CAPTURE_ERROR_MODE = "thread_local"


@contextlib.contextmanager
def capture_graph(graph: torch.cuda.CUDAGraph, *, pool=None, stream=None, name: str = "graph_capture"):
    """``torch.cuda.graph(graph, pool=pool, stream=stream)`` in thread-local mode with the
    garbage collector paused, inside a roctx range."""
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        with roctx_range(name), torch.cuda.graph(graph, pool=pool, stream=stream,
                                                 capture_error_mode=CAPTURE_ERROR_MODE):
            yield
    finally:
        if was_enabled:
            gc.enable()
