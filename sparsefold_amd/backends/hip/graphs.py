"""HIP-graph replay of repeated module calls (opt-in: ``configure_runtime(hip_graphs=True)`` or
``SPARSEFOLD_HIP_GRAPHS=1``).

A HIP module call launches 5-17 short kernels; at the configurations' sizes the host cost of
those launches (and of the Python around them) exceeds the GPU time of the call.  With graphs on,
a module call whose *signature* -- every tensor argument's address, shape, strides, dtype and
device, plus every scalar argument -- repeats is captured once (on its second occurrence) and
from then on replayed as one graph launch.

Replay reads the inputs at the captured addresses, so a call that passes the same tensors (or
new tensors at the same addresses, as a steady-state loop with torch's caching allocator does)
sees its current values; nothing is copied in.  Intermediates live in the graph's private pool;
the output is the graph's static buffer, returned as a copy (the module's contract is a fresh
tensor).  The per-module cache is LRU-bounded and is cleared whenever the module re-packs its
weights (``prepare_native``).  Calls made while another capture is running, or with arguments
that are neither tensors nor plain scalars, run eagerly.
"""
from __future__ import annotations

import collections
import functools

import torch

from sparsefold_amd.runtime import config

MAX_GRAPHS_PER_MODULE = 4
_SEEN = object()


def _signature(args, kwargs):
  parts = []
  for value in list(args) + [kwargs[k] for k in sorted(kwargs)]:
    if value is None or isinstance(value, (bool, int, float, str)):
      parts.append(value)
    elif isinstance(value, torch.Tensor):
      if value.device.type != "cuda" or value.requires_grad:
        return None
      parts.append((value.data_ptr(), tuple(value.shape), value.stride(), value.dtype, value.device.index))
    else:
      return None
  return tuple(sorted(kwargs)), tuple(parts)


def clear(module) -> None:
  module.__dict__.pop("_hip_graph_cache", None)


def graphed(forward):
  """Decorator for a HIP module's ``forward`` (or ``forward_indexed``)."""

  @functools.wraps(forward)
  def wrapped(self, *args, **kwargs):
    if not config.hip_graphs:
      return forward(self, *args, **kwargs)
    key = _signature(args, kwargs)
    if key is None or torch.cuda.is_current_stream_capturing():
      return forward(self, *args, **kwargs)
    key = (forward.__name__, key)
    cache = self.__dict__.setdefault("_hip_graph_cache", collections.OrderedDict())
    entry = cache.get(key)
    if entry is None:                       # first occurrence: eager (also warms the allocator)
      cache[key] = _SEEN
      while len(cache) > 2 * MAX_GRAPHS_PER_MODULE:
        cache.popitem(last=False)
      return forward(self, *args, **kwargs)
    if entry is _SEEN:                      # second occurrence: capture, then replay below
      graph = torch.cuda.CUDAGraph()
      with torch.cuda.graph(graph):
        out = forward(self, *args, **kwargs)
      entry = (graph, out)
      cache[key] = entry
      captured = [k for k, v in cache.items() if v is not _SEEN]
      while len(captured) > MAX_GRAPHS_PER_MODULE:
        del cache[captured.pop(0)]
    cache.move_to_end(key)
    graph, out = entry
    graph.replay()
    return out.clone()

  return wrapped
