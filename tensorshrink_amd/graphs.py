"""CUDAGraphQuantModel: a quantized model's forward captured once per input
shape as a HIP graph and replayed (modules.py:1589-1691).

A decode step runs each layer's kernel in a few microseconds, about what it
takes Python and the HIP runtime to launch it; replaying a graph issues the
whole step's launches from one call. The QuantLinear kernels are capturable:
their launches take only the stream, read the layer's resident buffers, and
make no allocation, host synchronization or memset.

Same interface as the reference: `CUDAGraphQuantModel(model, warmup_runs=3)`,
call it like the model, `release()`. Differences, all at the API edge:
- the shape key also holds dtype and device, so a bf16 call never replays an
  fp16 graph;
- warmup runs on a side stream (lazy one-time work such as library handles
  and kernel attributes happens before capture, outside the graph);
- graphs of one wrapper share one memory pool, so the captured shapes do not
  each reserve their own activations;
- outputs may be a tensor or a tuple/list/dict of them (HF model outputs):
  each tensor is cloned out of the graph's static buffer on return, as the
  reference clones its single output.
"""
from __future__ import annotations

from typing import Any, Dict, Tuple

import torch
import torch.nn as nn


def _tensors_key(args, kwargs) -> Tuple:
    key = tuple((tuple(a.shape), a.dtype, a.device) for a in args if isinstance(a, torch.Tensor))
    for k in sorted(kwargs):
        v = kwargs[k]
        if isinstance(v, torch.Tensor):
            key += ((k, tuple(v.shape), v.dtype, v.device),)
    return key


def _clone_out(o: Any) -> Any:
    if isinstance(o, torch.Tensor):
        return o.clone()
    if isinstance(o, (list, tuple)) and not hasattr(o, "_fields"):
        return type(o)(_clone_out(x) for x in o)
    if isinstance(o, dict):
        out = o.__class__() if o.__class__ is not dict else {}
        for k, v in o.items():
            out[k] = _clone_out(v)
        return out
    return o


class _CapturedGraph:
    """One captured graph with its static inputs and output (modules.py:1671-1691)."""

    def __init__(self, graph, static_args, static_kwargs, static_output):
        self.graph = graph
        self.static_args = static_args
        self.static_kwargs = static_kwargs
        self.static_output = static_output

    def replay(self, args, kwargs):
        for sa, a in zip(self.static_args, args):
            if isinstance(sa, torch.Tensor) and isinstance(a, torch.Tensor):
                sa.copy_(a)
        for k, v in kwargs.items():
            if isinstance(v, torch.Tensor) and k in self.static_kwargs:
                self.static_kwargs[k].copy_(v)
        self.graph.replay()
        return _clone_out(self.static_output)


class CUDAGraphQuantModel:
    """Replays a captured graph of `model`'s forward for every input shape
    seen before; the first call with a new shape runs `warmup_runs` eager
    forwards and captures (modules.py:1589-1668)."""

    def __init__(self, model: nn.Module, warmup_runs: int = 3):
        self.model = model
        self.warmup_runs = warmup_runs
        self._graphs: Dict[Tuple, _CapturedGraph] = {}
        self._pool = None

    def __call__(self, *args, **kwargs):
        if not torch.cuda.is_available():
            return self.model(*args, **kwargs)
        key = _tensors_key(args, kwargs)
        g = self._graphs.get(key)
        if g is None:
            g = self._graphs[key] = self._capture(args, kwargs)
        return g.replay(args, kwargs)

    def _capture(self, args, kwargs) -> _CapturedGraph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(self.warmup_runs):
                self.model(*args, **kwargs)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        static_args = tuple(a.clone() if isinstance(a, torch.Tensor) else a for a in args)
        static_kwargs = {k: v.clone() if isinstance(v, torch.Tensor) else v for k, v in kwargs.items()}
        if self._pool is None:
            self._pool = torch.cuda.graph_pool_handle()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self._pool):
            out = self.model(*static_args, **static_kwargs)
        return _CapturedGraph(graph, static_args, static_kwargs, out)

    def release(self) -> None:
        """Drop every captured graph (and with the last one its memory pool)."""
        self._graphs.clear()
        self._pool = None

    def __del__(self):
        self.release()
