"""Streaming QuantLinear weights from pinned host memory (streaming.py:1-272).

`StreamingQuantModel` keeps every QuantLinear's weight buffers in pinned
host memory and copies a layer's buffers to the GPU just before its forward,
prefetching the next `prefetch_depth` layers (in named_modules order) on a
copy stream while the current one computes, and dropping the GPU copy after
the forward returns. The bias stays resident on the GPU, as in the reference.

MI355X layout: a layer's buffers are packed into ONE pinned host block
(each buffer at a 256-byte aligned offset), so a prefetch is one
host-to-device copy into one device block whose views become the layer's
buffers; the layer's kernel view is rebuilt on the new addresses. Every
buffer whose size follows the layer's is streamed: packed, scale/gmin or the
double-quant codes and metadata (the reference's list misses the
double-quant set, streaming.py:57-67), 6-bit stage-2 buffers, the outlier
tables and their derived row offsets, per-tile slots and column-sorted copy.
The f32 codebook (at most 256 entries) stays resident.

With 288 GB of HBM per MI355X a quantized model rarely needs this; it is the
reference's answer for a model whose packed weights exceed the GPU.
"""
from __future__ import annotations

import dataclasses
from typing import Dict, List, Optional, Tuple

import torch

from .modules import QuantLinear

_STREAMED = ("packed", "scale", "gmin", "dq_scale_codes", "dq_scale_meta", "dq_gmin_codes", "dq_gmin_meta",
             "stage2_packed", "stage2_scale", "stage2_gmin", "outlier_row", "outlier_col", "outlier_delta",
             "outlier_row_ptr", "tile_outliers", "outlier_colsorted")
_ALIGN = 256


@dataclasses.dataclass
class _LayerState:
    host: torch.Tensor                                # pinned uint8 block
    layout: Dict[str, Tuple[int, torch.dtype, Tuple[int, ...]]]  # name -> (offset, dtype, shape)
    host_views: Dict[str, torch.Tensor]
    gpu: Optional[torch.Tensor] = None                # device uint8 block while streamed in
    event: Optional["torch.cuda.Event"] = None
    prefetched: bool = False


def _views(block: torch.Tensor, layout) -> Dict[str, torch.Tensor]:
    out = {}
    for name, (off, dt, shape) in layout.items():
        n = 1
        for d in shape:
            n *= d
        nbytes = n * torch.empty(0, dtype=dt).element_size()
        out[name] = block[off:off + nbytes].view(dt).view(shape)
    return out


class StreamingQuantModel:
    """Pre/post forward hooks on every QuantLinear of `model` that stream its
    buffers in and out (streaming.py:85-244)."""

    def __init__(self, model: torch.nn.Module, device: str = "cuda", prefetch_depth: int = 1,
                 pin_memory: bool = True, verbose: bool = True):
        if not torch.cuda.is_available():
            raise RuntimeError("StreamingQuantModel requires a ROCm device")
        self.model = model
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self.prefetch_depth = max(1, int(prefetch_depth))
        self._pin_memory = pin_memory
        self._verbose = verbose
        self._layers: List[Tuple[str, QuantLinear]] = [(n, m) for n, m in model.named_modules()
                                                       if isinstance(m, QuantLinear)]
        if not self._layers:
            raise ValueError("model has no QuantLinear layers to stream")
        self._copy_stream = torch.cuda.Stream(device=self.device)
        self._handles: List = []
        self._enabled = False
        self._states: List[_LayerState] = []
        self._prepare_host_buffers()

    # -- setup ---------------------------------------------------------------
    def _prepare_host_buffers(self) -> None:
        total = 0
        for _, q in self._layers:
            layout, off = {}, 0
            bufs = {n: q._kernel_tensor(n) for n in _STREAMED if q._kernel_tensor(n) is not None}
            for n, t in bufs.items():
                layout[n] = (off, t.dtype, tuple(t.shape))
                off += (t.numel() * t.element_size() + _ALIGN - 1) // _ALIGN * _ALIGN
            host = torch.empty(max(off, _ALIGN), dtype=torch.uint8, pin_memory=self._pin_memory)
            hv = _views(host, layout)
            for n, t in bufs.items():
                hv[n].copy_(t.detach())  # device -> host (synchronous)
            total += off
            keep = dict(hv)  # host-resident; a GPU copy exists only while streamed in
            if q.bias is not None:
                keep["bias"] = q.bias.detach().to(self.device)
            if q.codebook is not None:
                keep["codebook"] = q.codebook.to(self.device)
            q._set_tensors(keep)
            self._states.append(_LayerState(host=host, layout=layout, host_views=hv))
        if self._verbose:
            print(f"  streaming: {len(self._layers)} QuantLinear layers pinned in host RAM "
                  f"({total / 1e6:.1f}MB, prefetch_depth={self.prefetch_depth})")

    # -- per-layer prefetch / release -----------------------------------------
    def _prefetch(self, idx: int) -> None:
        if idx < 0 or idx >= len(self._layers) or self._states[idx].prefetched:
            return
        st = self._states[idx]
        compute = torch.cuda.current_stream(self.device)
        with torch.cuda.stream(self._copy_stream):
            gpu = torch.empty(st.host.numel(), dtype=torch.uint8, device=self.device)
            gpu.copy_(st.host, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(self._copy_stream)
        # allocated on the copy stream, read on the compute stream: the
        # allocator must not reuse it before the compute stream is done
        gpu.record_stream(compute)
        st.gpu, st.event, st.prefetched = gpu, ev, True

    def _swap_in(self, idx: int) -> None:
        _, q = self._layers[idx]
        st = self._states[idx]
        q._set_tensors(_views(st.gpu, st.layout))

    def _release(self, idx: int) -> None:
        _, q = self._layers[idx]
        st = self._states[idx]
        if not st.prefetched:
            return
        q._set_tensors(st.host_views)
        st.gpu, st.event, st.prefetched = None, None, False

    # -- hooks ---------------------------------------------------------------
    def _pre_hook(self, idx: int):
        def hook(module, inputs):
            self._prefetch(idx)  # no-op when already in flight
            torch.cuda.current_stream(self.device).wait_event(self._states[idx].event)
            self._swap_in(idx)
            for j in range(idx + 1, min(idx + 1 + self.prefetch_depth, len(self._layers))):
                self._prefetch(j)
            return None
        return hook

    def _post_hook(self, idx: int):
        def hook(module, inputs, output):
            self._release(idx)
            return None
        return hook

    # -- lifecycle -------------------------------------------------------------
    def enable(self) -> "StreamingQuantModel":
        if self._enabled:
            return self
        for idx, (_, q) in enumerate(self._layers):
            self._handles.append(q.register_forward_pre_hook(self._pre_hook(idx)))
            self._handles.append(q.register_forward_hook(self._post_hook(idx)))
        self._enabled = True
        return self

    def disable(self) -> None:
        for h in self._handles:
            h.remove()
        self._handles.clear()
        self._enabled = False
        for idx in range(len(self._layers)):
            self._release(idx)

    def stats(self) -> dict:
        host_bytes = sum(st.host.numel() for st in self._states)
        on = [st for st in self._states if st.prefetched]
        return {"n_layers": len(self._layers), "host_bytes": host_bytes, "layers_currently_on_gpu": len(on),
                "gpu_resident_bytes": sum(st.gpu.numel() for st in on)}


def stream_offload_module(model: torch.nn.Module, device: str = "cuda", vram_budget_mb: Optional[float] = None,
                          prefetch_depth: Optional[int] = None, pin_memory: bool = True,
                          verbose: bool = True) -> StreamingQuantModel:
    """Build and enable a StreamingQuantModel (streaming.py:247-272): the
    prefetch depth is `prefetch_depth`, else as many average layers as
    `vram_budget_mb` holds less the one computing, else 1."""
    layers = [m for _, m in model.named_modules() if isinstance(m, QuantLinear)]
    if not layers:
        raise ValueError("model has no QuantLinear layers to stream")
    depth = prefetch_depth
    if depth is None:
        if vram_budget_mb is not None:
            avg = sum(q.packed_nbytes() for q in layers) / len(layers)
            depth = max(1, int(vram_budget_mb * 1024 * 1024 // max(1, avg)) - 1)
        else:
            depth = 1
    return StreamingQuantModel(model, device=device, prefetch_depth=depth, pin_memory=pin_memory,
                               verbose=verbose).enable()
