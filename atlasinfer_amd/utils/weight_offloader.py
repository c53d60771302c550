"""Weight streaming for models whose quantized weights live in host memory.

Same names and hook interface as the reference module
/root/reference/atlasinfer_core/utils/weight_offloader.py (also importable
as ``atlasinfer_core.utils.weight_offloader``):

* ``QuantizedTensorOffloadHook`` (reference :48-177) -- an accelerate
  ``AlignDevicesHook`` attached to a decoder block (or the final norm, or the
  lm_head).  ``pre_forward`` puts the module's weights on the execution
  device and moves the call's tensors there; ``post_forward`` (with
  ``offload=True``) takes the weights back to their home and drops the
  dequantized fp16 copies the quantizer cached for them.
* ``_clear_specific_dequant_cache`` / ``clear_all_dequant_cache``
  (reference :28-44) -- act on the quantizer's own dequantization cache.

What differs from the reference, which (a) relied on ``module.to`` to move
``QuantizedLinear`` weights although they are plain attributes that
``nn.Module.to`` does not see, so they reached the GPU only through the
layer's lazy move and never left it, (b) cleared a cache dictionary of its
own that nothing else fills, so dequantized fp16 weights piled up on the GPU,
and (c) turned the hooked module's direct parameters into meta tensors in
``init_hook`` (accelerate's offload set-up), after which ``module.to`` fails:

* ``QuantizedLinear`` weights and biases move with their module
  (``QuantizedLinear._apply``) and come back in ``post_forward``;
* the quantizer's cache entries of the module's weights are dropped;
* ``init_hook`` leaves the module as it is;
* with a ``WeightStreamer`` (``setup_offloading_hooks`` in
  ``integration.model_modifier`` creates one), a module's tensors are packed
  into one page-locked host buffer and cross to the GPU in one copy on a side
  stream, one or more modules ahead of their use, so the copies overlap the
  previous modules' kernels (one copy per tensor costs a launch each: about
  60 per OPT-1.3b block, which held a streamed decode at two thirds of the
  link rate).  The compute stream waits for a module's copy with an event;
  the device copy is released after its forward and is not reused by the
  allocator before the kernels that read it have run (``record_stream``).
"""
from __future__ import annotations

import threading
from typing import Any, Dict, List, Optional

import torch
import torch.nn as nn
from accelerate.hooks import AlignDevicesHook

from ..quant import adaptive_quantizer as _aq
from ..quant.adaptive_quantizer import QuantizedTensor
from .helpers import map_structure  # noqa: F401  (re-exported, as the reference's module does)

_QT_TENSOR_FIELDS = ("fp8_data", "fp16_outliers", "outlier_indices", "scale_factors", "outlier_row_ptr",
                     "outlier_cols", "outlier_tile_ptr", "outlier_tile_ent")


def _clear_specific_dequant_cache(obj_id: int) -> None:
    """Drop the quantizer's cached fp16 copy of the QuantizedTensor with this
    id (reference :28-34, which cleared a dictionary of its own)."""
    _aq.discard_dequantized(obj_id)


def clear_all_dequant_cache() -> None:
    """Drop every cached fp16 weight (reference :36-44)."""
    _aq.clear_dequantized_cache()


def _is_qlinear(m) -> bool:
    return type(m).__name__ == "QuantizedLinear"


_ALIGN = 256  # byte alignment of each tensor inside a module's packed buffer


class _Entry:
    """One streamed module: its parameters, buffers and QuantizedLinear
    weights packed into one page-locked host buffer (each tensor a view at a
    256-byte aligned offset), so that the module crosses to the device in a
    single copy, and the device copy while it exists."""

    def __init__(self, module: nn.Module):
        self.module = module
        seen = set()
        srcs = []           # every tensor, in slot order
        self.qlinears = []  # (layer, QuantizedTensor, fields present, has bias)
        for m in module.modules():
            if _is_qlinear(m):
                q, b = m.quantized_weights, m.bias
                fields = [f for f in _QT_TENSOR_FIELDS if getattr(q, f) is not None]
                srcs += [getattr(q, f) for f in fields]
                if b is not None:
                    seen.add(id(b))
                    srcs.append(b)
                self.qlinears.append((m, q, fields, b is not None))
        self.params = []  # parameters
        for p in module.parameters():
            if id(p) not in seen:
                seen.add(id(p))
                self.params.append(p)
                srcs.append(p.data)
        self.buffers = []  # (owner, name)
        for owner in module.modules():
            for name, b in list(owner._buffers.items()):
                if b is not None and id(b) not in seen:
                    seen.add(id(b))
                    self.buffers.append((owner, name))
                    srcs.append(b)
        self.slots = []  # (offset, bytes, dtype, shape)
        off = 0
        for t in srcs:
            nb = t.numel() * t.element_size()
            self.slots.append((off, nb, t.dtype, tuple(t.shape)))
            off += (nb + _ALIGN - 1) // _ALIGN * _ALIGN
        self.nbytes = off
        self.host = torch.empty(max(off, 1), dtype=torch.uint8, pin_memory=True)
        for v, t in zip(self._views(self.host), srcs):
            v.copy_(t.detach())
        self.host_views = self._views(self.host)
        self._install(self.host_views)
        self.dev = None        # (device buffer, its views, event) once copied
        self.installed = False

    def _views(self, base: torch.Tensor):
        return [base[o:o + nb].view(dt).view(shape) for o, nb, dt, shape in self.slots]

    def _install(self, views):
        """Point the module's tensors at ``views`` (slot order); returns the
        QuantizedTensors installed."""
        it = iter(views)
        qts = []
        for m, q, fields, has_bias in self.qlinears:
            nq = q._replace(**{f: next(it) for f in fields})
            m._set_weights(nq, next(it) if has_bias else None)
            qts.append(nq)
        for p in self.params:
            p.data = next(it)
        for owner, name in self.buffers:
            owner._buffers[name] = next(it)
        return qts


class WeightStreamer:
    """Keeps the weights of an ordered list of modules in pinned host memory
    and brings each to ``device`` for its forward, copying the next
    ``depth`` modules (in registration order, cyclically: after the last
    module the first ones, for the next step) on a side stream meanwhile."""

    def __init__(self, device, depth: int = 1):
        device = torch.device(device)
        if device.type != "cuda":
            raise ValueError(f"WeightStreamer streams to a HIP device, got {device}")
        if device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        if depth < 0:
            raise ValueError(f"depth must be >= 0, got {depth}")
        self.device = device
        self.depth = int(depth)
        self.entries: List[_Entry] = []
        self._pos: Dict[int, int] = {}
        self._stream = None
        self._lock = threading.Lock()
        # uploads issued ahead of use / at use; bytes copied to the device
        self.stats = {"prefetched": 0, "on_demand": 0, "bytes": 0}

    def register(self, module: nn.Module) -> int:
        """Add ``module`` as the next one in forward order: its weights move
        to pinned host memory.  Returns its position."""
        if id(module) in self._pos:
            return self._pos[id(module)]
        e = _Entry(module)
        self._pos[id(module)] = len(self.entries)
        self.entries.append(e)
        return self._pos[id(module)]

    def host_bytes(self) -> int:
        return sum(e.nbytes for e in self.entries)

    def _copy_stream(self):
        if self._stream is None:
            self._stream = torch.cuda.Stream(device=self.device)  # default priority
        return self._stream

    def _upload(self, e: _Entry) -> None:
        s = self._copy_stream()
        with torch.cuda.stream(s):
            d = torch.empty(e.host.numel(), dtype=torch.uint8, device=self.device)
            d.copy_(e.host, non_blocking=True)
            ev = torch.cuda.Event()
            ev.record(s)
        e.dev = (d, e._views(d), ev)
        self.stats["bytes"] += e.nbytes

    def _prefetch_after(self, i: int) -> None:
        n = len(self.entries)
        for k in range(1, min(self.depth, n - 1) + 1):
            e = self.entries[(i + k) % n]
            if e.dev is None and not e.installed:
                self._upload(e)
                self.stats["prefetched"] += 1

    def acquire(self, module: nn.Module) -> None:
        """Install ``module``'s device weights (copying them now unless a
        prefetch did) on the current stream of the device, then start the
        copies of the modules after it."""
        with self._lock:
            i = self._pos[id(module)]
            e = self.entries[i]
            if e.installed:
                return
            if e.dev is None:
                self._upload(e)
                self.stats["on_demand"] += 1
            d, views, ev = e.dev
            cur = torch.cuda.current_stream(self.device)
            cur.wait_event(ev)
            d.record_stream(cur)  # the views share d's memory
            e._install(views)
            e.installed = True
            self._prefetch_after(i)

    def release(self, module: nn.Module) -> None:
        """Put ``module``'s host weights back and let go of the device copy
        (the allocator reuses its memory once the kernels queued on the
        compute stream so far have run)."""
        with self._lock:
            e = self.entries[self._pos[id(module)]]
            if not e.installed:
                return
            for m, _, _, _ in e.qlinears:
                _clear_specific_dequant_cache(id(m.quantized_weights))
            e._install(e.host_views)
            e.dev = None
            e.installed = False

    def is_streamed(self, module: nn.Module) -> bool:
        return id(module) in self._pos


class QuantizedTensorOffloadHook(AlignDevicesHook):
    """accelerate hook that places a module's weights (QuantizedLinear
    weights included) on ``execution_device`` for its forward and, with
    ``offload=True``, takes them back afterwards (reference :48-177).  With
    ``streamer`` the weights come from the streamer's pinned host copies,
    prefetched on a side stream."""

    def __init__(self, *args, streamer: Optional[WeightStreamer] = None, **kwargs):
        super().__init__(*args, **kwargs)
        self.hooked_module_original_devices: Dict[int, torch.device] = {}
        self.streamer = streamer

    def __deepcopy__(self, memo=None):
        return self

    def init_hook(self, module):
        # accelerate's offload set-up would turn the module's own parameters
        # into meta tensors; here the streamer or module.to places them
        return module

    def _target(self, module) -> Optional[torch.device]:
        d = self.execution_device
        if isinstance(d, dict):
            d = d.get(module, d.get(None))
        return None if d is None else torch.device(d)

    def _move_to_device(self, obj: Any, device: torch.device):
        """Tensors, QuantizedTensors and modules (QuantizedLinear with its
        weight and bias) to ``device`` (reference :61-88)."""
        if obj is None:
            return None
        if isinstance(obj, QuantizedTensor):
            if obj.fp8_data.device != device:
                _clear_specific_dequant_cache(id(obj))
                return obj.to(device)
            return obj
        if _is_qlinear(obj):
            q = obj.quantized_weights
            if isinstance(q, QuantizedTensor) and q.fp8_data.device != device:
                _clear_specific_dequant_cache(id(q))
            return obj.to(device)
        if isinstance(obj, nn.Module):
            return obj.to(device)
        if isinstance(obj, torch.Tensor):
            return obj if obj.device == device else obj.to(device)
        return obj

    @staticmethod
    def _module_device(module) -> torch.device:
        for t in module.parameters():
            return t.device
        for t in module.buffers():
            return t.device
        for m in module.modules():
            if _is_qlinear(m) and hasattr(m.quantized_weights, "fp8_data"):
                return m.quantized_weights.fp8_data.device
        return torch.device("cpu")

    def pre_forward(self, module, *args, **kwargs):
        target = self._target(module)
        if target is None:
            return args, kwargs
        if target.type == "cuda" and target.index is None:
            target = torch.device("cuda", torch.cuda.current_device())
        if self.streamer is not None and self.streamer.is_streamed(module):
            self.streamer.acquire(module)
        else:
            key = id(module)
            if key not in self.hooked_module_original_devices:
                self.hooked_module_original_devices[key] = self._module_device(module)
            if self._module_device(module) != target:
                module.to(target)  # QuantizedLinear._apply moves its weight and bias too
        move = lambda t: self._move_to_device(t, target)  # noqa: E731
        return map_structure(move, args), map_structure(move, kwargs)

    def post_forward(self, module, output):
        if self.streamer is not None and self.streamer.is_streamed(module):
            if self.offload:
                self.streamer.release(module)
            return output
        if self.offload and id(module) in self.hooked_module_original_devices:
            home = self.hooked_module_original_devices[id(module)]
            if self._module_device(module) != home:
                module.to(home)
        for m in module.modules():
            if _is_qlinear(m) and isinstance(m.quantized_weights, QuantizedTensor):
                _clear_specific_dequant_cache(id(m.quantized_weights))
        return output
