"""Tiered key/value cache: HBM, page-locked host memory, disk.

Same names and public interface as the reference module
/root/reference/atlasinfer_core/memory/unified_memory_manager.py (also
importable as ``atlasinfer_core.memory.unified_memory_manager``):
``UnifiedMemoryManager(vram_limit_gb, ram_limit_gb, disk_path,
disk_limit_gb=50, gpu_device, cpu_device, vram_only_kv_cache=False)`` with
``put_kv`` / ``get_kv`` / ``get_stats`` / ``close`` (reference :111-523) and
the same statistics keys.  Entries move down the tiers in least-recently-used
order when a tier is over its limit and come back to the GPU when read.

Designed for the GPU rather than restated:

* One entry per layer holds its keys and values ([batch, heads, seq, dim]).
  In HBM an entry is a pair of buffers with room to grow along the sequence
  (capacity doubled when full): ``append_kv`` writes a step's new keys and
  values in place and returns views of the whole history, so a decode step
  costs the new tokens' bytes, not a copy of the history (the reference
  stores each step's concatenation of the history with the new tokens,
  which copies the history every step).  ``put_kv`` / ``get_kv`` keep the
  reference's store-the-whole-history semantics on the same entries.
* The host tier is page-locked memory, so moves between HBM and host are
  asynchronous copies on the current stream.
* The disk tier (the reference's LMDB store, whose ``lmdb`` package is not
  part of this build) is a directory of raw tensor files with a small
  header (dtype, shape): nothing is unpickled when an entry comes back.
* ``KVCacheLayer`` lets an HF ``Cache`` keep a layer's keys and values here
  (AtlasAttentionWrapper installs it), so the model's own attention code
  and masks run unchanged on top of the tiers.
"""
from __future__ import annotations

import json
import os
import threading
from collections import OrderedDict
from typing import Any, Dict, Optional, Tuple

import numpy as np
import torch

_GiB = 1024 ** 3
_MIN_CAP = 256  # smallest sequence capacity of an HBM buffer


def _nbytes(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.numel() * t.element_size()


class DiskKVStore:
    """Entries as raw files under ``path``: ``<key>.bin`` holds the tensor's
    bytes, ``<key>.json`` its dtype and shape.  Writing past ``limit_bytes``
    fails (returns False), as the reference's LMDB map does when full."""

    def __init__(self, path: str, limit_bytes: int):
        self.path = path
        self.limit = int(limit_bytes)
        self.used = 0
        self.sizes: Dict[str, int] = {}
        os.makedirs(path, exist_ok=True)

    def _files(self, key: str):
        return os.path.join(self.path, key + ".bin"), os.path.join(self.path, key + ".json")

    def put(self, key: str, t: torch.Tensor) -> bool:
        size = _nbytes(t)
        old = self.sizes.get(key, 0)
        if self.used - old + size > self.limit:
            return False
        a = t.detach().to("cpu").contiguous()
        raw = a.view(torch.uint8) if a.numel() else a.reshape(0).view(torch.uint8)
        binf, meta = self._files(key)
        raw.numpy().tofile(binf)
        with open(meta, "w") as f:
            json.dump({"dtype": str(a.dtype).replace("torch.", ""), "shape": list(a.shape)}, f)
        self.used += size - old
        self.sizes[key] = size
        return True

    def get(self, key: str) -> Optional[torch.Tensor]:
        binf, meta = self._files(key)
        if key not in self.sizes or not os.path.exists(meta):
            return None
        with open(meta) as f:
            m = json.load(f)
        raw = torch.from_numpy(np.fromfile(binf, dtype=np.uint8))
        return raw.view(getattr(torch, m["dtype"])).reshape(m["shape"])

    def delete(self, key: str) -> bool:
        if key not in self.sizes:
            return False
        for f in self._files(key):
            if os.path.exists(f):
                os.remove(f)
        self.used -= self.sizes.pop(key)
        return True

    def close(self):
        for key in list(self.sizes):
            self.delete(key)


class _Entry:
    """A layer's keys and values: in HBM (buffers with spare sequence
    capacity and the valid length), in host memory or on disk."""

    __slots__ = ("k", "v", "length", "tier")

    def __init__(self):
        self.k = self.v = None
        self.length = 0
        self.tier = None  # "vram", "ram" or "disk"

    def bytes_held(self) -> int:
        return _nbytes(self.k) + _nbytes(self.v)

    def views(self):
        return self.k[:, :, :self.length], self.v[:, :, :self.length]


class UnifiedMemoryManager:
    """Key/value cache over HBM, page-locked host memory and disk with
    least-recently-used demotion (reference :111-523)."""

    def __init__(self, vram_limit_gb: float, ram_limit_gb: float, disk_path: Optional[str],
                 disk_limit_gb: int = 50, gpu_device: torch.device = torch.device("cuda:0"),
                 cpu_device: torch.device = torch.device("cpu"), vram_only_kv_cache: bool = False):
        gpu_device = torch.device(gpu_device)
        self.gpu_device = gpu_device if (gpu_device.type == "cuda" and torch.cuda.is_available()) else \
            torch.device(cpu_device)
        self.cpu_device = torch.device(cpu_device)
        self.can_use_gpu = self.gpu_device != self.cpu_device
        self.vram_capacity = int(vram_limit_gb * _GiB) if self.can_use_gpu else 0
        self.ram_capacity = int(ram_limit_gb * _GiB)
        self.vram_only_mode = vram_only_kv_cache if self.can_use_gpu else False
        # without a GPU the host tier is the top one (the reference then forces
        # a VRAM-only mode in which nothing can be stored)
        self.vram_cache: "OrderedDict[int, _Entry]" = OrderedDict()  # LRU order, oldest first
        self.ram_cache: "OrderedDict[int, _Entry]" = OrderedDict()
        self.disk_interface = None
        self.use_disk = False
        if disk_path and str(disk_path).lower() != "none" and not self.vram_only_mode:
            self.disk_interface = DiskKVStore(str(disk_path), int(disk_limit_gb * _GiB))
            self.use_disk = True
        self.disk_entries: Dict[int, _Entry] = {}
        self.vram_used = 0
        self.ram_used = 0
        self.stats = {"vram_hits": 0, "ram_hits": 0, "disk_hits": 0, "misses": 0, "evict_vram": 0,
                      "evict_ram": 0, "load_ram": 0, "load_disk": 0, "put_vram": 0, "put_ram": 0, "put_disk": 0}
        self._lock = threading.RLock()

    # ------------------------------------------------------------ tiers

    def _bump(self, key: str, n: int = 1):
        self.stats[key] += n

    def _detach(self, layer: int) -> Optional[_Entry]:
        """Remove a layer's entry from whichever tier holds it."""
        e = self.vram_cache.pop(layer, None)
        if e is not None:
            self.vram_used -= e.bytes_held()
            return e
        e = self.ram_cache.pop(layer, None)
        if e is not None:
            self.ram_used -= e.bytes_held()
            return e
        e = self.disk_entries.pop(layer, None)
        if e is not None:
            for kv in ("K", "V"):
                self.disk_interface.delete(self._get_kv_key(layer, kv))
        return e

    def _make_room_vram(self, size: int, keep: int) -> bool:
        if size > self.vram_capacity:
            return False  # would not fit in an empty tier: evict nothing
        while self.vram_used + size > self.vram_capacity:
            victim = next((k for k in self.vram_cache if k != keep), None)
            if victim is None:
                return False
            self._demote_vram(victim)
        return True

    def _make_room_ram(self, size: int, keep: int) -> bool:
        if size > self.ram_capacity:
            return False
        while self.ram_used + size > self.ram_capacity:
            victim = next((k for k in self.ram_cache if k != keep), None)
            if victim is None or not self._demote_ram(victim):
                return False
        return True

    def _demote_vram(self, layer: int) -> None:
        e = self.vram_cache.pop(layer)
        self.vram_used -= e.bytes_held()
        self._bump("evict_vram")
        if self.vram_only_mode:
            return  # dropped, as the reference's VRAM-only mode does
        k, v = e.views()
        hk = torch.empty(k.shape, dtype=k.dtype, pin_memory=True)
        hv = torch.empty(v.shape, dtype=v.dtype, pin_memory=True)
        hk.copy_(k, non_blocking=True)
        hv.copy_(v, non_blocking=True)
        e.k, e.v, e.tier = hk, hv, "ram"
        torch.cuda.current_stream(self.gpu_device).synchronize()  # host copies complete before any use
        self._place_ram(layer, e)

    def _place_ram(self, layer: int, e: _Entry) -> bool:
        size = e.bytes_held()
        if not self._make_room_ram(size, keep=layer):
            if self.use_disk and self._to_disk(layer, e):
                return True
            return False  # lost, as in the reference when no tier takes it
        e.tier = "ram"
        self.ram_cache[layer] = e
        self.ram_cache.move_to_end(layer)
        self.ram_used += size
        return True

    def _demote_ram(self, layer: int) -> bool:
        if not self.use_disk:
            return False
        e = self.ram_cache.pop(layer)
        self.ram_used -= e.bytes_held()
        self._bump("evict_ram")
        return self._to_disk(layer, e)

    def _to_disk(self, layer: int, e: _Entry) -> bool:
        k, v = e.views()
        kkey = self._get_kv_key(layer, "K")
        if not self.disk_interface.put(kkey, k):
            return False
        if not self.disk_interface.put(self._get_kv_key(layer, "V"), v):
            # no entry will own the keys' file: take it back out with its bytes
            self.disk_interface.delete(kkey)
            return False
        e.length = int(k.shape[2])
        e.k = e.v = None
        e.tier = "disk"
        self.disk_entries[layer] = e
        self._bump("put_disk")
        return True

    def _promote(self, layer: int, e: _Entry, extra: int = 0) -> Optional[_Entry]:
        """Bring an entry held in host memory or on disk to the top tier
        (HBM, with room for ``extra`` more positions), or keep it in host
        memory when there is no GPU."""
        if e.tier == "disk":
            k = self.disk_interface.get(self._get_kv_key(layer, "K"))
            v = self.disk_interface.get(self._get_kv_key(layer, "V"))
            self.disk_entries.pop(layer, None)
            for kv in ("K", "V"):
                self.disk_interface.delete(self._get_kv_key(layer, kv))
            self._bump("load_disk")
            e.k, e.v, e.tier = k, v, "ram_staged"
        elif e.tier == "ram":
            self.ram_cache.pop(layer)
            self.ram_used -= e.bytes_held()
            self._bump("load_ram")
        if not self.can_use_gpu:
            self._place_ram(layer, e)
            return e
        k, v = e.views()
        B, H, S, D = k.shape
        # a read takes exactly the history's room; an append some to grow into
        cap = S if extra == 0 else max(_MIN_CAP, S + extra)
        size = 2 * B * H * cap * D * k.element_size()
        if not self._make_room_vram(size, keep=layer):
            self._place_ram(layer, e)
            return None
        dk = torch.empty((B, H, cap, D), dtype=k.dtype, device=self.gpu_device)
        dv = torch.empty((B, H, cap, D), dtype=v.dtype, device=self.gpu_device)
        dk[:, :, :S].copy_(k, non_blocking=True)
        dv[:, :, :S].copy_(v, non_blocking=True)
        e.k, e.v, e.length, e.tier = dk, dv, S, "vram"
        self.vram_cache[layer] = e
        self.vram_used += size
        return e

    def _find(self, layer: int) -> Tuple[Optional[_Entry], Optional[str]]:
        if layer in self.vram_cache:
            return self.vram_cache[layer], "vram"
        if layer in self.ram_cache:
            return self.ram_cache[layer], "ram"
        if layer in self.disk_entries:
            return self.disk_entries[layer], "disk"
        return None, None

    # ------------------------------------------------------------ reference API

    def _get_kv_key(self, layer_idx: int, type: str) -> str:
        """Key of a layer's K or V in the disk tier (reference :350-352)."""
        return f"kv_{layer_idx}_{type.upper()}"

    def put_kv(self, layer_idx: int, k_tensor: torch.Tensor, v_tensor: torch.Tensor):
        """Store a layer's whole key/value history, replacing what it had
        (reference :354-438).  The tensors are kept as they are (no copy)
        in the top tier when they fit."""
        with self._lock:
            self._detach(layer_idx)
            e = _Entry()
            dev = self.gpu_device if self.can_use_gpu else self.cpu_device
            e.k, e.v = k_tensor.to(dev), v_tensor.to(dev)
            e.length = int(k_tensor.shape[2])
            size = e.bytes_held()
            if self.can_use_gpu and self._make_room_vram(size, keep=layer_idx):
                e.tier = "vram"
                self.vram_cache[layer_idx] = e
                self.vram_used += size
                self._bump("put_vram")
                return
            if self.vram_only_mode:
                return
            e.k, e.v = e.k.to(self.cpu_device), e.v.to(self.cpu_device)
            e.tier = "ram"
            if self._make_room_ram(size, keep=layer_idx):
                self.ram_cache[layer_idx] = e
                self.ram_used += size
                self._bump("put_ram")
            elif self.use_disk:
                self._to_disk(layer_idx, e)

    def get_kv(self, layer_idx: int) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """A layer's key/value history, brought to the GPU when there is one
        (reference :441-525); (None, None) when the layer holds nothing."""
        with self._lock:
            e, tier = self._find(layer_idx)
            if e is None:
                self._bump("misses")
                return None, None
            self._bump({"vram": "vram_hits", "ram": "ram_hits", "disk": "disk_hits"}[tier])
            if tier == "vram":
                self.vram_cache.move_to_end(layer_idx)
                return e.views()
            if tier == "ram" and not self.can_use_gpu:
                self.ram_cache.move_to_end(layer_idx)
                return e.views()
            p = self._promote(layer_idx, e)
            if p is None:  # no room in HBM: served from host memory
                k, v = e.k, e.v
                return k.to(self.gpu_device), v.to(self.gpu_device)
            return p.views() if p.tier == "vram" else (p.k, p.v)

    def _top_tier(self):
        """(name, LRU dict, room-making function, usage attribute) of the
        tier new entries go to: HBM, or host memory without a GPU."""
        if self.can_use_gpu:
            return "vram", self.vram_cache, self._make_room_vram, "vram_used"
        return "ram", self.ram_cache, self._make_room_ram, "ram_used"

    def append_kv(self, layer_idx: int, k_new: torch.Tensor, v_new: torch.Tensor
                  ) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append a step's keys and values ([batch, heads, new, dim]) to the
        layer's history in place and return the whole history (views of the
        top tier's buffers: HBM, or host memory without a GPU).  Not in the
        reference, whose attention stored the concatenated history each
        step."""
        with self._lock:
            q = int(k_new.shape[2])
            top, lru, make_room, used = self._top_tier()
            e, tier = self._find(layer_idx)
            if e is None:
                e = _Entry()
                B, H, _, D = k_new.shape
                cap = max(_MIN_CAP, q)
                size = 2 * B * H * cap * D * k_new.element_size()
                if not make_room(size, keep=layer_idx):
                    raise RuntimeError(f"KV cache: no room in the {top} tier for layer {layer_idx}")
                dev = self.gpu_device if top == "vram" else self.cpu_device
                e.k = k_new.new_empty((B, H, cap, D), device=dev)
                e.v = v_new.new_empty((B, H, cap, D), device=dev)
                e.tier = top
                lru[layer_idx] = e
                setattr(self, used, getattr(self, used) + size)
            elif tier == top:
                lru.move_to_end(layer_idx)
            else:
                e = self._promote(layer_idx, e, extra=q)
                if e is None or e.tier != top:
                    raise RuntimeError(f"KV cache: no room in the {top} tier for layer {layer_idx}")
            if e.k.shape[0] != k_new.shape[0] or e.k.shape[1] != k_new.shape[1] or e.k.shape[3] != k_new.shape[3]:
                raise ValueError(f"KV cache layer {layer_idx}: new states {tuple(k_new.shape)} do not extend "
                                 f"{tuple(e.k.shape)}")
            if e.length + q > e.k.shape[2]:
                self._grow(layer_idx, e, e.length + q)
            e.k[:, :, e.length:e.length + q].copy_(k_new)
            e.v[:, :, e.length:e.length + q].copy_(v_new)
            e.length += q
            self._bump("put_vram" if top == "vram" else "put_ram")
            return e.views()

    def _grow(self, layer: int, e: _Entry, need: int) -> None:
        """Give an entry of the top tier room for ``need`` positions
        (capacity at least doubled), keeping its history."""
        top, _, make_room, used = self._top_tier()
        B, H, cap, D = e.k.shape
        new_cap = max(2 * cap, need, _MIN_CAP)
        old = e.bytes_held()
        size = 2 * B * H * new_cap * D * e.k.element_size()
        setattr(self, used, getattr(self, used) - old)
        if not make_room(size, keep=layer):
            setattr(self, used, getattr(self, used) + old)
            raise RuntimeError(f"KV cache: no room in the {top} tier to grow layer {layer} to {new_cap} positions")
        nk = e.k.new_empty((B, H, new_cap, D))
        nv = e.v.new_empty((B, H, new_cap, D))
        nk[:, :, :e.length].copy_(e.k[:, :, :e.length])
        nv[:, :, :e.length].copy_(e.v[:, :, :e.length])
        e.k, e.v = nk, nv
        setattr(self, used, getattr(self, used) + size)

    def seq_length(self, layer_idx: int) -> int:
        """Positions held for a layer (0 when it holds nothing)."""
        e, _ = self._find(layer_idx)
        return 0 if e is None else e.length

    def reset_layer(self, layer_idx: int) -> None:
        with self._lock:
            self._detach(layer_idx)

    def truncate(self, layer_idx: int, length: int) -> None:
        """Keep the first ``length`` positions of a layer's history."""
        with self._lock:
            e, tier = self._find(layer_idx)
            if e is None:
                return
            if tier != "vram":
                e = self._promote(layer_idx, e) or e
            if e.tier != "vram":
                e.k, e.v = e.k[:, :, :length], e.v[:, :, :length]
            e.length = min(e.length, length)

    def clear(self) -> None:
        """Drop every entry (a new set of sequences)."""
        with self._lock:
            for layer in list(self.vram_cache) + list(self.ram_cache) + list(self.disk_entries):
                self._detach(layer)

    def get_stats(self) -> Dict[str, Any]:
        """Counters and tier usage (reference :528-553)."""
        s = dict(self.stats)
        s["vram_used_gb"] = self.vram_used / _GiB
        s["ram_used_gb"] = self.ram_used / _GiB
        s["vram_cache_items"] = len(self.vram_cache)
        s["ram_cache_items"] = len(self.ram_cache)
        s["total_hits"] = s["vram_hits"] + s["ram_hits"] + s["disk_hits"]
        s["disk_used_gb_est"] = (f"{self.disk_interface.used / _GiB:.3f}" if self.use_disk
                                 else "N/A (Disk Disabled)")
        return s

    def close(self):
        """Drop the entries and the disk tier's files (reference :555-560)."""
        self.clear()
        if self.disk_interface is not None:
            self.disk_interface.close()


def _cache_layer_base():
    from transformers.cache_utils import CacheLayerMixin
    return CacheLayerMixin


class KVCacheLayer(_cache_layer_base()):
    """One layer of an HF ``Cache`` whose keys and values live in a
    UnifiedMemoryManager: ``update`` appends in place there and returns the
    whole history, lengths and mask sizes come from the manager."""

    is_sliding = False

    def __init__(self, manager: UnifiedMemoryManager, layer_idx: int):
        super().__init__()
        self.manager = manager
        self.layer_idx = layer_idx

    def lazy_initialization(self, key_states, value_states):
        self.dtype, self.device = key_states.dtype, key_states.device
        self.is_initialized = True

    def update(self, key_states, value_states, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        return self.manager.append_kv(self.layer_idx, key_states, value_states)

    def get_mask_sizes(self, query_length: int):
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self) -> int:
        return self.manager.seq_length(self.layer_idx)

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        self.manager.reset_layer(self.layer_idx)

    def crop(self, max_length: int) -> None:
        """Keep the first ``max_length`` positions (a negative value: drop
        that many from the end), as HF's DynamicLayer.crop does; crop(0)
        empties the layer."""
        n = self.get_seq_length()
        keep = max_length if max_length >= 0 else n + max_length
        if keep < n:
            self.manager.truncate(self.layer_idx, max(keep, 0))

    def offload(self):
        pass  # the manager decides where the layer lives

    def prefetch(self):
        pass

    def batch_repeat_interleave(self, repeats: int) -> None:
        raise NotImplementedError("the tiered KV cache holds one set of sequences (no beam expansion)")

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        raise NotImplementedError("the tiered KV cache holds one set of sequences (no beam selection)")

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        raise NotImplementedError("the tiered KV cache holds one set of sequences (no beam reordering)")
