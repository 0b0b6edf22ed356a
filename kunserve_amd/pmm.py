"""Parameter memory remap: KV pools that dropped weight layers extend in place.

The balloon path of the reference drops the weights of the layers a worker
stops executing and turns their device memory into extra KV blocks
(LlamaOp.pmm_drop, kunserve/worker.py:454-482), numbered after the base
blocks (kunserve/block_manager.py:262-269); pmm_restore maps that memory
back to the weights (kunserve/worker.py:484-501, described at
kunserve/llm_engine.py:553-558).

PmmPool owns the K and V pools and the weight segments through the
kunserve_pmm_* C functions. Its `pool` is a KVPool over the pages mapped
now; drop() and restore() change the page count and replace `pool`, and a
KVPool taken before either call refuses further use. Tensors returned by
segment() view the segment's memory only while it is not dropped.
"""
from __future__ import annotations

import atexit
import ctypes
import weakref
from typing import Dict, List, Optional

import torch

from . import _lib
from .paged_kv import FP16, KVPool, _DTYPES

_live: "weakref.WeakSet[PmmPool]" = weakref.WeakSet()


class _DeviceBytes:
    """A device byte range in the form torch.as_tensor accepts; keeps the
    owning PmmPool alive for as long as a tensor views the range."""

    def __init__(self, ptr: int, nbytes: int, owner: "PmmPool"):
        self._owner = owner
        self.__cuda_array_interface__ = {
            "shape": (nbytes,), "typestr": "|u1", "data": (ptr, False), "version": 2,
            "strides": None,
        }


def _device_view(ptr: int, nbytes: int, device: torch.device, owner: "PmmPool") -> torch.Tensor:
    t = torch.as_tensor(_DeviceBytes(ptr, nbytes, owner), device=device)
    if t.data_ptr() != ptr or t.numel() != nbytes:
        raise RuntimeError("device view does not cover the requested range")
    return t


class PmmPool:
    """K and V pools of base_pages pages, extendable by up to
    max_extend_pages pages taken from dropped weight segments.

    A page holds all layers of page_size tokens, as in KVPool:
    [num_layers, num_kv_heads, page_size, head_dim] elements of K (and the
    same of V), so a segment of 2 * n * page_bytes bytes adds n pages.
    """

    def __init__(self, base_pages: int, num_layers: int, num_kv_heads: int, page_size: int,
                 head_dim: int, max_extend_pages: int, device=None, dtype: torch.dtype = FP16):
        if dtype not in _DTYPES:
            raise ValueError("KV pools must be float16 or bfloat16")
        dev = torch.device(device) if device is not None else torch.device(
            "cuda", torch.cuda.current_device())
        if dev.type != "cuda":
            raise ValueError(f"PmmPool needs a GPU device, got {dev}")
        self.device = torch.device("cuda", dev.index if dev.index is not None
                                   else torch.cuda.current_device())
        self.dtype = dtype
        self.shape_tail = (num_layers, num_kv_heads, page_size, head_dim)
        self.page_elems = num_layers * num_kv_heads * page_size * head_dim
        self.page_bytes = self.page_elems * torch.tensor([], dtype=dtype).element_size()
        self.base_pages = base_pages
        self.max_pages = base_pages + max_extend_pages
        self.generation = 0
        self._segments: Dict[int, int] = {}    # id -> bytes
        self._addr: Dict[int, int] = {}        # id -> device address while not dropped
        self._dropped: List[int] = []
        handle = ctypes.c_void_p()
        _lib.call("kunserve_pmm_create", self.device.index, self.page_bytes, base_pages,
                  max_extend_pages, ctypes.byref(handle))
        self._handle: Optional[ctypes.c_void_p] = handle
        k, v, n = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64()
        _lib.call("kunserve_pmm_pools", handle, ctypes.byref(k), ctypes.byref(v), ctypes.byref(n))
        self._k_base, self._v_base = int(k.value), int(v.value)
        self.num_pages = int(n.value)
        self.pool = self._make_pool()
        _live.add(self)

    # ----------------------------------------------------------- views

    def _make_pool(self) -> KVPool:
        nbytes = self.num_pages * self.page_bytes
        shape = (self.num_pages,) + self.shape_tail
        k = _device_view(self._k_base, nbytes, self.device, self).view(self.dtype).view(shape)
        v = _device_view(self._v_base, nbytes, self.device, self).view(self.dtype).view(shape)
        return KVPool(k, v, owner=self)

    def _check_open(self) -> ctypes.c_void_p:
        if self._handle is None:
            raise RuntimeError("PmmPool is closed")
        return self._handle

    def add_segment(self, nbytes: int) -> int:
        """Allocates a weight segment of at least nbytes, rounded up to whole
        page pairs (2 * page_bytes); returns its id."""
        h = self._check_open()
        unit = 2 * self.page_bytes
        size = max(1, -(-int(nbytes) // unit)) * unit
        sid, addr = ctypes.c_int32(), ctypes.c_void_p()
        _lib.call("kunserve_pmm_add_segment", h, size, ctypes.byref(sid), ctypes.byref(addr))
        self._segments[int(sid.value)] = size
        self._addr[int(sid.value)] = int(addr.value)
        return int(sid.value)

    def segment(self, segment_id: int) -> torch.Tensor:
        """uint8 view of a segment's memory; valid until the segment is dropped."""
        self._check_open()
        if segment_id not in self._segments:
            raise KeyError(f"no segment {segment_id}")
        if segment_id in self._dropped:
            raise RuntimeError(f"segment {segment_id} is dropped")
        return _device_view(self._addr[segment_id], self._segments[segment_id], self.device, self)

    def segment_pages(self, segment_id: int) -> int:
        return self._segments[segment_id] // (2 * self.page_bytes)

    # ------------------------------------------------------- drop/restore

    def drop(self, segment_id: int) -> range:
        """Turns a segment into K and V pages; returns their ids. Waits for
        the device; views of the segment must not be used afterwards."""
        h = self._check_open()
        n = ctypes.c_int64()
        _lib.call("kunserve_pmm_drop", h, int(segment_id), ctypes.byref(n))
        old = self.num_pages
        self._dropped.append(int(segment_id))
        self._remapped(int(n.value))
        return range(old, self.num_pages)

    def restore(self) -> int:
        """Gives the most recently dropped segment its memory back (holding
        what its pages held); returns its id. Waits for the device; pages
        past the new count must no longer be referenced."""
        h = self._check_open()
        sid, n = ctypes.c_int32(), ctypes.c_int64()
        _lib.call("kunserve_pmm_restore", h, ctypes.byref(sid), ctypes.byref(n))
        self._dropped.pop()
        self._remapped(int(n.value))
        return int(sid.value)

    @property
    def dropped(self) -> List[int]:
        return list(self._dropped)

    def _remapped(self, num_pages: int) -> None:
        self.generation += 1
        self.num_pages = num_pages
        self.pool = self._make_pool()

    # ------------------------------------------------------------ lifetime

    def close(self) -> None:
        """Frees every page and segment. Views taken from this pool must not
        be used afterwards."""
        if self._handle is not None:
            h, self._handle = self._handle, None
            self.generation += 1
            _lib.lib().kunserve_pmm_destroy(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@atexit.register
def _close_all() -> None:
    # Before the HIP runtime's own teardown.
    for p in list(_live):
        p.close()
