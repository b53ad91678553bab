"""Device memory: the slab allocator and a small typed device-array handle.

``SlabAllocator`` follows the reference's contract (vte/bridge/memory.py:26-200):
one large ``hipMalloc`` carved into best-fit blocks, so every tensor has a
fixed address for graph capture, with overlap checking and free-block
merging.  Differences for MI355X: 256-byte alignment (a full HBM burst /
cache-line pair) instead of 64, and every block carries 256 bytes of
readable slack, because the LDS-staged GEMV and attention kernels read whole
aligned 16-byte chunks that may run up to 15 bytes past a tensor's end.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import IntEnum
from typing import Optional

import numpy as np

from .hip_runtime import HIPRuntime, HIPSafetyError, MemoryGuardianOOMError

ALIGN = 256
SLACK = 256


class MemoryRegion(IntEnum):
    WEIGHTS = 0
    KV_CACHE = 1
    ACTIVATIONS = 2
    SCRATCH = 3


@dataclass
class MemoryBlock:
    offset: int
    size: int
    tag: str
    region: MemoryRegion
    ptr: int
    is_free: bool = False


def _round_up(n: int, a: int) -> int:
    return (n + a - 1) // a * a


class SlabAllocator:
    """One hipMalloc slab, best-fit sub-allocation, fixed addresses."""

    def __init__(self, hip_runtime: HIPRuntime, total_vram_bytes: int, requested_pool_size: Optional[int] = None):
        self.hip = hip_runtime
        self.pool_size = _round_up(requested_pool_size or int(total_vram_bytes * 0.9), ALIGN)
        self.base_ptr: Optional[ctypes.c_void_p] = None
        self.blocks: list[MemoryBlock] = []

    def initialize(self) -> None:
        self.base_ptr = self.hip.safe_malloc(self.pool_size, "slab_pool")
        self.blocks = [MemoryBlock(0, self.pool_size, "free", MemoryRegion.SCRATCH, self.base_ptr.value, True)]

    def allocate(self, size: int, tag: str, region: MemoryRegion = MemoryRegion.SCRATCH) -> MemoryBlock:
        if self.base_ptr is None:
            raise HIPSafetyError("SlabAllocator not initialised")
        if size <= 0:
            raise HIPSafetyError(f"invalid slab allocation size {size} [{tag}]")
        need = _round_up(size + SLACK, ALIGN)
        best = None
        for i, b in enumerate(self.blocks):
            if b.is_free and b.size >= need and (best is None or b.size < self.blocks[best].size):
                best = i
        if best is None:
            raise MemoryGuardianOOMError(f"slab exhausted: {need} bytes for [{tag}] "
                                         f"(largest free {max((b.size for b in self.blocks if b.is_free), default=0)})")
        b = self.blocks[best]
        blk = MemoryBlock(b.offset, need, tag, region, self.base_ptr.value + b.offset, False)
        rest = b.size - need
        self.blocks[best] = blk
        if rest > 0:
            self.blocks.insert(best + 1, MemoryBlock(b.offset + need, rest, "free", MemoryRegion.SCRATCH,
                                                     self.base_ptr.value + b.offset + need, True))
        self._check_overlap(blk)
        return blk

    def _check_overlap(self, new_block: MemoryBlock) -> None:
        for b in self.blocks:
            if b is new_block or b.is_free:
                continue
            if b.offset < new_block.offset + new_block.size and new_block.offset < b.offset + b.size:
                raise HIPSafetyError(f"slab overlap between [{b.tag}] and [{new_block.tag}]")

    def free(self, block: MemoryBlock) -> None:
        for b in self.blocks:
            if b.offset == block.offset and not b.is_free:
                b.is_free = True
                b.tag = "free"
                self._merge_adjacent_free_blocks()
                return
        raise HIPSafetyError(f"free of unknown slab block [{block.tag}]")

    def _merge_adjacent_free_blocks(self) -> None:
        merged: list[MemoryBlock] = []
        for b in self.blocks:
            if merged and merged[-1].is_free and b.is_free:
                merged[-1].size += b.size
            else:
                merged.append(b)
        self.blocks = merged

    def validate_pointer(self, ptr: int, size: int) -> bool:
        for b in self.blocks:
            if not b.is_free and b.ptr <= ptr and ptr + size <= b.ptr + b.size:
                return True
        return False

    def get_stats(self) -> dict:
        used = sum(b.size for b in self.blocks if not b.is_free)
        return {"pool_size": self.pool_size, "used": used, "free": self.pool_size - used,
                "blocks": sum(1 for b in self.blocks if not b.is_free)}

    def cleanup(self) -> None:
        if self.base_ptr is not None:
            self.hip.safe_free(self.base_ptr, "slab_pool")
            self.base_ptr = None
            self.blocks = []


class DeviceArray:
    """A typed view of device memory (own hipMalloc or a slab block)."""

    def __init__(self, hip: HIPRuntime, shape, dtype, tag: str = "array", slab: Optional[SlabAllocator] = None,
                 region: MemoryRegion = MemoryRegion.SCRATCH):
        self.hip = hip
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.tag = tag
        self._slab = slab
        if slab is not None:
            self._block = slab.allocate(max(self.nbytes, 1), tag, region)
            self.ptr = self._block.ptr
            self._own = None
        else:
            self._own = hip.safe_malloc(_round_up(max(self.nbytes, 1) + SLACK, ALIGN), tag)
            self.ptr = self._own.value
            self._block = None

    @classmethod
    def from_numpy(cls, hip: HIPRuntime, arr: np.ndarray, tag: str = "array", slab=None,
                   region: MemoryRegion = MemoryRegion.SCRATCH) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        d = cls(hip, arr.shape, arr.dtype, tag, slab, region)
        d.upload(arr)
        return d

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        if arr.nbytes != self.nbytes:
            raise HIPSafetyError(f"upload size {arr.nbytes} != {self.nbytes} [{self.tag}]")
        if self.nbytes:
            self._copy_h2d(arr)

    def _copy_h2d(self, arr: np.ndarray) -> None:
        if self._slab is None:
            self.hip.safe_memcpy_host_to_device(ctypes.c_void_p(self.ptr), arr, self.tag)
        else:
            self.hip.safe_memcpy_host_to_device(ctypes.c_void_p(self.ptr), arr, self.tag)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if self.nbytes:
            self.hip.safe_memcpy_device_to_host(out, ctypes.c_void_p(self.ptr), "output:" + self.tag)
        return out

    def zero(self) -> None:
        if self.nbytes:
            self.hip.safe_memset(ctypes.c_void_p(self.ptr), self.nbytes, self.tag)

    def free(self) -> None:
        if self._own is not None:
            self.hip.safe_free(self._own, self.tag)
            self._own = None
        elif self._block is not None:
            self._slab.free(self._block)
            self._block = None
