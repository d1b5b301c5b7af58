"""Free-list arena planner (counterpart of c34/memory_pool.py).

Slots are byte ranges of one arena: alloc() reuses the best-fitting free block
(splitting the remainder), free() returns a block and coalesces neighbours,
and the high-water mark becomes the slab size (c34/memory_pool.py:47-254).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Tuple

from .execution_plan import PoolStats


@dataclass
class _MemoryBlock:
    slot_id: int
    offset: int = 0
    size_bytes: int = 0
    is_free: bool = True

    @property
    def end(self) -> int:
        return self.offset + self.size_bytes


class FitPolicy:
    BEST_FIT = "best_fit"
    FIRST_FIT = "first_fit"
    SIZE_CLASS = "size_class"


class DeviceMemoryPool:
    def __init__(self, policy: str = FitPolicy.BEST_FIT, alignment: int = 64,
                 total_device_bytes: int = 288 * 1024 ** 3) -> None:
        self._policy = policy
        self._alignment = alignment
        self._total_bytes = total_device_bytes
        self._next_slot_id = 0
        self._free_list: List[_MemoryBlock] = []
        self._active: Dict[int, _MemoryBlock] = {}
        self._coalesce_counter = 0
        self._reuse_hits = 0
        self._total_allocs = 0
        self._total_frees = 0
        self._peak_reserved_bytes = 0
        self._requested_bytes = 0
        self._reserved_bytes = 0

    def alloc(self, size_bytes: int, alignment: int = 64) -> int:
        if size_bytes <= 0:
            raise ValueError(f"Invalid allocation size: {size_bytes}")
        size_bytes = self._align_up(size_bytes, max(alignment, self._alignment))
        self._requested_bytes += size_bytes
        self._total_allocs += 1
        slot = self._try_reuse(size_bytes)
        if slot >= 0:
            self._reuse_hits += 1
            return slot
        slot = self._next_slot_id
        self._next_slot_id += 1
        self._active[slot] = _MemoryBlock(slot, self._reserved_bytes, size_bytes, False)
        self._reserved_bytes += size_bytes
        self._peak_reserved_bytes = max(self._peak_reserved_bytes, self._reserved_bytes)
        return slot

    def free(self, slot_id: int) -> None:
        block = self._active.pop(slot_id, None)
        if block is None:
            raise ValueError(f"Slot {slot_id} is not allocated")
        block.is_free = True
        self._free_list.append(block)
        self._total_frees += 1
        self._coalesce()

    def stats(self) -> PoolStats:
        free_bytes = sum(b.size_bytes for b in self._free_list)
        return PoolStats(requested_bytes=self._requested_bytes, reserved_bytes=self._reserved_bytes,
                         active_bytes=sum(b.size_bytes for b in self._active.values()),
                         peak_reserved_bytes=self._peak_reserved_bytes, internal_fragmentation=free_bytes,
                         reuse_hits=self._reuse_hits, total_allocs=self._total_allocs,
                         total_frees=self._total_frees, free_list_blocks=len(self._free_list))

    def describe(self, slot_id: int) -> Tuple[int, int]:
        block = self._active.get(slot_id)
        if block is None:
            raise ValueError(f"Slot {slot_id} is not allocated")
        return block.offset, block.size_bytes

    def _try_reuse(self, size_bytes: int) -> int:
        fits = [b for b in self._free_list if b.size_bytes >= size_bytes]
        if not fits:
            return -1
        if self._policy == FitPolicy.BEST_FIT:
            chosen = min(fits, key=lambda b: b.size_bytes)
        elif self._policy == FitPolicy.SIZE_CLASS:
            want = self._size_class(size_bytes)
            exact = [b for b in fits if self._size_class(b.size_bytes) == want]
            chosen = exact[0] if exact else min(fits, key=lambda b: self._size_class(b.size_bytes))
        else:
            chosen = fits[0]
        self._free_list.remove(chosen)
        if chosen.size_bytes > size_bytes:
            self._free_list.append(_MemoryBlock(self._next_slot_id, chosen.offset + size_bytes,
                                                chosen.size_bytes - size_bytes, True))
            self._next_slot_id += 1
            chosen.size_bytes = size_bytes
        chosen.is_free = False
        self._active[chosen.slot_id] = chosen
        return chosen.slot_id

    def _coalesce(self) -> None:
        if len(self._free_list) < 2:
            return
        self._free_list.sort(key=lambda b: b.offset)
        merged = [self._free_list[0]]
        for b in self._free_list[1:]:
            if merged[-1].end == b.offset:
                merged[-1].size_bytes += b.size_bytes
                self._coalesce_counter += 1
            else:
                merged.append(b)
        self._free_list = merged

    @staticmethod
    def _align_up(size: int, alignment: int) -> int:
        return (size + alignment - 1) // alignment * alignment

    @staticmethod
    def _size_class(size: int) -> int:
        return 1 << max(0, (size - 1).bit_length()) if size > 0 else 0
