"""Page allocator (python/aios/scheduler/cache.py:9-51).

A device int32 free list: ``allocate(n)`` hands out the first n free pages,
``_free`` appends released pages at the end, so the page order is a
deterministic function of the allocate/free history, as in the reference.
"""
from __future__ import annotations

import torch


class CacheManager:
    def __init__(self, device: torch.device, num_pages: int):
        self._free_slots = torch.arange(num_pages, dtype=torch.int32, device=device)
        self.device = device
        self.num_pages = num_pages

    def _free(self, indices: torch.Tensor) -> None:
        if len(indices) > 0:
            self._free_slots = torch.cat([self._free_slots, indices.to(torch.int32)])

    @property
    def available_size(self) -> int:
        return len(self._free_slots)

    def allocate_paged(self, reqs, page_table: torch.Tensor) -> None:
        for req in reqs:
            assert req.table_idx is not None
            extend_len = req.extend_len
            if extend_len == 0:
                continue
            indices = self.allocate(extend_len)
            page_table[req.table_idx, req.cached_len : req.device_len] = indices

    def allocate(self, needed_len: int) -> torch.Tensor:
        if needed_len <= len(self._free_slots):
            allocated = self._free_slots[:needed_len]
            self._free_slots = self._free_slots[needed_len:]
            return allocated
        raise NotImplementedError("CacheManager eviction is not implemented.")
