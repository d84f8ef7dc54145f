"""Token-granular paged KV pool.

Layout and API of python/aios/kvcache/mha_pool.py:8-68: one buffer
``[2, num_layers, num_pages, page_size=1, num_kv_heads, head_dim]`` (K = [0],
V = [1]); layer ``i`` of K is the contiguous slice ``[num_pages, 1, Hkv, D]``.
At 288 GB of HBM per MI355X the pool is sized by the caller (the
long-context workload, 36 layers of 8 kv-heads x 128 over 65,536 pages,
needs 65,536 x 36 x 2 x 2 KiB = 9 GiB).
"""
from __future__ import annotations

import torch

from .base import BaseKVCache


class MHAKVCache(BaseKVCache):
    def __init__(
        self,
        num_kv_heads: int,
        num_layers: int,
        head_dim: int,
        num_pages: int,
        page_size: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> None:
        device = torch.device(device)
        assert device.type == "cuda", "AIOS only supports GPU execution"
        assert page_size == 1, "the MI355X backend only supports page_size=1"
        self._kv_buffer = torch.empty(
            (2, num_layers, num_pages, page_size, num_kv_heads, head_dim),
            device=device,
            dtype=dtype,
        )
        self._num_layers = num_layers
        self._k_buffer = self._kv_buffer[0]
        self._v_buffer = self._kv_buffer[1]
        self._device = device
        self._storage_shape = (num_pages * page_size, num_kv_heads, head_dim)

    def k_cache(self, index: int) -> torch.Tensor:
        return self._k_buffer[index]

    def v_cache(self, index: int) -> torch.Tensor:
        return self._v_buffer[index]

    def store_kv(
        self, k: torch.Tensor, v: torch.Tensor, out_loc: torch.Tensor, layer_id: int
    ) -> None:
        from aios_amd.kernel import store_cache

        store_cache(
            k_cache=self._k_buffer[layer_id].view(self._storage_shape),
            v_cache=self._v_buffer[layer_id].view(self._storage_shape),
            indices=out_loc,
            k=k,
            v=v,
        )

    @property
    def device(self) -> torch.device:
        return self._device

    @property
    def dtype(self) -> torch.dtype:
        return self._kv_buffer.dtype

    @property
    def num_layers(self) -> int:
        return self._num_layers

    @property
    def num_pages(self) -> int:
        return self._storage_shape[0]
