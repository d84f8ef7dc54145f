"""Paged KV append entry point (HIP kernel (a) behind the C ABI).

Same signature, validation and error messages as the reference's Triton
``store_cache`` (python/aios/kernel/store.py:32-61): scatter a flat batch of
K/V rows into a ``(num_slots, num_heads, head_dim)`` cache view, with k and v
allowed independent token strides.
"""
from __future__ import annotations

import torch

from aios_amd import _lib


def store_cache(
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    indices: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
) -> None:
    """Scatter ``k[t]``/``v[t]`` into cache row ``indices[t]``."""
    if k_cache.ndim != 3 or v_cache.ndim != 3:
        raise ValueError("KV cache must have shape (num_slots, num_heads, head_dim)")
    if k.shape[1:] != k_cache.shape[1:] or v.shape[1:] != v_cache.shape[1:]:
        raise ValueError("K/V input shape does not match the cache layout")
    if indices.numel() != k.shape[0] or k.shape != v.shape:
        raise ValueError("KV write indices and K/V tensors must have matching token counts")
    assert all(t.is_cuda for t in (k_cache, v_cache, indices, k, v))
    if k_cache.dtype != k.dtype or v_cache.dtype != v.dtype or k.dtype != v.dtype:
        raise ValueError("K/V dtype does not match the cache dtype")
    if k_cache.stride() != v_cache.stride():
        raise ValueError("K and V caches must share one layout")
    width = k_cache.shape[1] * k_cache.shape[2]
    # Rows must be contiguous inside a token; the token stride is free.
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("k", k), ("v", v)):
        if t.stride(2) != 1 or t.stride(1) != t.shape[2]:
            raise ValueError(f"{name} must have contiguous (heads, head_dim) rows")
    if indices.dtype != torch.int32:
        indices = indices.to(torch.int32)
    indices = indices.contiguous()
    stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    _lib.check(
        _lib.lib().aios_kv_append(
            k_cache.data_ptr(),
            v_cache.data_ptr(),
            k_cache.shape[0],
            k_cache.stride(0),
            indices.data_ptr(),
            k.data_ptr(),
            k.stride(0),
            v.data_ptr(),
            v.stride(0),
            k.shape[0],
            width,
            k.element_size(),
            stream,
        ),
        "aios_kv_append",
    )
