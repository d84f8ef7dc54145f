"""Oracle: paged KV scatter (test infrastructure only).

Restates python/aios/kernel/store.py:8-29: for every token t,
``k_cache[indices[t], :] = k[t, :]`` and ``v_cache[indices[t], :] = v[t, :]``
on the ``(num_slots, Hkv * D)`` view of one layer.  Rows are byte copies, so
the arrays may be any dtype (bf16 tensors are handled as uint16 bit patterns).
"""
from __future__ import annotations

import numpy as np


def scatter_rows(cache: np.ndarray, indices: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """Return a copy of ``cache`` with ``cache[indices[t]] = rows[t]``.

    ``cache`` is [num_slots, ...] and ``rows`` is [T, ...] with the same
    trailing shape.  Tokens are applied in order (store.py launches one
    program per token; out_loc is unique within a batch, so order is moot).
    """
    out = cache.copy()
    idx = np.asarray(indices).astype(np.int64).reshape(-1)
    if idx.shape[0] != rows.shape[0]:
        raise ValueError("KV write indices and K/V tensors must have matching token counts")
    for t in range(idx.shape[0]):
        out[idx[t]] = rows[t]
    return out


def store_kv(k_cache: np.ndarray, v_cache: np.ndarray, indices: np.ndarray,
             k: np.ndarray, v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Both halves of store_cache (store.py:32-61) on one layer."""
    if k_cache.ndim != 3 or v_cache.ndim != 3:
        raise ValueError("KV cache must have shape (num_slots, num_heads, head_dim)")
    if k.shape[1:] != k_cache.shape[1:] or v.shape[1:] != v_cache.shape[1:]:
        raise ValueError("K/V input shape does not match the cache layout")
    if np.asarray(indices).size != k.shape[0] or k.shape != v.shape:
        raise ValueError("KV write indices and K/V tensors must have matching token counts")
    return scatter_rows(k_cache, indices, k), scatter_rows(v_cache, indices, v)
