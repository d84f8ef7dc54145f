"""Oracle: batch metadata of the paged backend (test infrastructure only).

Restates FlashInferAttentionBackend.prepare_metadata
(python/aios/attention/flashinfer.py:209-250: the ``seqlens_q/k``,
``cu_seqlens`` and ``indices = cat(page_table[row, :len])`` lines) and
``get_last_indices`` (:111-112).
"""
from __future__ import annotations

import numpy as np


def cumulative(lengths) -> np.ndarray:
    """[0, l0, l0+l1, ...] as int32 (flashinfer.py:221-222)."""
    out = np.zeros(len(lengths) + 1, dtype=np.int64)
    for i, n in enumerate(lengths):
        out[i + 1] = out[i] + int(n)
    return out.astype(np.int32)


def build_metadata(seqlens_q, seqlens_k, page_table: np.ndarray, row_ids) -> dict:
    """cu_seqlens_q/k, flat page indices and last-token rows of one batch."""
    cu_q = cumulative(seqlens_q)
    cu_k = cumulative(seqlens_k)
    parts = [np.asarray(page_table[r, : int(n)], dtype=np.int32) for r, n in zip(row_ids, seqlens_k)]
    indices = np.concatenate(parts) if parts else np.zeros(0, dtype=np.int32)
    last = (cu_q[1:] - 1).astype(np.int64)
    return {
        "cu_seqlens_q": cu_q,
        "cu_seqlens_k": cu_k,
        "indices": indices.astype(np.int32),
        "last_indices": last,
        "seq_lens": np.asarray(seqlens_k, dtype=np.int32),
        "last_page_len": np.ones(len(seqlens_k), dtype=np.int32),
    }
