"""Oracle: offset-causal GQA paged attention in float64 (test infrastructure only).

Restates the math of the reference's attention path:

* ``_sdpa_prefill_attention`` (python/aios/attention/flashinfer.py:33-91):
  query row i of a request sits at absolute position ``cached_len + i`` and
  attends to key positions ``<= cached_len + i``; GQA maps query head ``hq``
  to KV head ``hq // (Hq / Hkv)`` (``repeat_interleave`` over heads, :62-65);
  scale ``head_dim ** -0.5`` (:131 of the backend).
* the per-request paged gather of ``_prefill_with_sdpa`` (:328-372): K/V rows
  of request r are ``cache[indices[cu_k[r] : cu_k[r+1]]]``.
* decode (:374-394): one query per row, ``cached_len = kv_len - 1``.
* the log-sum-exp split/merge of online softmax
  (resources/lesson-41-flashattention-online-softmax/run_lesson41.py:7-18).
"""
from __future__ import annotations

import math

import numpy as np


def attention_one(q: np.ndarray, k: np.ndarray, v: np.ndarray, cached_len: int,
                  sm_scale: float) -> np.ndarray:
    """One request.  q [Lq, Hq, D], k/v [Lk, Hkv, D]; returns [Lq, Hq, D] float64."""
    if q.ndim != 3 or k.ndim != 3 or v.ndim != 3:
        raise ValueError("q, k and v must use [tokens, heads, head_dim]")
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    if q.shape[2] != k.shape[2]:
        raise ValueError("q and k must have the same head_dim")
    if q.shape[1] % k.shape[1]:
        raise ValueError("query head count must be divisible by KV head count")
    if cached_len < 0 or cached_len + q.shape[0] != k.shape[0]:
        raise ValueError("cached_len + query length must equal KV length")
    lq, hq, _ = q.shape
    lk, hkv, _ = k.shape
    g = hq // hkv
    q64 = q.astype(np.float64)
    k64 = np.repeat(k.astype(np.float64), g, axis=1)  # head hq -> kv head hq // g
    v64 = np.repeat(v.astype(np.float64), g, axis=1)
    scores = np.einsum("qhd,khd->hqk", q64, k64) * sm_scale
    qpos = np.arange(cached_len, cached_len + lq)[:, None]
    kpos = np.arange(lk)[None, :]
    allowed = kpos <= qpos
    scores = np.where(allowed[None], scores, -np.inf)
    m = scores.max(axis=-1, keepdims=True)
    p = np.exp(scores - m)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hqk,khd->qhd", p, v64)


def paged_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                    indices: np.ndarray, cu_q: np.ndarray, cu_k: np.ndarray,
                    sm_scale: float) -> np.ndarray:
    """Varlen paged attention over a batch.

    q [total_q, Hq, D]; k_cache/v_cache [num_pages, Hkv, D] (page_size 1);
    request r owns q rows cu_q[r]:cu_q[r+1] and KV pages
    indices[cu_k[r]:cu_k[r+1]].  Returns [total_q, Hq, D] float64.
    """
    out = np.zeros(q.shape, dtype=np.float64)
    for r in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[r]), int(cu_q[r + 1])
        k0, k1 = int(cu_k[r]), int(cu_k[r + 1])
        if q1 == q0:
            continue
        pages = np.asarray(indices[k0:k1], dtype=np.int64)
        cached = (k1 - k0) - (q1 - q0)
        out[q0:q1] = attention_one(q[q0:q1], k_cache[pages], v_cache[pages], cached, sm_scale)
    return out


def decode_attention(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
                     indices: np.ndarray, cu_k: np.ndarray, sm_scale: float) -> np.ndarray:
    """Decode: row b has one query token and kv_len_b = cu_k[b+1]-cu_k[b] keys."""
    bs = len(cu_k) - 1
    cu_q = np.arange(bs + 1, dtype=np.int64)
    return paged_attention(q, k_cache, v_cache, indices, cu_q, cu_k, sm_scale)


def partial_state(q: np.ndarray, k: np.ndarray, v: np.ndarray, sm_scale: float):
    """Unmasked softmax partial of one query head set over a key subset.

    q [Hq, D], k/v [L, Hkv, D].  Returns (o [Hq, D] normalised, lse [Hq]) with
    lse the natural-log sum of exp(scores); an empty key set gives
    (zeros, -inf).
    """
    hq = q.shape[0]
    if k.shape[0] == 0:
        return np.zeros(q.shape, dtype=np.float64), np.full(hq, -np.inf)
    g = hq // k.shape[1]
    k64 = np.repeat(k.astype(np.float64), g, axis=1)
    v64 = np.repeat(v.astype(np.float64), g, axis=1)
    s = np.einsum("hd,khd->hk", q.astype(np.float64), k64) * sm_scale
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(axis=-1, keepdims=True)
    o = np.einsum("hk,khd->hd", p / l, v64)
    return o, (m + np.log(l))[:, 0]


def merge_states(states) -> tuple[np.ndarray, np.ndarray]:
    """Log-sum-exp merge of normalised partials [(o, lse), ...].

    m = max lse_i;  w_i = exp(lse_i - m);  o = sum w_i o_i / sum w_i.
    """
    os_ = [np.asarray(o, dtype=np.float64) for o, _ in states]
    ls = np.stack([np.asarray(l, dtype=np.float64) for _, l in states])  # [n, H]
    m = ls.max(axis=0)
    safe_m = np.where(np.isfinite(m), m, 0.0)
    w = np.exp(ls - safe_m)  # exp(-inf) = 0 for empty partials
    den = w.sum(axis=0)
    num = sum(w[i][:, None] * os_[i] for i in range(len(os_)))
    with np.errstate(invalid="ignore", divide="ignore"):
        o = np.where(den[:, None] > 0, num / np.where(den > 0, den, 1.0)[:, None], 0.0)
    lse = np.where(den > 0, safe_m + np.log(np.where(den > 0, den, 1.0)), -np.inf)
    return o, lse


def online_softmax(scores, values, block: int):
    """Blocked online softmax of one query (run_lesson41.py:7-18 restated).

    Returns (output, final m, final l).  Equals softmax(scores) @ values for
    every block size.
    """
    m = -math.inf
    l = 0.0
    out = [0.0] * len(values[0])
    for start in range(0, len(scores), block):
        s = scores[start:start + block]
        vb = values[start:start + block]
        new_m = max(m, max(s))
        alpha = 0.0 if m == -math.inf else math.exp(m - new_m)
        p = [math.exp(x - new_m) for x in s]
        out = [alpha * x for x in out]
        for w, row in zip(p, vb):
            for j, x in enumerate(row):
                out[j] += w * x
        l = alpha * l + sum(p)
        m = new_m
    return [x / l for x in out], m, l
