"""Oracle: Block-AttnRes depth mixer in float64 (test infrastructure only).

Two independent restatements of the mixer of
python/aios/models/minimind_ime.py:92-190:

* ``mix`` follows the production (Triton) kernels,
  python/aios/kernel/attnres.py:8-127: per source and token
  score = <x, query * key_norm_w> * rsqrt(mean(x^2) + eps); softmax over the
  sources; the weights rounded to bf16 (:92-97, the training rounding
  contract); output = sum_s w_s x_s, accumulated without intermediate
  rounding (the caller rounds it to bf16 where the kernel stores bf16).
* ``mix_materialized`` follows the materialised reference
  (minimind_ime.py:125-150): normalise every source with its RMS and the
  key-norm weight first, then dot with the query.

The two agree algebraically; tests/test_oracle.py pins them against each
other, against the reference's own known answer (zero query gives the plain
depth mean, tests/test_ime_attnres.py:59-66), and against closed forms (one
source returns itself; identical sources return that source; RMS
normalisation makes a score invariant to scaling its source).

Inputs are float arrays (bf16 values already widened); ``partial`` is the
optional last source.
"""
from __future__ import annotations

import numpy as np


def round_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even to bfloat16, returned as float32 values."""
    f = np.asarray(x, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = ((bits + 0x7FFF + lsb) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(f), f, out)


def _sources(bank: np.ndarray, partial: np.ndarray | None) -> np.ndarray:
    bank = np.asarray(bank, dtype=np.float64)
    if partial is None:
        return bank
    return np.concatenate([bank, np.asarray(partial, dtype=np.float64)[None]], axis=0)


def scores(bank, partial, query, key_norm_weight, eps: float) -> np.ndarray:
    """[S(+1), N] routing scores, expanded form (attnres.py:8-57)."""
    x = _sources(bank, partial)
    wq = np.asarray(query, dtype=np.float64) * np.asarray(key_norm_weight, dtype=np.float64)
    inv_rms = 1.0 / np.sqrt((x * x).mean(axis=-1) + eps)
    return np.einsum("snd,d->sn", x, wq) * inv_rms


def softmax_weights(sc: np.ndarray, round_weights: bool = True) -> np.ndarray:
    """Softmax over the source axis (attnres.py:86-97); bf16-rounded weights."""
    e = np.exp(sc - sc.max(axis=0, keepdims=True))
    w = e / e.sum(axis=0, keepdims=True)
    return round_bf16(w).astype(np.float64) if round_weights else w


def mix(bank, partial, query, key_norm_weight, eps: float,
        round_weights: bool = True) -> np.ndarray:
    """[N, D] float64 mixed hidden states (before the kernel's bf16 store)."""
    x = _sources(bank, partial)
    w = softmax_weights(scores(bank, partial, query, key_norm_weight, eps), round_weights)
    return np.einsum("sn,snd->nd", w, x)


def mix_materialized(bank, partial, query, key_norm_weight, eps: float,
                     round_weights: bool = True) -> np.ndarray:
    """minimind_ime.py:125-150: normalise, weight, dot, softmax, mix."""
    x = _sources(bank, partial)
    rms = np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    normalized = x / rms * np.asarray(key_norm_weight, dtype=np.float64)
    logits = np.einsum("d,snd->sn", np.asarray(query, dtype=np.float64), normalized)
    w = softmax_weights(logits, round_weights)
    return np.einsum("sn,snd->nd", w, x)
