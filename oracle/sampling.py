"""Oracle: stateless candidate sampling (test infrastructure only).

Restates python/aios/engine/sample.py:
  * ``splitmix64_uniform`` / ``stateless_uniforms`` (:12-47): one U(0, 1)
    per (candidate seed, token step) from the SplitMix64 output function,
    53 high bits + 0.5 over 2^53, stored as float32;
  * ``sample_row`` (:66-160, the ``uniforms`` path): raw log-probs from the
    unmodified logits; forbidden ids set to -inf on a sampling copy; greedy
    (temperature <= 0 or top_k == 1, with top_p == 1) is the argmax;
    otherwise logits / temperature, the top-k candidates in descending
    order (or every id in index order when top_k == 0 and top_p == 1, or
    all ids sorted when top_k == 0), softmax, the top-p cut (remove where
    the cumulative probability before the id exceeds top_p, keep the
    first), softmax again, and the sampled position = the number of
    cumulative probabilities below u, clamped to the last candidate.

Ties in the descending order go to the lower token id (torch.topk / sort
leave tie order to the implementation; this is the order the kernel uses
and the documented rule).  Probabilities are float64 here; ``margin`` is
the distance from u to the nearest cumulative boundary (or from top_p to
the nearest cumulative sum that decides the cut), within which a float32
implementation may legitimately pick a neighbouring candidate.
"""
from __future__ import annotations

import numpy as np

_M64 = (1 << 64) - 1


def splitmix64(seed: int, step: int) -> int:
    """SplitMix64 output for state ``seed + (step + 1) * golden``."""
    v = (int(seed) + (int(step) + 1) * 0x9E3779B97F4A7C15) & _M64
    v = ((v ^ (v >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    v = ((v ^ (v >> 27)) * 0x94D049BB133111EB) & _M64
    return v ^ (v >> 31)


def splitmix64_uniform(seed: int, step: int) -> float:
    return (((splitmix64(seed, step) >> 11) & ((1 << 53) - 1)) + 0.5) / float(1 << 53)


def stateless_uniforms(seeds, steps: int) -> np.ndarray:
    if steps < 1:
        raise ValueError("steps must be positive")
    return np.array([[splitmix64_uniform(s, t) for t in range(steps)] for s in seeds],
                    dtype=np.float32)


def is_greedy(temperature: float, top_k: int, top_p: float) -> bool:
    """core.py SamplingParams.is_greedy."""
    return (temperature <= 0.0 or top_k == 1) and top_p == 1.0


def sample_row(logits, temperature: float, top_k: int, top_p: float, u: float,
               forbidden=(), detail: bool = False):
    """One row: (token, raw log-prob of the token, margin); with ``detail``
    the third item is a dict of both margins, the candidate ids in order and
    their cumulative probabilities (after the top-p cut)."""
    x = np.asarray(logits, dtype=np.float64)
    mx = x.max()
    raw = x - mx - np.log(np.exp(x - mx).sum())
    samp = x.copy()
    for f in set(int(i) for i in forbidden):
        samp[f] = -np.inf
    if is_greedy(temperature, top_k, top_p):
        tok = int(np.argmax(samp))  # first index of the maximum
        if detail:
            return tok, float(raw[tok]), {"u_margin": float("inf"), "cut_margin": float("inf"),
                                          "order": np.array([tok]), "cum": np.array([1.0])}
        return tok, float(raw[tok]), float("inf")
    scaled = samp / temperature
    ids = np.arange(len(x))
    if top_k > 0:
        order = np.lexsort((ids, -scaled))[: min(top_k, len(x))]
    elif top_p >= 1.0:
        order = ids
    else:
        order = np.lexsort((ids, -scaled))
    cand = scaled[order]
    e = np.exp(cand - cand.max())
    p = e / e.sum()
    cut_margin = float("inf")
    if top_p < 1.0:
        cum = np.cumsum(p)
        cut_margin = float(np.min(np.abs(cum[:-1] - top_p))) if len(p) > 1 else float("inf")
        remove = np.zeros(len(p), dtype=bool)
        remove[1:] = cum[:-1] > top_p
        e = np.where(remove, 0.0, e)
        p = e / e.sum()
    cum = np.cumsum(p)
    pos = min(int((cum < u).sum()), len(p) - 1)
    # distance to the nearest boundary: of u among the cumulative sums, and
    # of top_p among the sums that decide the cut
    u_margin = float(np.min(np.abs(cum - u)))
    margin = min(u_margin, cut_margin)
    tok = int(order[pos])
    if detail:
        return tok, float(raw[tok]), {"u_margin": u_margin, "cut_margin": cut_margin,
                                      "order": order, "cum": cum}
    return tok, float(raw[tok]), margin
