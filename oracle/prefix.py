"""Oracle: token-LCP prefix-reuse plan (test infrastructure only).

Restates ImeCompletionEngine._prepare_prefix's decision
(python/aios/ime.py:1116-1168): reuse the longest common token prefix of the
persisted and the new prefix, except that a strict backspace (new ids are a
proper prefix of the old ids) re-prefills from zero so the final-token logits
are exact; pages past the reused length are released and the extension is
freshly allocated.
"""
from __future__ import annotations


def token_lcp(left, right) -> int:
    n = 0
    for a, b in zip(left, right):
        if a != b:
            break
        n += 1
    return n


def plan_prefix(old_ids, old_pages, new_ids, next_page: int = 100):
    """Returns (reused, kept_pages, released_pages, allocated_pages, same)."""
    reused = token_lcp(old_ids, new_ids)
    same = bool(old_ids) and reused == len(old_ids) == len(new_ids)
    if same:
        return reused, list(old_pages), [], [], True
    if old_ids and reused == len(new_ids) < len(old_ids):
        reused = 0
    kept = list(old_pages[:reused])
    released = list(old_pages[reused:])
    allocated = list(range(next_page, next_page + len(new_ids) - reused))
    return reused, kept, released, allocated, False
