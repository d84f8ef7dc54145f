"""Torch restatement of the reference's CPU attention path (test infrastructure only).

This is the path the reference runs when FlashInfer cannot (head_dim not in
{64, 128, 256}) and the only attention of the reference that executes on a
CPU: python/aios/attention/flashinfer.py:33-91 (``_sdpa_prefill_attention``)
driven per request by ``_prefill_with_sdpa`` (:328-372), with decode issued as
q_len 1 and cached_len = kv_len - 1.  ``bench.py`` times it on the host cores
as the ``cpu_baseline`` ("port": a restatement, not the reference's code).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def sdpa_prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                           cached_len: int, sm_scale: float) -> torch.Tensor:
    """One request: NHD q/k/v -> BHLD, repeat GQA heads, offset-causal SDPA."""
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
    qb = q.transpose(0, 1).unsqueeze(0)
    kb = k.transpose(0, 1).unsqueeze(0)
    vb = v.transpose(0, 1).unsqueeze(0)
    rep = q.shape[1] // k.shape[1]
    if rep != 1:
        kb = kb.repeat_interleave(rep, dim=1)
        vb = vb.repeat_interleave(rep, dim=1)
    if cached_len == 0:
        mask = None
        causal = True
    else:
        qpos = torch.arange(cached_len, cached_len + q.shape[0], device=q.device)
        kpos = torch.arange(k.shape[0], device=q.device)
        mask = (kpos.unsqueeze(0) <= qpos.unsqueeze(1)).unsqueeze(0).unsqueeze(0)
        causal = False
    out = F.scaled_dot_product_attention(qb, kb, vb, attn_mask=mask, dropout_p=0.0,
                                         is_causal=causal, scale=sm_scale)
    return out.squeeze(0).transpose(0, 1).contiguous()


def paged_attention_cpu(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        indices: torch.Tensor, cu_q, cu_k, sm_scale: float) -> torch.Tensor:
    """Per-request loop: gather pages, then sdpa_prefill_attention (:328-372)."""
    outs = []
    for r in range(len(cu_q) - 1):
        q0, q1 = int(cu_q[r]), int(cu_q[r + 1])
        k0, k1 = int(cu_k[r]), int(cu_k[r + 1])
        pages = indices[k0:k1].to(torch.long)
        keys = k_cache[pages]
        vals = v_cache[pages]
        outs.append(sdpa_prefill_attention(q[q0:q1], keys, vals, cached_len=(k1 - k0) - (q1 - q0),
                                           sm_scale=sm_scale))
    return torch.cat(outs, dim=0).reshape(q.shape[0], -1)
