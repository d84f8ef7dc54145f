"""Oracle: float32 CPU Qwen3 decoder and greedy CandidateGroup loop
(test infrastructure only).

Restates, densely and without a KV cache, what the reference's model computes
for a token sequence:

* decoder layer (python/aios/models/qwen3.py:52-109): fused QKV projection,
  per-head QK-RMSNorm, RoPE (layers/rotary.py:8-29, layers/attention.py:11-16),
  causal GQA attention with scale ``head_dim ** -0.5``, o_proj, residual-add
  RMSNorm (layers/norm.py:18-40), SwiGLU MLP (layers/activation.py:9-12);
* model (qwen3.py:112-173): embedding, layers, final norm, tied LM head
  (layers/embedding.py:13-41);
* the Block-AttnRes trunk of the 0.214B MiniMind-IME model
  (minimind_ime.py:193-326) with its depth mixers in the materialised
  form (:125-150): a list of bank sources, the block's running partial,
  a mixer before every attention and MLP and a final mixer;
* candidate rule of the CandidateGroup engine (ime.py:891-1115 with greedy
  sampling): candidate i starts from the i-th most likely first token, then
  takes the argmax at every step; the score is the average raw log-prob.

Everything is float32 (weights are the same bf16 values, widened), attention
is dense over the whole sequence, so the paged/cascade decomposition of the
product path does not appear here at all.

Pinning: the standard trunk equals transformers' Qwen3ForCausalLM on the same
weights (tests/test_oracle_hf.py).  The Block-AttnRes trunk composition is
pinned by its zero-query closed form in the same file: with every mixer query
zero each depth softmax is uniform, each mixer returns the standard residual
stream divided by its source count, and since every mixer output feeds an
RMSNorm (RMSNorm(x/S) is RMSNorm(x) with eps*S^2), the trunk at eps 1e-12
equals transformers' Qwen3 on the same weights; a planted wiring mistake (the
MLP mixer reading the sources without the attention delta) fails that check
by more than 1e-2.  Non-zero queries are pinned by the mixer's known answers
(oracle/attnres.py, tests/test_oracle.py).
"""
from __future__ import annotations

import torch


def _w32(w: dict) -> dict:
    f = lambda t: t.detach().to("cpu", torch.float32)
    out = {k: f(v) for k, v in w.items() if k != "layers"}
    out["layers"] = [{k: f(v) for k, v in lw.items()} for lw in w["layers"]]
    return out


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w


def _rope(x: torch.Tensor, pos: torch.Tensor, theta: float) -> torch.Tensor:
    """x [B, L, H, D]; rotate-half RoPE at integer positions pos [L]."""
    d = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    ang = pos.to(torch.float32)[:, None] * inv[None, :]
    cos = torch.cat([ang.cos(), ang.cos()], -1)[None, :, None, :]
    sin = torch.cat([ang.sin(), ang.sin()], -1)[None, :, None, :]
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return x * cos + torch.cat([-x2, x1], -1) * sin


class OracleModel:
    def __init__(self, config, weights: dict) -> None:
        self.c = config
        self.w = _w32(weights)

    def _attention(self, lw: dict, x: torch.Tensor) -> torch.Tensor:
        """Self-attention of normalised hidden states x [B, L, H] at positions
        0..L-1 (qwen3.py:52-75): projection, q/k norm, RoPE, causal GQA, o_proj."""
        c = self.c
        b, n, _ = x.shape
        hq, hkv, d = c.num_qo_heads, c.num_kv_heads, c.head_dim
        g = hq // hkv
        pos = torch.arange(n)
        mask = torch.ones(n, n, dtype=torch.bool).tril()
        qkv = x @ lw["qkv"].T
        q, k, v = qkv.split([hq * d, hkv * d, hkv * d], dim=-1)
        q = _rms(q.reshape(b, n, hq, d), lw["q_norm"], c.rms_norm_eps)
        k = _rms(k.reshape(b, n, hkv, d), lw["k_norm"], c.rms_norm_eps)
        v = v.reshape(b, n, hkv, d)
        q = _rope(q, pos, c.rope_theta)
        k = _rope(k, pos, c.rope_theta)
        k = k.repeat_interleave(g, dim=2)
        v = v.repeat_interleave(g, dim=2)
        s = torch.einsum("bihd,bjhd->bhij", q, k) * d ** -0.5
        s = s.masked_fill(~mask, float("-inf"))
        o = torch.einsum("bhij,bjhd->bihd", s.softmax(-1), v).reshape(b, n, hq * d)
        return o @ lw["o"].T

    @staticmethod
    def _mlp(lw: dict, x: torch.Tensor) -> torch.Tensor:
        gate, up = (x @ lw["gate_up"].T).chunk(2, dim=-1)
        return (torch.nn.functional.silu(gate) * up) @ lw["down"].T

    def _mix(self, sources: list, query: torch.Tensor, key_norm: torch.Tensor) -> torch.Tensor:
        """Depth mixer in its materialised form (minimind_ime.py:125-150):
        normalise each source, dot with the query, softmax over depth."""
        x = torch.stack(sources, 0)
        normalized = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.c.rms_norm_eps)
        logits = (normalized * key_norm * query).sum(-1)
        w = logits.softmax(0)
        return (w[..., None] * x).sum(0)

    @torch.no_grad()
    def logits(self, ids: torch.Tensor, start: int = 0) -> torch.Tensor:
        """ids [B, L] int64 -> logits [B, L - start, V] float32 of positions
        start..L-1 (causal attention, positions 0..L-1)."""
        c = self.c
        if c.residual_type == "block_attnres":
            return self._attnres_logits(ids, start)
        h = self.w["embed"][ids]
        residual = None
        for lw in self.w["layers"]:
            if residual is None:
                residual = h
            else:
                residual = h + residual
            x = self._attention(lw, _rms(residual, lw["input_norm"], c.rms_norm_eps))
            residual = x + residual
            h = self._mlp(lw, _rms(residual, lw["post_norm"], c.rms_norm_eps))
        x = _rms(h + residual, self.w["final_norm"], c.rms_norm_eps)
        return x[:, start:] @ self.w.get("lm_head", self.w["embed"]).T

    def _attnres_logits(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        """Block-AttnRes trunk (minimind_ime.py:193-326): a bank of the
        embedding and one summed delta per finished block; every layer mixes
        the bank (plus the block's running partial) before its attention and
        before its MLP; a final mixer over the whole bank feeds the norm."""
        c = self.c
        per = c.num_layers // c.attnres_num_blocks
        bank = [self.w["embed"][ids]]
        partial = None
        for i, lw in enumerate(self.w["layers"]):
            if i % per == 0:
                partial = None
            srcs = bank if partial is None else bank + [partial]
            h = self._mix(srcs, lw["attn_res_query"], lw["attn_res_norm"])
            delta = self._attention(lw, _rms(h, lw["input_norm"], c.rms_norm_eps))
            partial = delta if partial is None else partial + delta
            h = self._mix(bank + [partial], lw["mlp_res_query"], lw["mlp_res_norm"])
            partial = partial + self._mlp(lw, _rms(h, lw["post_norm"], c.rms_norm_eps))
            if (i + 1) % per == 0:
                bank.append(partial)
        h = self._mix(bank, self.w["final_res_query"], self.w["final_res_norm"])
        x = _rms(h, self.w["final_norm"], c.rms_norm_eps)
        return x[:, start:] @ self.w.get("lm_head", self.w["embed"]).T

    @torch.no_grad()
    def candidates(self, prefix, n: int, steps: int):
        """Greedy CandidateGroup: returns (ids [n, steps], avg_logprob [n],
        step_logprobs [n, steps, V]) with no EOS."""
        prefix = torch.as_tensor(prefix, dtype=torch.long)
        lp0 = self.logits(prefix[None], len(prefix) - 1)[0, -1].log_softmax(-1)
        top = lp0.topk(n)
        seq = torch.cat([prefix[None].expand(n, -1), top.indices[:, None]], 1)
        raw = [top.values]
        step_lp = [lp0[None].expand(n, -1)]
        for _ in range(steps - 1):
            lp = self.logits(seq, seq.shape[1] - 1)[:, -1].log_softmax(-1)
            tok = lp.argmax(-1)
            raw.append(lp.gather(1, tok[:, None]).squeeze(1))
            step_lp.append(lp)
            seq = torch.cat([seq, tok[:, None]], 1)
        ids = seq[:, len(prefix):]
        avg = torch.stack(raw, 1).mean(1)
        return ids, avg, torch.stack(step_lp, 1)

    @torch.no_grad()
    def teacher_forced(self, prefix, ids: torch.Tensor) -> torch.Tensor:
        """Log-probs [n, steps, V] of each step of given continuations ids [n, steps]."""
        prefix = torch.as_tensor(prefix, dtype=torch.long)
        n, steps = ids.shape
        seq = torch.cat([prefix[None].expand(n, -1), ids[:, :-1]], 1)
        return self.logits(seq, len(prefix) - 1).log_softmax(-1)


def top3_by_average(ids: torch.Tensor, avg: torch.Tensor, k: int = 3):
    """Distinct sequences ranked by average log-prob (ime.py:1109-1115 base score)."""
    order = torch.argsort(avg, descending=True, stable=True).tolist()
    seen, out = set(), []
    for i in order:
        t = tuple(ids[i].tolist())
        if t in seen:
            continue
        seen.add(t)
        out.append(t)
        if len(out) == k:
            break
    return out
