"""KV-cached Qwen3 decoder on the host cores (test infrastructure only).

The CPU leg of the full-model baseline: the reference's decoder forward
(python/aios/models/qwen3.py:52-173: fused QKV projection, per-head
QK-RMSNorm, rotate-half RoPE, o_proj, residual-add RMSNorm, SwiGLU MLP, final
norm, LM head on each request's last token) over a token-granular paged KV
pool ``[layers, pages, kv_heads, head_dim]`` written the way
kernel/store.py:8-29 writes it (row ``out_loc[i]`` receives token i's K/V),
with attention by the reference's CPU path, oracle/sdpa_cpu.py
(flashinfer.py:33-91 driven per request as in :328-372).  Standard residual
trunk only.

Runs in bfloat16 (the reference's dtype: matmuls and attention in bf16,
RMSNorm and RoPE computed in float32 and rounded back) or float32.  Used by
bench.py's ``cpu_baseline`` leg; pinned by tests/test_oracle.py against
OracleModel (itself pinned against transformers' Qwen3ForCausalLM): float32
prefill and decode logits equal the dense recomputation within 1e-4, and a
relabelling of the pages leaves them unchanged.
"""
from __future__ import annotations

import torch

from .sdpa_cpu import paged_attention_cpu


class PagedCpuDecoder:
    def __init__(self, config, weights: dict, dtype: torch.dtype = torch.bfloat16,
                 num_pages: int = 1024) -> None:
        if config.residual_type != "standard":
            raise ValueError("PagedCpuDecoder restates the standard residual trunk only")
        self.c = config
        self.dtype = dtype
        cvt = lambda t: t.detach().to("cpu", dtype).contiguous()
        self.w = {k: cvt(v) for k, v in weights.items() if k != "layers"}
        self.layers = [{k: cvt(v) for k, v in lw.items()} for lw in weights["layers"]]
        shape = (config.num_layers, num_pages, config.num_kv_heads, config.head_dim)
        self.k_cache = torch.zeros(shape, dtype=dtype)
        self.v_cache = torch.zeros(shape, dtype=dtype)
        d = config.head_dim
        self.inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.float32) / d))

    def _rms(self, x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
        x32 = x.float()
        y = x32 * torch.rsqrt(x32.pow(2).mean(-1, keepdim=True) + self.c.rms_norm_eps)
        return (y * w.float()).to(self.dtype)

    def _rope(self, x: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """x [T, H, D] at integer positions pos [T] (rotate-half form)."""
        ang = pos.to(torch.float32)[:, None] * self.inv_freq[None, :]
        cos = torch.cat([ang.cos(), ang.cos()], -1)[:, None, :]
        sin = torch.cat([ang.sin(), ang.sin()], -1)[:, None, :]
        x32 = x.float()
        h = x.shape[-1] // 2
        rot = torch.cat([-x32[..., h:], x32[..., :h]], -1)
        return (x32 * cos + rot * sin).to(self.dtype)

    @torch.no_grad()
    def forward(self, ids: torch.Tensor, positions: torch.Tensor, out_loc: torch.Tensor,
                indices: torch.Tensor, cu_q: list, cu_k: list) -> torch.Tensor:
        """One batch: tokens ``ids`` [T] at ``positions`` [T] whose K/V go to
        pages ``out_loc`` [T]; request r owns tokens cu_q[r]:cu_q[r+1] and
        attends to the pages indices[cu_k[r]:cu_k[r+1]] (its own new tokens
        last).  Returns the logits [R, vocab] of each request's last token."""
        c = self.c
        hq, hkv, d = c.num_qo_heads, c.num_kv_heads, c.head_dim
        t = ids.shape[0]
        loc = out_loc.to(torch.long)
        h = self.w["embed"][ids.to(torch.long)]
        residual = None
        for li, lw in enumerate(self.layers):
            residual = h if residual is None else h + residual
            x = self._rms(residual, lw["input_norm"])
            q, k, v = (x @ lw["qkv"].T).split([hq * d, hkv * d, hkv * d], dim=-1)
            q = self._rope(self._rms(q.reshape(t, hq, d), lw["q_norm"]), positions)
            k = self._rope(self._rms(k.reshape(t, hkv, d), lw["k_norm"]), positions)
            self.k_cache[li][loc] = k
            self.v_cache[li][loc] = v.reshape(t, hkv, d)
            o = paged_attention_cpu(q, self.k_cache[li], self.v_cache[li], indices, cu_q, cu_k,
                                    d ** -0.5)
            residual = o @ lw["o"].T + residual
            x = self._rms(residual, lw["post_norm"])
            gate, up = (x @ lw["gate_up"].T).chunk(2, dim=-1)
            h = (torch.nn.functional.silu(gate.float()).to(self.dtype) * up) @ lw["down"].T
        last = torch.tensor([int(e) - 1 for e in cu_q[1:]], dtype=torch.long)
        x = self._rms((h + residual)[last], self.w["final_norm"])
        return (x @ self.w.get("lm_head", self.w["embed"]).T).float()

    def prefill(self, ids: list, pages: torch.Tensor, cached_len: int = 0) -> torch.Tensor:
        """One request: ids[cached_len:] against the cached ids[:cached_len]
        (page i holds position i); logits [vocab] of the last token."""
        n = len(ids)
        pos = torch.arange(cached_len, n, dtype=torch.int32)
        new = torch.as_tensor(ids[cached_len:], dtype=torch.long)
        return self.forward(new, pos, pages[cached_len:n], pages[:n].to(torch.int32),
                            [0, n - cached_len], [0, n])[0]

    def decode(self, tokens: torch.Tensor, rows_pages: list, out_loc: torch.Tensor) -> torch.Tensor:
        """One decode step: row r feeds tokens[r] whose K/V go to out_loc[r],
        the last page of rows_pages[r] (its whole page list, prefix first)."""
        cu_k = [0]
        for p in rows_pages:
            cu_k.append(cu_k[-1] + len(p))
        pos = torch.tensor([len(p) - 1 for p in rows_pages], dtype=torch.int32)
        idx = torch.cat(rows_pages).to(torch.int32)
        return self.forward(tokens, pos, out_loc, idx, list(range(len(rows_pages) + 1)), cu_k)
