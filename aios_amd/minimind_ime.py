"""MiniMind-IME decoders: the standard-residual model is the Qwen3 decoder;
the 0.214B Block-AttnRes model replaces its residual stream with a depth
bank and 2 * L + 1 depth mixers (python/aios/models/minimind_ime.py:193-354).

Block-AttnRes trunk (minimind_ime.py:255-326), per block of
``layers_per_attnres_block`` layers over a bank whose source 0 is the token
embedding and whose source b + 1 is block b's summed deltas:

    h       = mix(bank, partial)               attention mixer
    partial = partial + attention(RMSNorm(h))  (the delta itself at block start)
    h       = mix(bank, partial)               MLP mixer
    partial = partial + mlp(RMSNorm(h))
    (block end) bank.append(partial)
    final:  logits = LMHead(RMSNorm(mix(bank)))

gfx950 composition: every mixer is one launch of the depth-mix kernel
(``aios_attnres_mix_ex``) that also forms the running partial from the
pending delta (the bf16 adds above, rounded as torch rounds them) and, at a
block end, stores it straight into the bank's next slot -- so the mix of
``bank[:k]`` with that partial is the mix of ``bank[:k + 1]`` the reference
performs after its copy.  Each RMSNorm is folded into the projection that
consumes it (the few-row GEMM prologue), as in the standard decoder.
"""
from __future__ import annotations

import torch

from aios_amd.attention import BaseAttentionBackend
from aios_amd.config import ModelConfig
from aios_amd.core import get_global_ctx
from aios_amd.qwen3 import Qwen3ForCausalLM


class DepthBank:
    """The depth bank of one forward and the block's running partial, with
    the mixer calls that advance them (minimind_ime.py:215-252, 287-326).

    ``add(delta, closes_block)`` records a layer's delta without touching
    memory; the next ``mix`` forms ``partial + delta`` inside its launch and
    stores it -- into the partial buffer, or, when the delta closed a block,
    into the bank's next slot (the block's new depth source).
    """

    def __init__(self, storage: torch.Tensor, part_buf: torch.Tensor, ops, eps: float) -> None:
        self.storage = storage      # [blocks + 1, tokens, hidden]; storage[0] = embedding
        self.part_buf = part_buf    # [tokens, hidden]
        self.ops = ops
        self.eps = eps
        self.count = 1              # sources in the bank
        self.partial = None         # the block's running partial, as materialised so far
        self.pending = None         # the delta not yet added into it
        self.to_bank = False        # pending closes its block

    def add(self, delta: torch.Tensor, closes_block: bool = False) -> None:
        if self.pending is not None:
            raise RuntimeError("two deltas without a mix between them")
        self.pending = delta
        self.to_bank = closes_block

    def mix(self, weighted_query: torch.Tensor) -> torch.Tensor:
        bank = self.storage[: self.count]
        if self.pending is None:
            return self.ops.attnres_mix(bank, self.partial, weighted_query, self.eps)
        if self.to_bank:
            out = self.ops.attnres_mix_step(bank, self.partial, self.pending, weighted_query,
                                            self.eps, self.storage[self.count])
            self.count += 1
            self.partial = None
        else:
            out = self.ops.attnres_mix_step(bank, self.partial, self.pending, weighted_query,
                                            self.eps, self.part_buf)
            self.partial = self.part_buf
        self.pending = None
        self.to_bank = False
        return out


class MiniMindBlockAttnResForCausalLM(Qwen3ForCausalLM):
    """Block-AttnRes decoder + tied LM head (minimind_ime.py:255-354).
    Mixer weights per layer: ``attn_res_query`` / ``attn_res_norm`` and
    ``mlp_res_query`` / ``mlp_res_norm``; the final mixer's are
    ``final_res_query`` / ``final_res_norm``."""

    # the embedding rows go straight into the depth bank (forward below)
    takes_input_embeds = False

    def __init__(self, config: ModelConfig, weights: dict, device,
                 attn_backend: BaseAttentionBackend | None = None,
                 max_positions: int | None = None, ops=None) -> None:
        if config.residual_type != "block_attnres":
            raise ValueError("MiniMindBlockAttnResForCausalLM needs residual_type 'block_attnres'")
        super().__init__(config, weights, device, attn_backend, max_positions, ops)

        # Routing query folded with the key-norm weight once, in fp32
        # (BlockAttnResMixer._routing_query, minimind_ime.py:115-127).
        def wq(query, norm):
            return (query.float() * norm.float()).contiguous()

        self._wq_attn = [wq(lw["attn_res_query"], lw["attn_res_norm"]) for lw in weights["layers"]]
        self._wq_mlp = [wq(lw["mlp_res_query"], lw["mlp_res_norm"]) for lw in weights["layers"]]
        self._wq_final = wq(weights["final_res_query"], weights["final_res_norm"])

    def forward(self) -> torch.Tensor:
        ctx = get_global_ctx()
        batch = ctx.batch
        c = self.config
        ops = self.ops
        eps = c.rms_norm_eps
        per_block = c.layers_per_attnres_block
        ids = batch.input_ids
        t = ids.shape[0]
        embed = self.w["embed"]
        # The whole depth bank, allocated once per forward (minimind_ime.py:287-299).
        bank = torch.empty((c.attnres_num_blocks + 1, t, c.hidden_size), dtype=embed.dtype,
                           device=embed.device)
        torch.index_select(embed, 0, ids, out=bank[0])
        part_buf = torch.empty((t, c.hidden_size), dtype=embed.dtype, device=embed.device)
        depth = DepthBank(bank, part_buf, ops, eps)
        positions = batch.positions
        for i, lw in enumerate(self.w["layers"]):
            h = depth.mix(self._wq_attn[i])
            qkv, _ = ops.add_rmsnorm_linear(h, None, lw["input_norm"], eps, lw["qkv"])
            depth.add(self._attention(i, qkv, positions, ctx.kv_cache, batch))
            h = depth.mix(self._wq_mlp[i])
            act, _ = ops.add_rmsnorm_linear(h, None, lw["post_norm"], eps, lw["gate_up"],
                                            silu=True)
            depth.add(ops.linear(act, lw["down"]), closes_block=(i + 1) % per_block == 0)
        h = depth.mix(self._wq_final)
        if depth.count != c.attnres_num_blocks + 1:
            raise RuntimeError("AttnRes block produced no residual delta")
        if batch.is_prefill and not batch.return_all_logits:
            h = h[batch.attn_metadata.get_last_indices(batch.size)]
        logits, _ = ops.add_rmsnorm_linear(h, None, self.w["final_norm"], eps,
                                           self.w.get("lm_head", embed))
        return logits


def build_causal_lm(config: ModelConfig, weights: dict, device,
                    attn_backend: BaseAttentionBackend | None = None,
                    max_positions: int | None = None, ops=None) -> Qwen3ForCausalLM:
    """The decoder class a config selects (MiniMindIMEForCausalLM's dispatch,
    minimind_ime.py:329-350): standard residuals -> the Qwen3 decoder,
    block_attnres -> the Block-AttnRes trunk."""
    cls = (MiniMindBlockAttnResForCausalLM if config.residual_type == "block_attnres"
           else Qwen3ForCausalLM)
    return cls(config, weights, device, attn_backend=attn_backend, max_positions=max_positions,
               ops=ops)
