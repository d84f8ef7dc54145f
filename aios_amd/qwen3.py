"""Qwen3 / MiniMind decoder in PyTorch-ROCm eager, the caller of the backend.

Restates python/aios/models/qwen3.py:31-173 and the layer ops it uses
(python/aios/layers/norm.py:10-40, activation.py:9-12, rotary.py:8-29,
attention.py:6-16, embedding.py:13-41) without FlashInfer: RMSNorm, the
residual-add RMSNorm, per-head q/k RMSNorm + RoPE and SiLU-and-mul are the
gfx950 kernels of aios_amd.layers (one launch each); the projections are
torch GEMMs.  Attention goes through the backend exactly as in the
reference: ``backend.forward(q, k, v, kv_cache, layer_id, batch)`` once per
layer with q/k/v as ``[tokens, heads, head_dim]`` (v a strided view into the
fused qkv projection).

Weights are synthetic (seeded N(0, 0.02), norm weights 1, tied embedding);
no checkpoint is loaded.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from aios_amd.attention import BaseAttentionBackend, Mi355xAttentionBackend
from aios_amd.config import ModelConfig
from aios_amd.core import get_global_ctx


def init_weights(config: ModelConfig, seed: int, device="cpu",
                 dtype: torch.dtype = torch.bfloat16, std: float = 0.02) -> dict:
    """Seeded synthetic weights.  Generated on ``device`` with a generator of
    that device, so CPU-generated weights copied to the GPU match a CPU run."""
    dev = torch.device(device)
    g = torch.Generator(device=dev).manual_seed(seed)
    h, d = config.hidden_size, config.head_dim
    q_size, kv_size = config.num_qo_heads * d, config.num_kv_heads * d

    def lin(out_f, in_f):
        return (torch.randn(out_f, in_f, generator=g, device=dev, dtype=torch.float32) * std).to(dtype)

    w = {"embed": lin(config.vocab_size, h), "final_norm": torch.ones(h, device=dev, dtype=dtype),
         "layers": []}
    for _ in range(config.num_layers):
        w["layers"].append({
            "input_norm": torch.ones(h, device=dev, dtype=dtype),
            "qkv": lin(q_size + 2 * kv_size, h),
            "q_norm": torch.ones(d, device=dev, dtype=dtype),
            "k_norm": torch.ones(d, device=dev, dtype=dtype),
            "o": lin(h, q_size),
            "post_norm": torch.ones(h, device=dev, dtype=dtype),
            "gate_up": lin(2 * config.intermediate_size, h),
            "down": lin(h, config.intermediate_size),
        })
        if config.residual_type == "block_attnres":
            # the two depth mixers of the layer (minimind_ime.py:208-213):
            # routing query and key-norm weight each
            w["layers"][-1].update({
                "attn_res_query": lin(1, h)[0],
                "attn_res_norm": torch.ones(h, device=dev, dtype=dtype),
                "mlp_res_query": lin(1, h)[0],
                "mlp_res_norm": torch.ones(h, device=dev, dtype=dtype),
            })
    if config.residual_type == "block_attnres":
        w["final_res_query"] = lin(1, h)[0]
        w["final_res_norm"] = torch.ones(h, device=dev, dtype=dtype)
    if not config.tie_word_embeddings:
        w["lm_head"] = lin(config.vocab_size, h)
    return w


def weights_to(w: dict, device, dtype=None) -> dict:
    def mv(t):
        t = t.to(device)
        return t.to(dtype) if dtype is not None else t
    out = {k: mv(v) for k, v in w.items() if k != "layers"}
    out["layers"] = [{k: mv(v) for k, v in lw.items()} for lw in w["layers"]]
    return out


class RotaryEmbedding:
    """fp32 cos/sin tables [max_positions, head_dim] (rotary.py:8-29), and
    the same rounded to bf16 (nearest even: the rounding the q/k rotation
    applies to each entry) for the decode launch that rotates on load."""

    def __init__(self, head_dim: int, max_positions: int, base: float, device) -> None:
        inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
        t = torch.arange(max_positions, dtype=torch.float32)
        emb = torch.cat((torch.outer(t, inv_freq),) * 2, dim=-1)
        self.cos = emb.cos().to(device)
        self.sin = emb.sin().to(device)
        self.cos_bf16 = self.cos.to(torch.bfloat16)
        self.sin_bf16 = self.sin.to(torch.bfloat16)


class Qwen3ForCausalLM:
    """Decoder + tied LM head.  ``forward()`` reads the batch from the global
    context like the reference (qwen3.py:140-173).  ``ops`` supplies linear,
    add_rmsnorm_linear and qk_norm_rope (default: the gfx950 kernels,
    aios_amd.layers.HipOps)."""

    # forward() uses batch.input_embeds when the caller gathered them
    takes_input_embeds = True

    def __init__(self, config: ModelConfig, weights: dict, device,
                 attn_backend: BaseAttentionBackend | None = None,
                 max_positions: int | None = None, ops=None) -> None:
        self.config = config
        self.device = torch.device(device)
        self.w = weights
        self.attn_backend = attn_backend or Mi355xAttentionBackend(config)
        if ops is None:
            from aios_amd.layers import HipOps

            ops = HipOps()
        self.ops = ops
        self.rotary = RotaryEmbedding(config.head_dim,
                                      max_positions or min(config.max_position_embeddings, 8192),
                                      config.rope_theta, self.device)
        self._q_size = config.num_qo_heads * config.head_dim
        self._kv_size = config.num_kv_heads * config.head_dim

    def _attention(self, i: int, qkv: torch.Tensor, positions, kv_cache, batch) -> torch.Tensor:
        """qwen3.py:52-75 after the qkv projection: per-head q/k RMSNorm +
        RoPE, the backend, o_proj (v stays a strided view into qkv, as in the
        reference)."""
        out = self.attention_core(i, qkv, positions, kv_cache, batch)
        return self.ops.linear(out.reshape(qkv.shape[0], -1), self.w["layers"][i]["o"])

    def attention_core(self, i: int, qkv: torch.Tensor, positions, kv_cache,
                       batch) -> torch.Tensor:
        """The attention of layer i between the qkv projection and o_proj:
        q/k norm + RoPE and the backend call -> [T, Hq, D] (or [T, Hq*D]).
        An appending decode batch on the gfx950 ops takes the norm and
        rotation inside the decode launch (forward_rope)."""
        c = self.config
        lw = self.w["layers"][i]
        t = qkv.shape[0]
        hq, hkv, d = c.num_qo_heads, c.num_kv_heads, c.head_dim
        v = qkv[:, self._q_size + self._kv_size:].view(t, hkv, d)
        be = self.attn_backend
        if (getattr(self.ops, "rope_in_decode", False)
                and getattr(be, "decode_rope_applies", None) is not None
                and be.decode_rope_applies(batch)):
            q = qkv[:, :self._q_size].view(t, hq, d)
            k = qkv[:, self._q_size:self._q_size + self._kv_size].view(t, hkv, d)
            out = be.forward_rope(q, k, v, lw["q_norm"], lw["k_norm"], self.rotary.cos_bf16,
                                  self.rotary.sin_bf16, positions, c.rms_norm_eps, kv_cache, i,
                                  batch)
        else:
            q, k = self.ops.qk_norm_rope(qkv, lw["q_norm"], lw["k_norm"], self.rotary.cos,
                                         self.rotary.sin, positions, hq, hkv, d, c.rms_norm_eps)
            out = be.forward(q, k, v, kv_cache, i, batch)
        return out

    def forward(self) -> torch.Tensor:
        """Decoder layers of qwen3.py:76-109: input RMSNormFused -> qkv
        projection, attention, post RMSNormFused -> gate/up projection ->
        SiLU-and-mul, down projection; each norm is folded into the projection
        that consumes it and the activation into the gate/up projection."""
        ctx = get_global_ctx()
        batch = ctx.batch
        c = self.config
        ops = self.ops
        h = (batch.input_embeds if batch.input_embeds is not None
             else F.embedding(batch.input_ids, self.w["embed"]))
        positions = batch.positions
        residual = None
        for i, lw in enumerate(self.w["layers"]):
            qkv, residual = ops.add_rmsnorm_linear(h, residual, lw["input_norm"], c.rms_norm_eps,
                                                   lw["qkv"])
            x = self._attention(i, qkv, positions, ctx.kv_cache, batch)
            act, residual = ops.add_rmsnorm_linear(x, residual, lw["post_norm"], c.rms_norm_eps,
                                                   lw["gate_up"], silu=True)
            h = ops.linear(act, lw["down"])
        if batch.is_prefill and not batch.return_all_logits:
            last = batch.attn_metadata.get_last_indices(batch.size)
            h, residual = h[last], residual[last]
        logits, _ = ops.add_rmsnorm_linear(h, residual, self.w["final_norm"], c.rms_norm_eps,
                                           self.w.get("lm_head", self.w["embed"]))
        return logits
