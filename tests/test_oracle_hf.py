"""Pins the float32 model oracle (oracle/model.py) against an independent
Qwen3 implementation: transformers' ``Qwen3ForCausalLM`` (CPU only).

The reference's decoder (python/aios/models/qwen3.py:52-173, its packing in
models/weight.py:48-70 and SiLU of the first half in layers/activation.py:
9-12) is standard Qwen3, which transformers implements independently of this
repository.  The same weights reach both models through the exported bundle
(``aios_amd.weights.save_bundle`` writes the HF tensor names, splitting the
packed q/k/v and gate/up projections), so a shared misreading of the MLP
half order, the q/k-norm -> RoPE order, the residual placement or the
packing order fails here.  The Block-AttnRes trunk
(python/aios/models/minimind_ime.py:193-326) is pinned here by its
zero-query closed form: with every mixer query zero it must equal the
standard trunk, i.e. transformers' model on the same weights.
"""
from __future__ import annotations

import pytest
import torch

transformers = pytest.importorskip("transformers")

from aios_amd.config import ModelConfig  # noqa: E402
from aios_amd.qwen3 import init_weights  # noqa: E402
from aios_amd.weights import save_bundle  # noqa: E402
from oracle.model import OracleModel  # noqa: E402


def _hf_model(c: ModelConfig, bundle):
    from safetensors.torch import load_file
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hc = Qwen3Config(
        vocab_size=c.vocab_size, hidden_size=c.hidden_size,
        intermediate_size=c.intermediate_size, num_hidden_layers=c.num_layers,
        num_attention_heads=c.num_qo_heads, num_key_value_heads=c.num_kv_heads,
        head_dim=c.head_dim, rms_norm_eps=c.rms_norm_eps, rope_theta=c.rope_theta,
        max_position_embeddings=c.max_position_embeddings,
        tie_word_embeddings=c.tie_word_embeddings, attention_bias=False,
        attn_implementation="eager")
    model = Qwen3ForCausalLM(hc).to(torch.float32).eval()
    sd = load_file(str(bundle / "model.safetensors"))
    missing, unexpected = model.load_state_dict({k: v.float() for k, v in sd.items()},
                                                strict=False)
    assert not unexpected, unexpected
    assert set(missing) <= ({"lm_head.weight"} if c.tie_word_embeddings else set()), missing
    if c.tie_word_embeddings:
        model.tie_weights()
        assert torch.equal(model.lm_head.weight, model.model.embed_tokens.weight)
    return model


def _weights(c: ModelConfig, seed: int) -> dict:
    """Synthetic float32 weights with non-trivial norm weights (all-ones
    norms would hide a norm applied to the wrong tensor)."""
    w = init_weights(c, seed, "cpu", dtype=torch.float32, std=0.15)
    g = torch.Generator().manual_seed(seed + 1)
    for lw in w["layers"]:
        for key in ("input_norm", "post_norm", "q_norm", "k_norm"):
            lw[key].copy_(torch.rand(lw[key].shape, generator=g) + 0.5)
    w["final_norm"].copy_(torch.rand(w["final_norm"].shape, generator=g) + 0.5)
    return w


SHAPES = {
    # 8 query / 2 KV heads of 96 (the MiniMind-0.1B and op-test head shape, G = 4)
    "g4_d96": dict(num_layers=3, num_qo_heads=8, num_kv_heads=2, head_dim=96, hidden_size=128,
                   vocab_size=211, intermediate_size=160, rms_norm_eps=1e-5,
                   rope_theta=1000000.0),
    # 4 query / 2 KV heads of 128 (the Qwen3-0.6B head shape, G = 2), rope 1e4
    "g2_d128": dict(num_layers=2, num_qo_heads=4, num_kv_heads=2, head_dim=128, hidden_size=96,
                    vocab_size=173, intermediate_size=128, rms_norm_eps=1e-6,
                    rope_theta=10000.0),
    # untied LM head, G = 3 at head_dim 64
    "g3_d64_untied": dict(num_layers=2, num_qo_heads=6, num_kv_heads=2, head_dim=64,
                          hidden_size=64, vocab_size=101, intermediate_size=96,
                          rms_norm_eps=1e-6, rope_theta=1000000.0, tie_word_embeddings=False),
}


@pytest.mark.parametrize("shape", sorted(SHAPES))
def test_oracle_logits_match_transformers_qwen3(shape, tmp_path):
    c = ModelConfig(**SHAPES[shape])
    w = _weights(c, 11)
    bundle = save_bundle(c, w, tmp_path / "bundle")
    hf = _hf_model(c, bundle)
    ids = torch.randint(0, c.vocab_size, (2, 19), generator=torch.Generator().manual_seed(5))
    with torch.no_grad():
        ref = hf(input_ids=ids).logits
    got = OracleModel(c, w).logits(ids)
    assert got.shape == ref.shape
    scale = ref.abs().max().item()
    assert scale > 1.0  # the logits are not trivially small
    err = (got - ref).abs().max().item()
    assert err <= 1e-5, (shape, err, scale)
    # the oracle's `start` selects the last positions of the same forward
    tail = OracleModel(c, w).logits(ids, start=15)
    assert (tail - ref[:, 15:]).abs().max().item() <= 1e-5


def test_oracle_greedy_candidates_match_transformers(tmp_path):
    """The oracle's greedy CandidateGroup (top-n first tokens, then argmax)
    reproduces a loop over transformers' logits token for token."""
    c = ModelConfig(**SHAPES["g4_d96"])
    w = _weights(c, 23)
    hf = _hf_model(c, save_bundle(c, w, tmp_path / "bundle"))
    prefix = torch.randint(0, c.vocab_size, (12,), generator=torch.Generator().manual_seed(9))
    n, steps = 4, 6
    ids, avg, _ = OracleModel(c, w).candidates(prefix.tolist(), n, steps)
    with torch.no_grad():
        lp0 = hf(input_ids=prefix[None]).logits[0, -1].log_softmax(-1)
        top = lp0.topk(n)
        seq = torch.cat([prefix[None].expand(n, -1), top.indices[:, None]], 1)
        raw = [top.values]
        for _ in range(steps - 1):
            lp = hf(input_ids=seq).logits[:, -1].log_softmax(-1)
            tok = lp.argmax(-1)
            raw.append(lp.gather(1, tok[:, None])[:, 0])
            seq = torch.cat([seq, tok[:, None]], 1)
    assert torch.equal(ids, seq[:, len(prefix):])
    assert torch.allclose(avg, torch.stack(raw, 1).mean(1), atol=1e-5)


def test_bundle_packing_order_against_transformers(tmp_path):
    """The fused qkv rows are [q | k | v] and gate_up rows [gate | up] in the
    HF projections' order: a swapped pair changes transformers' logits."""
    c = ModelConfig(**SHAPES["g2_d128"])
    w = _weights(c, 3)
    hf = _hf_model(c, save_bundle(c, w, tmp_path / "ok"))
    ids = torch.arange(10)[None] % c.vocab_size
    with torch.no_grad():
        ref = hf(input_ids=ids).logits
    swapped = _weights(c, 3)
    inter = c.intermediate_size
    for lw in swapped["layers"]:
        g, u = lw["gate_up"][:inter].clone(), lw["gate_up"][inter:].clone()
        lw["gate_up"][:inter], lw["gate_up"][inter:] = u, g
    hf_bad = _hf_model(c, save_bundle(c, swapped, tmp_path / "bad"))
    with torch.no_grad():
        bad = hf_bad(input_ids=ids).logits
    assert (bad - ref).abs().max().item() > 1e-2
    assert (OracleModel(c, w).logits(ids) - ref).abs().max().item() <= 1e-5


# --- Block-AttnRes trunk: the zero-query closed form ------------------------
#
# The reference's trunk (python/aios/models/minimind_ime.py:193-326) mixes a
# depth bank before every attention and MLP: bank = [embedding, one summed
# delta per finished block], plus the block's running partial.  With every
# mixer query zero, each softmax over depth is uniform, so a mixer returns
# the mean of its S sources.  Within a block the sources sum to the standard
# residual stream (embedding + every delta so far), so each mixer output is
# that stream divided by S.  Every consumer of a mixer output is an RMSNorm,
# and RMSNorm(x / S) = RMSNorm(x) with eps * S^2 in place of eps; at eps
# 1e-12 the difference is far below float32 rounding.  The zero-query trunk
# therefore equals the standard Qwen3 trunk on the same weights, which
# transformers implements independently.  Non-zero queries are pinned by the
# mixer's own known answers (tests/test_ime_attnres.py:47-66 of the
# reference, restated in tests/test_oracle.py).

ATTNRES_SHAPES = {
    # 8 layers in 4 blocks of 2, the MiniMind head shape (8/2 x 96)
    "l8_b4_g4_d96": dict(num_layers=8, num_qo_heads=8, num_kv_heads=2, head_dim=96,
                         hidden_size=128, vocab_size=157, intermediate_size=160,
                         rms_norm_eps=1e-12, rope_theta=1000000.0,
                         residual_type="block_attnres", attnres_num_blocks=4),
    # 6 layers in 2 blocks of 3, 12/4 x 64 (the deployed 0.214B head shape)
    "l6_b2_g3_d64": dict(num_layers=6, num_qo_heads=12, num_kv_heads=4, head_dim=64,
                         hidden_size=96, vocab_size=131, intermediate_size=128,
                         rms_norm_eps=1e-12, rope_theta=10000.0,
                         residual_type="block_attnres", attnres_num_blocks=2),
}


def _attnres_zero_query_weights(c: ModelConfig, seed: int) -> dict:
    """Synthetic float32 Block-AttnRes weights: non-trivial layer norms and
    mixer key-norm weights, every mixer query zero."""
    w = init_weights(c, seed, "cpu", dtype=torch.float32, std=0.15)
    g = torch.Generator().manual_seed(seed + 1)
    for lw in w["layers"]:
        for key in ("input_norm", "post_norm", "q_norm", "k_norm",
                    "attn_res_norm", "mlp_res_norm"):
            lw[key].copy_(torch.rand(lw[key].shape, generator=g) + 0.5)
        lw["attn_res_query"].zero_()
        lw["mlp_res_query"].zero_()
    for key in ("final_norm", "final_res_norm"):
        w[key].copy_(torch.rand(w[key].shape, generator=g) + 0.5)
    w["final_res_query"].zero_()
    return w


def _standard_view(c: ModelConfig, w: dict):
    """The same decoder weights as a standard-residual Qwen3 model."""
    from dataclasses import replace

    sc = replace(c, residual_type="standard", attnres_num_blocks=0)
    drop = {"attn_res_query", "attn_res_norm", "mlp_res_query", "mlp_res_norm"}
    sw = {k: v for k, v in w.items()
          if k not in ("layers", "final_res_query", "final_res_norm")}
    sw["layers"] = [{k: v for k, v in lw.items() if k not in drop} for lw in w["layers"]]
    return sc, sw


class _StaleMlpMixerOracle(OracleModel):
    """A planted wiring mistake: the MLP mixer reads the sources the attention
    mixer read (without the attention delta just added to the partial)."""

    def _attnres_logits(self, ids, start):
        from oracle.model import _rms

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
            h = self._mix(srcs, lw["mlp_res_query"], lw["mlp_res_norm"])
            partial = delta if partial is None else partial + delta
            partial = partial + self._mlp(lw, _rms(h, lw["post_norm"], c.rms_norm_eps))
            if (i + 1) % per == 0:
                bank.append(partial)
        h = self._mix(bank, self.w["final_res_query"], self.w["final_res_norm"])
        x = _rms(h, self.w["final_norm"], c.rms_norm_eps)
        return x[:, start:] @ self.w.get("lm_head", self.w["embed"]).T


@pytest.mark.parametrize("shape", sorted(ATTNRES_SHAPES))
def test_attnres_trunk_zero_queries_equals_transformers_qwen3(shape, tmp_path):
    c = ModelConfig(**ATTNRES_SHAPES[shape])
    w = _attnres_zero_query_weights(c, 31)
    sc, sw = _standard_view(c, w)
    hf = _hf_model(sc, save_bundle(sc, sw, tmp_path / "bundle"))
    ids = torch.randint(0, c.vocab_size, (2, 17), generator=torch.Generator().manual_seed(7))
    with torch.no_grad():
        ref = hf(input_ids=ids).logits
    got = OracleModel(c, w).logits(ids)
    scale = ref.abs().max().item()
    assert scale > 1.0
    err = (got - ref).abs().max().item()
    # float32 rounding through 6-8 layers: a few ulps of the logit scale
    assert err <= 3e-6 * scale, (shape, err, scale)
    # the oracle's standard trunk agrees too (same weights, standard config)
    assert (OracleModel(sc, sw).logits(ids) - ref).abs().max().item() <= 3e-6 * scale
    # a plausible wiring mistake is caught by this closed form
    bad = _StaleMlpMixerOracle(c, w).logits(ids)
    assert (bad - ref).abs().max().item() > 1e-2


def test_attnres_trunk_nonzero_queries_differ_from_standard(tmp_path):
    """The closed form holds only at zero queries: non-zero queries make the
    depth routing non-uniform and the logits leave the standard trunk's."""
    c = ModelConfig(**ATTNRES_SHAPES["l8_b4_g4_d96"])
    w = _attnres_zero_query_weights(c, 31)
    sc, sw = _standard_view(c, w)
    ids = torch.randint(0, c.vocab_size, (2, 17), generator=torch.Generator().manual_seed(7))
    ref = OracleModel(sc, sw).logits(ids)
    g = torch.Generator().manual_seed(3)
    for lw in w["layers"]:
        lw["mlp_res_query"].copy_(torch.randn(lw["mlp_res_query"].shape, generator=g))
    assert (OracleModel(c, w).logits(ids) - ref).abs().max().item() > 1e-2
