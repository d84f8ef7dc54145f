"""Pins the float32 model oracle (oracle/model.py) against an independent
Qwen3 implementation: transformers' ``Qwen3ForCausalLM`` (CPU only).

The reference's decoder (python/aios/models/qwen3.py:52-173, its packing in
models/weight.py:48-70 and SiLU of the first half in layers/activation.py:
9-12) is standard Qwen3, which transformers implements independently of this
repository.  The same weights reach both models through the exported bundle
(``aios_amd.weights.save_bundle`` writes the HF tensor names, splitting the
packed q/k/v and gate/up projections), so a shared misreading of the MLP
half order, the q/k-norm -> RoPE order, the residual placement or the
packing order fails here.  The Block-AttnRes trunk has no independent
implementation available offline and stays unpinned by this file.
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
