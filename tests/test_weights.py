"""Weight bundles (aios_amd/weights.py) on the CPU: the exporter's tensor
names and layout (scripts/export_minimind_ime.py:241-407), packing on load
(python/aios/models/weight.py:12-70), config fields
(python/aios/models/config.py:91-112), and a model run from a loaded bundle."""
from __future__ import annotations

import json

import pytest
import torch

from aios_amd.config import ModelConfig
from aios_amd.qwen3 import init_weights
from aios_amd.weights import (SCHEMA, config_from_hf, load_bundle, required_tensor_names,
                              save_bundle)


def _tiny(**kw):
    base = dict(num_layers=8, num_qo_heads=2, num_kv_heads=1, head_dim=4, hidden_size=8,
                vocab_size=32, intermediate_size=16, rms_norm_eps=1e-6, rope_theta=100000.0,
                max_position_embeddings=32, model_type="minimind_ime_v3")
    base.update(kw)
    return ModelConfig(**base)


def test_attnres_tensor_names_follow_the_checkpoint_layout():
    """Names the reference's own tests require (tests/test_ime_attnres.py:69-78)
    and the tied head omitted."""
    c = _tiny(residual_type="block_attnres", attnres_num_blocks=2)
    names = set(required_tensor_names(c))
    assert "model.layers.0.attn_res_mixer.query" in names
    assert "model.layers.7.mlp_res_mixer.key_norm.weight" in names
    assert "model.final_attn_res_mixer.query" in names
    assert "lm_head.weight" not in names
    assert "model.layers.3.self_attn.q_proj.weight" in names
    assert "model.layers.3.mlp.gate_proj.weight" in names
    # 2 + 11 per layer + 4 mixer tensors per layer + 2 final mixer tensors
    assert len(names) == 2 + 8 * (11 + 4) + 2
    std = _tiny(tie_word_embeddings=False)
    assert "lm_head.weight" in set(required_tensor_names(std))
    assert len(required_tensor_names(std)) == 2 + 8 * 11 + 1


@pytest.mark.parametrize("kw", [dict(), dict(residual_type="block_attnres", attnres_num_blocks=2),
                                dict(tie_word_embeddings=False)])
def test_bundle_round_trip(tmp_path, kw):
    c = _tiny(**kw)
    w = init_weights(c, 3, "cpu")
    save_bundle(c, w, tmp_path)
    manifest = json.loads((tmp_path / "aios_manifest.json").read_text())
    assert manifest["schema_version"] == SCHEMA
    from safetensors import safe_open

    with safe_open(str(tmp_path / "model.safetensors"), framework="pt") as f:
        assert set(f.keys()) == set(required_tensor_names(c))
        q = f.get_tensor("model.layers.2.self_attn.q_proj.weight")
        v = f.get_tensor("model.layers.2.self_attn.v_proj.weight")
        up = f.get_tensor("model.layers.2.mlp.up_proj.weight")
    # packing order: q, k, v rows; gate rows then up rows
    assert torch.equal(w["layers"][2]["qkv"][: c.num_qo_heads * c.head_dim], q)
    assert torch.equal(w["layers"][2]["qkv"][-c.num_kv_heads * c.head_dim:], v)
    assert torch.equal(w["layers"][2]["gate_up"][c.intermediate_size:], up)
    c2, w2 = load_bundle(tmp_path)
    assert c2 == c
    assert w2.keys() == w.keys()
    for k in w:
        if k == "layers":
            for a, b in zip(w["layers"], w2["layers"]):
                assert a.keys() == b.keys()
                assert all(torch.equal(a[n], b[n]) for n in a)
        else:
            assert torch.equal(w[k], w2[k])


def test_bundle_errors(tmp_path):
    c = _tiny()
    save_bundle(c, init_weights(c, 1, "cpu"), tmp_path)
    data = json.loads((tmp_path / "config.json").read_text())
    data["num_hidden_layers"] = 9  # the bundle holds 8
    (tmp_path / "config.json").write_text(json.dumps(data))
    with pytest.raises(KeyError, match="missing required tensor: model.layers.8"):
        load_bundle(tmp_path)
    data["num_hidden_layers"] = 8
    (tmp_path / "config.json").write_text(json.dumps(data))
    with open(tmp_path / "model.safetensors", "r+b") as f:  # corrupt one byte of data
        f.seek(-2, 2)
        b = f.read(1)
        f.seek(-2, 2)
        f.write(bytes([b[0] ^ 1]))
    with pytest.raises(ValueError, match="SHA-256"):
        load_bundle(tmp_path)


def test_config_from_hf_defaults():
    """config.py:91-112 field mapping and defaults."""
    c = config_from_hf({"num_hidden_layers": 14, "num_attention_heads": 12,
                        "num_key_value_heads": 4, "hidden_size": 768, "vocab_size": 16384,
                        "intermediate_size": 2048})
    assert (c.num_layers, c.num_qo_heads, c.num_kv_heads, c.head_dim) == (14, 12, 4, 64)
    assert c.rms_norm_eps == 1e-6 and c.rope_theta == 1000000.0
    assert c.max_position_embeddings == 32768 and c.tie_word_embeddings is False
    assert c.residual_type == "standard"
    with pytest.raises(ValueError, match="divisible"):
        config_from_hf({"num_hidden_layers": 7, "num_attention_heads": 2, "hidden_size": 8,
                        "vocab_size": 32, "intermediate_size": 16,
                        "residual_type": "block_attnres", "attnres_num_blocks": 2})


def test_untied_head_is_used(tmp_path):
    """An untied bundle's lm_head drives the logits (oracle model)."""
    from oracle.model import OracleModel

    c = _tiny(num_layers=2, tie_word_embeddings=False)
    w = init_weights(c, 4, "cpu", dtype=torch.float32)
    save_bundle(c, w, tmp_path)
    c2, w2 = load_bundle(tmp_path, dtype=torch.float32)
    ids = torch.tensor([[1, 5, 7]])
    got = OracleModel(c2, w2).logits(ids)
    tied = dict(w2)
    del tied["lm_head"]
    assert not torch.allclose(got, OracleModel(c2, tied).logits(ids))
    assert torch.equal(got, OracleModel(c, w).logits(ids))
