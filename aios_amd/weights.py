"""MiniMind-IME / Qwen3 weight bundles: load the exported inference bundle
into the decoder's weight dict, and write one.

Bundle layout (scripts/export_minimind_ime.py:358-407): a directory with
``model.safetensors`` (HF tensor names, the exact inference set of
``required_tensor_names``, :276-305), ``config.json`` (HF config fields,
:241-274) and ``aios_manifest.json`` (schema ``aios.minimind_ime_bundle.v3``
with the model file's SHA-256).  Loading follows
python/aios/models/weight.py:12-70: tensors are read with safetensors (no
pickle), q/k/v are packed into the fused qkv projection and gate/up into
the merged gate/up projection along the output dimension, everything else
keeps its tensor.  The config follows ModelConfig.from_json
(python/aios/models/config.py:91-112).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch

from aios_amd.config import ModelConfig

SCHEMA = "aios.minimind_ime_bundle.v3"


def config_from_hf(data: dict) -> ModelConfig:
    """ModelConfig from config.json fields (config.py:91-112)."""
    heads = data["num_attention_heads"]
    return ModelConfig(
        num_layers=data["num_hidden_layers"],
        num_qo_heads=heads,
        num_kv_heads=data.get("num_key_value_heads", heads),
        head_dim=data.get("head_dim", data["hidden_size"] // heads),
        hidden_size=data["hidden_size"],
        vocab_size=data["vocab_size"],
        intermediate_size=data["intermediate_size"],
        hidden_act=data.get("hidden_act", "silu"),
        rms_norm_eps=data.get("rms_norm_eps", 1e-6),
        rope_theta=data.get("rope_theta", 1000000.0),
        max_position_embeddings=data.get("max_position_embeddings", 32768),
        tie_word_embeddings=data.get("tie_word_embeddings", False),
        model_type=data.get("model_type", "unknown"),
        residual_type=data.get("residual_type", "standard"),
        attnres_num_blocks=data.get("attnres_num_blocks", 0),
        attnres_alpha=data.get("attnres_alpha", 1.0),
        pad_token_id=data.get("pad_token_id"),
    )


def config_to_hf(c: ModelConfig) -> dict:
    data = {
        "architectures": ["MiniMindIMEForCausalLM"], "model_type": c.model_type,
        "vocab_size": c.vocab_size, "hidden_size": c.hidden_size,
        "num_hidden_layers": c.num_layers, "intermediate_size": c.intermediate_size,
        "num_attention_heads": c.num_qo_heads, "num_key_value_heads": c.num_kv_heads,
        "head_dim": c.head_dim, "hidden_act": c.hidden_act, "rms_norm_eps": c.rms_norm_eps,
        "rope_theta": c.rope_theta, "max_position_embeddings": c.max_position_embeddings,
        "tie_word_embeddings": c.tie_word_embeddings, "torch_dtype": "bfloat16",
        "residual_type": c.residual_type, "attnres_num_blocks": c.attnres_num_blocks,
        "attnres_alpha": c.attnres_alpha,
    }
    if c.pad_token_id is not None:
        data["pad_token_id"] = c.pad_token_id
    if c.residual_type == "block_attnres":
        data["layers_per_attnres_block"] = c.layers_per_attnres_block
    return data


def _layer_names(i: int, c: ModelConfig) -> dict:
    """HF tensor name of every per-layer entry of the weight dict
    (export_minimind_ime.py:276-305); qkv and gate_up are packed."""
    b = f"model.layers.{i}"
    names = {
        "input_norm": f"{b}.input_layernorm.weight",
        "post_norm": f"{b}.post_attention_layernorm.weight",
        "qkv": (f"{b}.self_attn.q_proj.weight", f"{b}.self_attn.k_proj.weight",
                f"{b}.self_attn.v_proj.weight"),
        "o": f"{b}.self_attn.o_proj.weight",
        "q_norm": f"{b}.self_attn.q_norm.weight",
        "k_norm": f"{b}.self_attn.k_norm.weight",
        "gate_up": (f"{b}.mlp.gate_proj.weight", f"{b}.mlp.up_proj.weight"),
        "down": f"{b}.mlp.down_proj.weight",
    }
    if c.residual_type == "block_attnres":
        names.update({
            "attn_res_query": f"{b}.attn_res_mixer.query",
            "attn_res_norm": f"{b}.attn_res_mixer.key_norm.weight",
            "mlp_res_query": f"{b}.mlp_res_mixer.query",
            "mlp_res_norm": f"{b}.mlp_res_mixer.key_norm.weight",
        })
    return names


def _top_names(c: ModelConfig) -> dict:
    names = {"embed": "model.embed_tokens.weight", "final_norm": "model.norm.weight"}
    if c.residual_type == "block_attnres":
        names["final_res_query"] = "model.final_attn_res_mixer.query"
        names["final_res_norm"] = "model.final_attn_res_mixer.key_norm.weight"
    if not c.tie_word_embeddings:
        names["lm_head"] = "lm_head.weight"
    return names


def required_tensor_names(c: ModelConfig) -> list[str]:
    """The bundle's tensor set, in the exporter's order."""
    out = ["model.embed_tokens.weight", "model.norm.weight"]
    for i in range(c.num_layers):
        for v in _layer_names(i, c).values():
            out.extend(v if isinstance(v, tuple) else (v,))
    top = _top_names(c)
    out.extend(top[k] for k in ("final_res_query", "final_res_norm", "lm_head") if k in top)
    return out


def _sha256(path: Path) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            h.update(block)
    return h.hexdigest()


def load_bundle(path, device="cpu", dtype: torch.dtype = torch.bfloat16,
                verify: bool = True) -> tuple[ModelConfig, dict]:
    """(config, weight dict) of an exported bundle directory."""
    from safetensors import safe_open

    path = Path(path)
    config = config_from_hf(json.loads((path / "config.json").read_text(encoding="utf-8")))
    model_file = path / "model.safetensors"
    if not model_file.is_file():
        raise FileNotFoundError(f"No .safetensors files found in {path}")
    manifest_file = path / "aios_manifest.json"
    if verify and manifest_file.is_file():
        manifest = json.loads(manifest_file.read_text(encoding="utf-8"))
        if manifest.get("schema_version") != SCHEMA:
            raise ValueError(f"unsupported bundle schema {manifest.get('schema_version')!r}")
        if manifest.get("model_sha256") not in (None, _sha256(model_file)):
            raise ValueError("model.safetensors does not match the manifest's SHA-256")
    dev = torch.device(device)
    with safe_open(str(model_file), framework="pt", device="cpu") as f:
        keys = set(f.keys())

        def read(name):
            if name not in keys:
                raise KeyError(f"Checkpoint is missing required tensor: {name}")
            return f.get_tensor(name)

        def get(spec):
            t = torch.cat([read(n) for n in spec], 0) if isinstance(spec, tuple) else read(spec)
            return t.to(device=dev, dtype=dtype).contiguous()

        w = {k: get(v) for k, v in _top_names(config).items()}
        w["layers"] = [{k: get(v) for k, v in _layer_names(i, config).items()}
                       for i in range(config.num_layers)]
    return config, w


def save_bundle(config: ModelConfig, weights: dict, path) -> Path:
    """Write a bundle in the exporter's layout (q/k/v and gate/up split back
    into their HF tensors)."""
    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    c = config
    tensors = {}

    def put(spec, t):
        t = t.detach().to("cpu").contiguous()
        if isinstance(spec, tuple):
            if len(spec) == 3:
                sizes = [c.num_qo_heads * c.head_dim, c.num_kv_heads * c.head_dim,
                         c.num_kv_heads * c.head_dim]
            else:
                sizes = [c.intermediate_size, c.intermediate_size]
            for n, part in zip(spec, torch.split(t, sizes, 0)):
                tensors[n] = part.contiguous()
        else:
            tensors[spec] = t

    for k, v in _top_names(c).items():
        put(v, weights[k])
    for i, lw in enumerate(weights["layers"]):
        for k, v in _layer_names(i, c).items():
            put(v, lw[k])
    model_file = path / "model.safetensors"
    save_file(tensors, str(model_file))
    (path / "config.json").write_text(json.dumps(config_to_hf(c), indent=2) + "\n",
                                      encoding="utf-8")
    manifest = {
        "schema_version": SCHEMA, "model_sha256": _sha256(model_file),
        "dtype": str(next(iter(tensors.values())).dtype).replace("torch.", ""),
        "inference_parameter_tensors": len(tensors),
        "inference_parameter_count": sum(t.numel() for t in tensors.values()),
        "tied_lm_head_omitted": bool(c.tie_word_embeddings),
        "residual_type": c.residual_type, "attnres_num_blocks": c.attnres_num_blocks,
        "config": config_to_hf(c),
    }
    (path / "aios_manifest.json").write_text(json.dumps(manifest, indent=2) + "\n",
                                             encoding="utf-8")
    return path
