"""Safetensors checkpoint directories for the loader tests: a minimal writer of
the published format (8-byte little-endian header length, JSON header,
tensor bytes) and a Hugging Face model directory (config.json + shards) for a
test model's weights under the Llama/Qwen2 tensor names."""
import json
import os

import numpy as np

from model_fixtures import bf16_round

DTYPE_NAME = {np.dtype(np.float32): "F32", np.dtype(np.float16): "F16"}


def bf16_bits(x):
    """f32 values (already bf16-representable or not) -> RNE bf16 bit patterns."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def write_safetensors(path, tensors, metadata=None, order=None):
    """tensors: name -> (dtype name, shape, raw bytes)."""
    header = {}
    if metadata is not None:
        header["__metadata__"] = metadata
    off = 0
    blobs = []
    for name in (order or sorted(tensors)):
        dt, shape, raw = tensors[name]
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def tensor_entry(x, dtype):
    """(dtype name, shape, bytes) of array x stored as "F32", "F16" or "BF16"."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == "BF16":
        return "BF16", x.shape, bf16_bits(x).tobytes()
    if dtype == "F16":
        return "F16", x.shape, x.astype(np.float16).tobytes()
    return "F32", x.shape, x.tobytes()


def hf_tensors(spec, W):
    """Llama/Qwen2 tensor names (transformer.rs:6-19) -> f32 arrays."""
    t = {"model.embed_tokens.weight": W["embed"], "model.norm.weight": W["final_norm"]}
    if W["lm_head"] is not None:
        t["lm_head.weight"] = W["lm_head"]
    names = [("input_norm", "input_layernorm.weight"), ("q", "self_attn.q_proj.weight"),
             ("k", "self_attn.k_proj.weight"), ("v", "self_attn.v_proj.weight"),
             ("o", "self_attn.o_proj.weight"), ("post_norm", "post_attention_layernorm.weight"),
             ("gate", "mlp.gate_proj.weight"), ("up", "mlp.up_proj.weight"),
             ("down", "mlp.down_proj.weight"), ("q_bias", "self_attn.q_proj.bias"),
             ("k_bias", "self_attn.k_proj.bias"), ("v_bias", "self_attn.v_proj.bias")]
    for l, w in enumerate(W["layers"]):
        for key, hf in names:
            if w[key] is not None:
                t[f"model.layers.{l}.{hf}"] = w[key]
    return t


def write_model_dir(directory, spec, W, dtype="BF16", shards=2, config_extra=None):
    """config.json + `shards` safetensors files holding every tensor."""
    os.makedirs(directory, exist_ok=True)
    cfg = {
        "architectures": ["Qwen2ForCausalLM" if spec.bias else "LlamaForCausalLM"],
        "hidden_size": spec.H, "num_hidden_layers": spec.L,
        "num_attention_heads": spec.hq, "num_key_value_heads": spec.hkv,
        "vocab_size": spec.V, "intermediate_size": spec.F,
        "max_position_embeddings": spec.max_pos, "rope_theta": spec.theta,
        "rms_norm_eps": spec.eps, "tie_word_embeddings": bool(spec.tied),
        "torch_dtype": {"BF16": "bfloat16", "F16": "float16", "F32": "float32"}[dtype],
    }
    if spec.H // spec.hq != spec.d:
        cfg["head_dim"] = spec.d
    cfg.update(config_extra or {})
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(cfg, f)
    t = hf_tensors(spec, W)
    names = sorted(t)
    for s in range(shards):
        part = {n: tensor_entry(t[n], dtype) for n in names[s::shards]}
        write_safetensors(os.path.join(directory, f"model-{s + 1:05d}-of-{shards:05d}.safetensors"),
                          part, metadata={"format": "pt"})
    return cfg
