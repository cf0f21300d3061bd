"""Writes safetensors files and tiny Qwen2-shaped HF checkpoints for the checkpoint-import
tests (format: 8-byte little-endian header length, JSON header {name: {dtype, shape,
data_offsets}}, then the packed little-endian payloads)."""
from __future__ import annotations

import json
import os
import struct

import numpy as np


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (finite inputs)."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def encode(values: np.ndarray, dtype: str) -> bytes:
    v = np.asarray(values, np.float32)
    if dtype == "F32":
        return v.astype("<f4").tobytes()
    if dtype == "F16":
        return v.astype("<f2").tobytes()
    return f32_to_bf16_bits(v).astype("<u2").tobytes()


def write_safetensors(path, tensors, metadata=None, header_override=None):
    """tensors: list of (name, dtype, shape, raw bytes).  header_override (dict) replaces the
    generated header, for malformed-file tests."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    text = json.dumps(header_override if header_override is not None else header).encode()
    text += b" " * (-len(text) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for b in blobs:
            f.write(b)


def qwen2_config(cfg: dict, **extra) -> dict:
    c = {
        "architectures": ["Qwen2ForCausalLM"], "model_type": "qwen2", "hidden_act": "silu",
        "hidden_size": cfg["hidden"], "intermediate_size": cfg["intermediate"],
        "max_position_embeddings": cfg["max_pos"], "num_attention_heads": cfg["heads"],
        "num_hidden_layers": cfg["layers"], "num_key_value_heads": cfg["kv_heads"],
        "rms_norm_eps": cfg["eps"], "rope_theta": cfg["theta"],
        "tie_word_embeddings": cfg["tie"], "vocab_size": cfg["vocab"],
    }
    c.update(extra)
    return c


def write_qwen2_checkpoint(model_dir, cfg: dict, dtype: str = "BF16", seed: int = 0, shards: int = 1,
                           biases: bool = True, std: float = 0.05, config_extra=None):
    """A random Qwen2 checkpoint in HF naming ([out, in] projections).  Returns {external
    name: (dtype, shape, raw bytes)} of everything written."""
    os.makedirs(model_dir, exist_ok=True)
    rng = np.random.default_rng(seed)
    h, f, v = cfg["hidden"], cfg["intermediate"], cfg["vocab"]
    kvw = cfg["kv_heads"] * (h // cfg["heads"])

    def t(name, *shape, ones=False):
        vals = (1.0 + 0.1 * rng.standard_normal(shape)) if ones else rng.standard_normal(shape) * std
        return (name, dtype, list(shape), encode(vals.astype(np.float32), dtype))

    tensors = [t("model.embed_tokens.weight", v, h)]
    for layer in range(cfg["layers"]):
        p = f"model.layers.{layer}."
        tensors += [t(p + "input_layernorm.weight", h, ones=True),
                    t(p + "self_attn.q_proj.weight", h, h), t(p + "self_attn.k_proj.weight", kvw, h),
                    t(p + "self_attn.v_proj.weight", kvw, h), t(p + "self_attn.o_proj.weight", h, h),
                    t(p + "post_attention_layernorm.weight", h, ones=True),
                    t(p + "mlp.gate_proj.weight", f, h), t(p + "mlp.up_proj.weight", f, h),
                    t(p + "mlp.down_proj.weight", h, f)]
        if biases:
            tensors += [t(p + "self_attn.q_proj.bias", h), t(p + "self_attn.k_proj.bias", kvw),
                        t(p + "self_attn.v_proj.bias", kvw)]
    tensors.append(t("model.norm.weight", h, ones=True))
    if not cfg["tie"]:
        tensors.append(t("lm_head.weight", v, h))
    with open(os.path.join(model_dir, "config.json"), "w") as fh:
        json.dump(qwen2_config(cfg, **(config_extra or {})), fh)
    if shards == 1:
        write_safetensors(os.path.join(model_dir, "model.safetensors"), tensors, metadata={"format": "pt"})
    else:
        weight_map = {}
        for s in range(shards):
            part = tensors[s::shards]
            fname = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(os.path.join(model_dir, fname), part, metadata={"format": "pt"})
            weight_map.update({name: fname for name, *_ in part})
        with open(os.path.join(model_dir, "model.safetensors.index.json"), "w") as fh:
            json.dump({"metadata": {"total_size": sum(len(r) for *_, r in tensors)}, "weight_map": weight_map}, fh)
    return {name: (dt, shape, raw) for name, dt, shape, raw in tensors}
